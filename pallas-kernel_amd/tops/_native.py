"""ctypes binding of libtops_hip.so (the C ABI declared in include/tops_hip.h).

The HIP library is the only compute path: if it is missing, every op raises
instead of falling back to anything else.
"""
from __future__ import annotations

import ctypes
import os

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "libtops_hip.so")

TOPS_F32 = 0
TOPS_BF16 = 1
TOPS_F16 = 2

_vp = ctypes.c_void_p
_i32 = ctypes.c_int
_f32 = ctypes.c_float
_i64 = ctypes.c_int64

# name -> argtypes (every entry point returns int)
SIGNATURES = {
    "tops_gla_chunk_fwd": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                           _i32, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _vp],
    "tops_gla_chunk_bwd": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                           _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32,
                           _i32, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _vp],
    "tops_gla_chunk_bwd_dh": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                              _i32, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _vp],
    "tops_gla_chunk_bwd_dqkg": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                _vp, _vp, _vp, _i32,
                                _i32, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _vp],
    "tops_gla_chunk_fwd_gamma": [_vp] * 10 + [_i32] * 7 + [_f32, _vp],
    "tops_gla_chunk_bwd_dh_gamma": [_vp] * 10 + [_i32] * 7 + [_f32, _vp],
    "tops_gla_chunk_bwd_dqkg_gamma": [_vp] * 13 + [_i32] * 8 + [_f32, _vp],
    "tops_simple_gla_chunk_fwd": [_vp] * 11 + [_i32] * 7 + [_f32, _vp],
    "tops_simple_gla_chunk_bwd": [_vp] * 17 + [_i32] * 8 + [_f32, _vp],
    "tops_gla_fused_recurrent_fwd": [_vp] * 10 + [_i32] * 7 + [_f32, _i32, _vp],
    "tops_gla_fused_recurrent_fwd_decode": [_vp] * 10 + [_i32] * 7 + [_f32, _i32, _vp],
    "tops_gla_fused_recurrent_fwd_decode_norm_gate": [_vp] * 8 + [_f32, _vp, _vp, _vp]
                                                     + [_i32] * 7 + [_f32, _i32, _vp],
    "tops_gla_decode_conv_norm_gate": [_vp] * 15 + [_i32, _i32] + [_vp] * 4 + [_f32, _vp, _i32,
                                                                               _vp, _vp]
                                      + [_i32] * 7 + [_f32, _vp],
    "tops_kda_fused_recurrent_fwd_decode": [_vp] * 9 + [_i32] * 7 + [_f32, _vp],
    "tops_gla_fused_recurrent_bwd": [_vp] * 17 + [_i32] * 7 + [_f32, _i32, _vp],
    "tops_prepare_chunk_indices": [_vp, _i32, _i32, _vp, _vp, _i32],
    "tops_kda_chunk_fwd": [_vp] * 16 + [_i32] * 8 + [_f32, _vp],
    "tops_kda_chunk_bwd": [_vp] * 24 + [_i32] * 8 + [_f32, _vp],
    "tops_kda_chunk_fwd_c16": [_vp] * 17 + [_i32] * 8 + [_f32, _vp],
    "tops_simple_gla_chunk_fwd_c16": [_vp] * 12 + [_i32] * 7 + [_f32, _vp],
    "tops_simple_gla_chunk_bwd_dh_c16": [_vp] * 12 + [_i32] * 7 + [_f32, _vp],
    "tops_simple_gla_chunk_bwd_dqkg_c16": [_vp] * 16 + [_i32] * 8 + [_f32, _vp],
    "tops_kda_chunk_bwd_c16": [_vp] * 24 + [_i32] * 8 + [_f32, _vp],
    "tops_kda_chunk_fwd_noalloc": [_vp] * 11 + [_i32] * 8 + [_f32, _vp],
    "tops_simple_gla_chunk_bwd_dh": [_vp] * 11 + [_i32] * 7 + [_f32, _vp],
    "tops_simple_gla_chunk_bwd_dqkg": [_vp] * 14 + [_i32] * 8 + [_f32, _vp],
    "tops_chunk_fwd_paired": [_vp] * 4 + [_i32] + [_vp] * 6 + [_i32] * 7 + [_f32, _vp],
    "tops_chunk_bwd_dh_paired": [_vp] * 3 + [_i32] + [_vp] * 7 + [_i32] * 7 + [_f32, _vp],
    "tops_chunk_bwd_dqkg_paired": [_vp] * 4 + [_i32] + [_vp] * 10 + [_i32] * 8 + [_f32, _vp],
    "tops_chunk_reverse_fwd": [_vp] * 4 + [_i32] + [_vp] * 4 + [_i32] * 7 + [_f32, _vp],
    "tops_gla_chunk_fwd_c16": [_vp] * 9 + [_vp] * 2 + [_i32] * 7 + [_f32, _vp],
    "tops_gla_chunk_bwd_dh_c16": [_vp] * 9 + [_vp] * 2 + [_i32] * 7 + [_f32, _vp],
    "tops_gla_chunk_bwd_dqkg_c16": [_vp] * 12 + [_vp] * 3 + [_i32] * 8 + [_f32, _vp],
    "tops_chunk_fwd_slice": [_vp] * 4 + [_i32] + [_vp] * 3 + [_i32] + [_vp] * 4 + [_i32] * 8
                            + [_f32, _vp],
    "tops_chunk_bwd_dh_slice": [_vp] * 3 + [_i32] + [_vp] * 5 + [_i32] + [_vp] * 3 + [_i32] * 8
                               + [_f32, _vp],
    "tops_chunk_bwd_dqkg_slice": [_vp] * 4 + [_i32] + [_vp] * 8 + [_i32] * 2 + [_vp] * 3
                                 + [_i32] * 10 + [_f32, _vp],
    "tops_gla_chunk_fwd_gv": [_vp] * 8 + [_i32] * 7 + [_f32, _vp],
    "tops_gla_chunk_fwd_gv32": [_vp] * 9 + [_i32] * 7 + [_f32, _vp],
    "tops_gv_gate_grad": [_vp] * 8 + [_i32] * 6 + [_vp],
    "tops_gla_chunk_bwd_dv_gv32": [_vp] * 8 + [_i32] * 7 + [_f32, _vp],
    "tops_gla_chunk_rev_dv": [_vp] * 8 + [_i32] * 7 + [_f32, _vp],
    "tops_kda_stage_intra_fwd": [_vp] * 6 + [_i32] + [_vp] * 6 + [_i32] * 6 + [_f32, _vp],
    "tops_delta_rule_fwd_h": [_vp] * 5 + [_i32] + [_vp] * 6 + [_i32] * 7 + [_vp],
    "tops_chunk_state_pass": [_vp, _vp, _vp, _i32, _vp, _vp, _vp, _vp] + [_i32] * 6 + [_f32, _i32, _vp],
    "tops_chunk_state_combine": [_vp] * 7 + [_i32] * 5 + [_vp],
    "tops_kda_gate_fwd": [_vp, _i32, _vp, _vp, _vp] + [_i32] * 6 + [_f32, _vp],
    "tops_kda_gate_chunk_cumsum": [_vp, _i32] + [_vp] * 6 + [_i32] * 9 + [_f32, _f32, _vp],
    "tops_kda_gate_bwd": [_vp, _i32] + [_vp] * 7 + [_i64] + [_i32] * 6 + [_f32, _vp],
    "tops_l2norm_fwd": [_vp, _i32, _vp, _i32, _i32, _vp],
    "tops_l2norm_bwd": [_vp, _i32, _vp, _vp, _i32, _i32, _vp],
    "tops_rmsnorm_gated_fwd": [_vp, _i32, _vp, _i32, _vp, _vp, _i32, _i32, _f32, _vp],
    "tops_rmsnorm_gated_bwd": [_vp, _i32, _vp, _i32] + [_vp] * 6 + [_i64, _i32, _i32, _f32, _vp],
    "tops_short_conv_fwd": [_vp, _i32, _vp, _vp, _vp, _i32, _vp, _vp] + [_i32] * 6 + [_vp],
    "tops_short_conv_bwd": [_vp, _i32, _vp, _vp, _vp, _i32] + [_vp] * 4 + [_i64, _vp]
                           + [_i32] * 6 + [_vp],
    "tops_short_conv_step": [_vp, _i32, _vp, _vp, _vp, _vp, _vp] + [_i32] * 5 + [_vp],
    "tops_chunk_local_cumsum": [_vp, _i32, _vp, _i32, _vp, _vp, _vp] + [_i32] * 8 + [_f32, _vp],
    "tops_chunk_state_recurrence": [_vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp]
                                   + [_i32] * 9 + [_f32, _vp],
    "tops_gla_stage_attn": [_vp, _vp, _i32, _vp, _vp] + [_i32] * 5 + [_f32, _vp],
    "tops_gla_stage_o": [_vp, _vp, _i32, _vp, _vp, _vp, _vp] + [_i32] * 6 + [_f32, _i32, _vp],
    "tops_gla_stage_dattn": [_vp, _vp, _i32, _vp, _i32] + [_i32] * 5 + [_f32, _vp],
    "tops_gla_stage_dv": [_vp, _vp, _i32, _vp, _vp, _vp, _vp] + [_i32] * 6 + [_vp],
    "tops_gla_stage_dqk_intra": [_vp, _vp, _i32, _vp, _vp, _vp, _vp] + [_i32] * 5 + [_vp],
    "tops_gla_stage_dqkg": [_vp, _vp, _vp, _vp, _i32] + [_vp] * 8 + [_i32] * 6 + [_f32, _vp],
    "tops_kda_stage_intra_bwd": [_vp, _vp, _i32] + [_vp] * 8 + [_i32] * 5 + [_vp],
}

_lib = None


class TopsError(RuntimeError):
    pass


def lib() -> ctypes.CDLL:
    """Load the native library once; raise loudly when it is absent."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise TopsError(
                f"tops-hip native library not found at {LIB_PATH}; build it with "
                "`python pallas-kernel_amd/build.py` (hipcc, gfx950)")
        L = ctypes.CDLL(LIB_PATH)
        L.tops_last_error.restype = ctypes.c_char_p
        L.tops_version.restype = ctypes.c_char_p
        L.tops_gla_state_bytes.restype = ctypes.c_int64
        L.tops_gla_state_bytes.argtypes = [_i32, _i32, _i32, _i32]
        L.tops_kda_chunk_fwd_noalloc_max_bytes.restype = ctypes.c_int64
        L.tops_kda_chunk_fwd_noalloc_max_bytes.argtypes = []
        L.tops_gla_fused_recurrent_bwd_workspace.restype = ctypes.c_int64
        L.tops_gla_fused_recurrent_bwd_workspace.argtypes = [_i32] * 7
        L.tops_kda_gate_bwd_workspace.restype = ctypes.c_int64
        L.tops_kda_gate_bwd_workspace.argtypes = [_i32] * 3
        L.tops_rmsnorm_gated_bwd_workspace.restype = ctypes.c_int64
        L.tops_rmsnorm_gated_bwd_workspace.argtypes = [_i32] * 2
        L.tops_short_conv_bwd_workspace.restype = ctypes.c_int64
        L.tops_short_conv_bwd_workspace.argtypes = [_i32] * 4
        _lib = L
    return _lib


_bound = {}


def _fn(name: str):
    fn = _bound.get(name)
    if fn is None:
        fn = getattr(lib(), name)
        fn.argtypes = SIGNATURES[name]
        fn.restype = ctypes.c_int
        _bound[name] = fn
    return fn


# Optional per-entry-point timing: when enabled, every call() is bracketed by a pair
# of HIP events recorded on the stream the kernels are enqueued on.
_timing = None


def enable_timing(on: bool = True) -> None:
    global _timing
    _timing = {} if on else None


def timing_events() -> dict:
    """{entry point: [(start_event, end_event), ...]} recorded since enable_timing()."""
    return {} if _timing is None else _timing


def call(name: str, *args) -> None:
    if _timing is not None:
        ev0 = torch.cuda.Event(enable_timing=True)
        ev1 = torch.cuda.Event(enable_timing=True)
        ev0.record()
        rc = _fn(name)(*args)
        ev1.record()
        _timing.setdefault(name, []).append((ev0, ev1))
    else:
        rc = _fn(name)(*args)
    if rc != 0:
        msg = lib().tops_last_error().decode()
        if rc == -2:
            raise ValueError(f"{name}: {msg}")
        raise TopsError(f"{name} failed ({rc}): {msg}")


class _Ptr(int):
    """A device address that keeps its tensor alive.  `call(name, ptr(f(x)), ...)` evaluates
    every argument before the launch; a bare address of a temporary such as `f(x)` would let
    the tensor go back to the caching allocator at once, and a later argument's own
    allocation (a copy, an upload) could then take that block and write it before the kernel
    that reads it is queued.  Holding the tensor until `call` returns closes that window;
    freeing it afterwards is stream-ordered behind the launch."""

    def __new__(cls, t):
        p = super().__new__(cls, t.data_ptr())
        p.tensor = t
        return p


def ptr(t) -> int | None:
    return None if t is None else _Ptr(t)


def stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.bfloat16:
        return TOPS_BF16
    if dt == torch.float32:
        return TOPS_F32
    raise TypeError(f"tops-hip kernels take float32 or bfloat16 tensors, got {dt}")


def chunk_dtype_code(dt: torch.dtype) -> int:
    """dtype code of the GLA / simple GLA chunk entry points, which also take fp16."""
    return TOPS_F16 if dt == torch.float16 else dtype_code(dt)


def require_cuda(*ts) -> None:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise TopsError("tops-hip ops take device (HIP) tensors; got a CPU tensor")
