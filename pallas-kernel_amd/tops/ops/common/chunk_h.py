"""Inter-chunk state recurrence on MI355X (mirrors tops/ops/common/chunk_h.py).

Forward: the state before every chunk, h [B, NT, H, K, V], and the final state
(chunk_h.py:100-272 kernel, :363-489 reference).  Backward: the gradient of the state
after every chunk, dh [B, NT, H, K, V], and dh0 (chunk_h.py:575-682 reference, :785-884
kernel).  The gates are the chunk-local cumsums of g [B,T,H] (scalar), g_gamma [H]
(constant per head) and gk [B,T,H,K] (per channel), any combination.

Both directions run tops_chunk_state_recurrence: one workgroup per (sequence, head,
64-column V tile) walks the chunks holding its [K, 64] slice of the state in MFMA
accumulators (fp32), staging each chunk's gated keys / queries and values through LDS.
"""
from __future__ import annotations

import torch

from ... import _native as N
from ...utils import to_device
from ._stage import act, chunk_size_ok, cu_host, f32, require


def _recurrence(x, y, g, g_gamma, gk, s0, cu, C, reverse, scale, every, states_dtype,
                want_final):
    B, T, H, K = x.shape
    V = y.shape[-1]
    chunk_size_ok(C)
    require(T % C == 0, "T must be a multiple of chunk_size")
    require(tuple(y.shape[:3]) == (B, T, H), f"shape mismatch {tuple(x.shape)} / {tuple(y.shape)}")
    require(g is None or tuple(g.shape) == (B, T, H), "g must be [B, T, H]")
    require(g_gamma is None or tuple(g_gamma.shape) == (H,), "g_gamma must be [H]")
    require(gk is None or tuple(gk.shape) == (B, T, H, K), "gk must be [B, T, H, K]")
    cuh = cu_host(cu)
    if cuh is not None:
        require(B == 1, "cu_seqlens requires B=1")
        require(cuh[0] == 0 and cuh[-1] == T and all(a <= b for a, b in zip(cuh, cuh[1:])),
                "cu_seqlens must rise from 0 to T")
        require(all(c % C == 0 for c in cuh), "cu_seqlens must be multiples of chunk_size")
    Nseq = B if cuh is None else len(cuh) - 1
    require(s0 is None or tuple(s0.shape) == (Nseq, H, K, V),
            f"initial state must be {(Nseq, H, K, V)}")
    (xk, yk), code = act(x, y)
    NT = T // C
    sdt = states_dtype if states_dtype in (torch.float32, torch.bfloat16) else torch.float32
    states = torch.empty((B, NT // every, H, K, V), device=x.device, dtype=sdt)
    final = torch.empty((Nseq, H, K, V), device=x.device, dtype=torch.float32) if want_final else None
    cu_dev = None
    if cuh is not None:
        cu_dev = to_device(cuh, x.device, torch.int32)
    with torch.no_grad():
        N.call("tops_chunk_state_recurrence", N.ptr(xk), N.ptr(yk), code, N.ptr(f32(gk)),
               N.ptr(f32(g)), N.ptr(f32(g_gamma)), N.ptr(f32(s0)), N.ptr(states),
               N.dtype_code(sdt), N.ptr(final), N.ptr(cu_dev), B, T, H, K, V, Nseq, C,
               int(every), int(reverse), float(scale), N.stream())
    if sdt != states_dtype:
        states = states.to(states_dtype)
    return states, final


def chunk_fwd_h_ref(k, v, g=None, g_gamma=None, gk=None, gv=None, h0=None,
                    output_final_state: bool = False, states_in_fp32: bool = False,
                    cu_seqlens_cpu=None, cu_seqlens_dev=None, chunk_size: int = 64):
    """h [B, NT, H, K, V] (k.dtype, float32 with ``states_in_fp32``), the state before each
    chunk; ht [N, H, K, V] float32 when ``output_final_state`` else None
    (tops/ops/common/chunk_h.py:363-489).  ``gv`` is not used, as in the reference."""
    del gv
    cu = cu_seqlens_cpu if cu_seqlens_cpu is not None else cu_seqlens_dev
    h, ht = _recurrence(k, v, g, g_gamma, gk, h0, cu, int(chunk_size), False, 1.0, 1,
                        torch.float32 if states_in_fp32 else k.dtype, output_final_state)
    return h, ht


def chunk_fwd_h_kernel(k, v, *, g=None, g_gamma=None, gk=None, gv=None, h0=None,
                       output_final_state: bool = False, cu_seqlens_cpu=None,
                       cu_seqlens_dev=None, chunk_size: int = 64, split_size: int | None = None,
                       states_in_fp32: bool = False):
    """Kernel form (tops/ops/common/chunk_h.py:100-272): as chunk_fwd_h_ref, with the states
    emitted every ``split_size`` tokens (h [B, T / split_size, H, K, V])."""
    require(gv is None, "gv is currently not supported")
    C = int(chunk_size)
    BS = C if split_size is None else int(split_size)
    require(BS % C == 0, f"The `split_size` (got {BS}) must be a multiple of `chunk_size` {C}")
    require(k.shape[1] % BS == 0, f"T must be a multiple of split_size {BS}")
    cu = cu_seqlens_cpu if cu_seqlens_cpu is not None else cu_seqlens_dev
    if cu is not None:
        require(BS == C, "split_size with cu_seqlens is not supported")
    return _recurrence(k, v, g, g_gamma, gk, h0, cu, C, False, 1.0, BS // C,
                       torch.float32 if states_in_fp32 else k.dtype, output_final_state)


def chunk_bwd_dh_ref(q, k, v, g, g_gamma, gk, do, h0=None, dht=None, scale: float = 1.0,
                     output_dh0: bool = False, states_in_fp32: bool = False,
                     cu_seqlens_cpu=None, cu_seqlens_dev=None, chunk_size: int = 64):
    """dh [B, NT, H, K, V] float32 (gradient w.r.t. the state after each chunk) and dh0
    [N, H, K, V] float32 (tops/ops/common/chunk_h.py:575-682).  dh0 is returned when
    ``output_dh0`` (or, for varlen input, when h0 or dht is given), else None."""
    del k, v, states_in_fp32
    cu = cu_seqlens_cpu if cu_seqlens_cpu is not None else cu_seqlens_dev
    want = bool(output_dh0) or (cu is not None and (h0 is not None or dht is not None))
    return _recurrence(q, do, g, g_gamma, gk, dht, cu, int(chunk_size), True, float(scale), 1,
                       torch.float32, want)


def chunk_bwd_dh_kernel(q, k, v, g=None, g_gamma=None, gk=None, do=None, dht=None,
                        scale: float = 1.0, output_dh0: bool = False, cu_seqlens_dev=None,
                        chunk_size: int = 128, states_in_fp32: bool = False):
    """Kernel form (tops/ops/common/chunk_h.py:785-884): dh in q.dtype (float32 with
    ``states_in_fp32``), dh0 in the same dtype when ``output_dh0`` else None."""
    del k, v
    require(do is not None, "do must be provided")
    sdt = torch.float32 if states_in_fp32 else q.dtype
    dh, dh0 = _recurrence(q, do, g, g_gamma, gk, dht, cu_seqlens_dev, int(chunk_size), True,
                          float(scale), 1, sdt, bool(output_dh0))
    if dh0 is not None and dh0.dtype != sdt:
        dh0 = dh0.to(sdt)
    return dh, dh0


def chunk_fwd_h_kernel_varlen(k, v, g=None, g_gamma=None, gk=None, gv=None, h0=None,
                              output_final_state: bool = False, cu_seqlens_dev=None,
                              chunk_size: int = 128, split_size: int | None = None,
                              states_in_fp32: bool = False, interpret: bool = False):
    """Packed-varlen form (tops/ops/common/chunk_h.py:970-1113): k [B,T,H,K], v [B,T,H,V]
    with the B*T tokens one packed stream and cu_seqlens_dev [N+1] (multiples of
    chunk_size) its sequence boundaries.  Returns h [B*T / chunk_size, H, K, V] (the state
    before every chunk, k.dtype or float32 with ``states_in_fp32``) and ht [N, H, K, V]
    float32 when ``output_final_state`` else None.  g and gv are rejected as there
    (check_chunk_fwd, chunk_h.py:965-966)."""
    del interpret
    require(g is None, "x should be None.")
    require(gv is None, "x should be None.")
    C = int(chunk_size)
    BS = C if split_size is None else int(split_size)
    require(BS % C == 0, f"The `split_size` (got {BS}) must be a multiple of `chunk_size` {C}")
    require(BS == C, "split_size with cu_seqlens is not supported")
    B, T, H, K = k.shape
    V = v.shape[-1]
    require(T % C == 0, "T mod chunk_size must equal to 0.")
    flat = (lambda x: None if x is None else x.reshape((1, B * T) + tuple(x.shape[2:])))
    cu = cu_seqlens_dev if cu_seqlens_dev is not None else [0, B * T]
    h, ht = _recurrence(flat(k), flat(v), None, g_gamma, flat(gk), h0, cu, C, False, 1.0, 1,
                        torch.float32 if states_in_fp32 else k.dtype, output_final_state)
    return h.reshape(-1, H, K, V), ht


__all__ = ["chunk_fwd_h_ref", "chunk_fwd_h_kernel", "chunk_fwd_h_kernel_varlen", "chunk_bwd_dh_ref",
           "chunk_bwd_dh_kernel"]
