"""Host side of the chunk kernels shared by GLA and simple GLA: argument checks, output
allocation and the C-ABI calls (include/tops_hip.h)."""
from __future__ import annotations

import torch

from typing import NamedTuple

from .. import _native as N
from ..utils import ChunkPlan, cdiv, checkpoint_layout

GATE_K, GATE_S, GATE_GAMMA, GATE_GAMMA_K = "k", "s", "gamma", "gamma_k"


def tiling(K: int, V: int, tile_v: bool):
    """Split of K (and V when tile_v) into equal slices of at most 128, multiples of 8, for
    the kernels' K <= 128 (backward: V <= 128) limit: (nK, K slice, nV, V slice)."""
    nk = -(-K // 128)
    nv = -(-V // 128) if tile_v else 1
    if K % nk or (K // nk) % 8 or V % nv or (V // nv) % 8:
        raise NotImplementedError(f"tops-hip chunk kernels need K and V that split into equal "
                                  f"slices of at most 128, multiples of 8 (got K={K}, V={V})")
    return nk, K // nk, nv, V // nv


def check_qkv(q, k, v, initial_state, cu_seqlens, split_ok: bool = False):
    """Shape / dtype checks.  split_ok: the op is linear in its K and V slices (GLA, simple
    GLA), so K, V > 128 run as slices (tiling); otherwise (delta rule) K <= 128."""
    assert q.ndim == 4, f"q must be [B,T,H,K], got {tuple(q.shape)}"
    B, T, H, K = q.shape
    V = v.shape[-1]
    assert k.shape == q.shape, f"k shape {tuple(k.shape)} != q shape {tuple(q.shape)}"
    assert v.ndim == 4 and v.shape[:3] == (B, T, H), f"v shape {tuple(v.shape)} incompatible with q"
    assert q.dtype == k.dtype == v.dtype, "q, k, v must share a dtype"
    if cu_seqlens is not None:
        assert B == 1, f"B must be 1 for varlen, got {B}"
    n = (len(cu_seqlens) - 1) if cu_seqlens is not None else B
    if initial_state is not None:
        assert tuple(initial_state.shape) == (n, H, K, V), (
            f"initial_state shape {tuple(initial_state.shape)} != {(n, H, K, V)}")
    if split_ok:
        tiling(K, V, True)
    elif K > 128 or K % 8 or V % 8:
        raise NotImplementedError(f"tops-hip chunk kernels need K <= 128 and K, V multiples of 8 "
                                  f"(got K={K}, V={V})")
    N.require_cuda(q, k, v, initial_state)


_GATE_CODE = {GATE_K: 0, GATE_S: 1, GATE_GAMMA: 2, GATE_GAMMA_K: 3}


def _gate_ptrs(gate):
    """(g, g_gamma) pointer pair of the simple-GLA entry points."""
    mode, gt = gate
    return (N.ptr(gt) if mode == GATE_S else None, N.ptr(gt) if mode == GATE_GAMMA else None)


def _segment_states(z, y, gate, s_in, scale, sp, reverse: bool):
    """Incoming state of every segment of a sequence-parallel sweep: the state pass over the
    pieces that hand a state on, then the scan over each sequence's pieces."""
    B, T, H, K = z.shape
    V = y.shape[-1]
    mode, gt = gate
    dev = z.device
    pc = sp.rev if reverse else sp.fwd
    s_loc = dec = None
    if pc.n:
        s_loc = torch.empty(pc.n, H, K, V, device=dev, dtype=torch.float32)
        dec = torch.empty(pc.n, H, K, device=dev, dtype=torch.float32)
        N.call("tops_chunk_state_pass", N.ptr(z), N.ptr(y), N.ptr(gt), _GATE_CODE[mode],
               N.ptr(s_loc), N.ptr(dec), N.ptr(pc.start_dev), N.ptr(pc.end_dev), B * T, H, K, V,
               pc.n, N.chunk_dtype_code(z.dtype), float(scale), int(reverse), N.stream())
    init = torch.empty(sp.Nv, H, K, V, device=dev, dtype=torch.float32)
    N.call("tops_chunk_state_combine", N.ptr(s_loc), N.ptr(dec), N.ptr(s_in), N.ptr(init),
           N.ptr(sp.seg_first_dev), N.ptr(pc.first_dev), N.ptr(pc.dst_dev),
           len(sp.seg_first) - 1, H, K, V, int(reverse), N.stream())
    return init


def paired_states(q, K: int, V: int) -> bool:
    """Whether chunk_fwd(keep_states=PAIRED) keeps the interleaved checkpoints: one
    [chunks, H, K, V] buffer with the state before every even global chunk, into which the
    backward's reverse sweep writes dh after every odd one; the dq / dk / dg kernel rebuilds
    each chunk's other state from its pair partner.  Only with
    tops.utils.set_checkpoint_layout("paired"), bf16 inputs and K, V <= 128."""
    return (checkpoint_layout() == "paired" and q.dtype == torch.bfloat16
            and _direct(q, K, V, True))


PAIRED = "paired"


class States16(NamedTuple):
    """fp16 state checkpoints (the GLA training path for bf16 inputs with per-channel gates):
    h [chunks, H, K, V] fp16 times one factor per (chunk, head, 64-column tile of V), scale
    [chunks, H, ceil(V / 64)] fp32 (include/tops_hip.h, tops_gla_chunk_fwd_c16)."""
    h: torch.Tensor
    scale: torch.Tensor


def _c16(q, mode, K: int, V: int) -> bool:
    """Whether kept states are fp16 checkpoints: bf16, per-channel gates or one gate per token
    (or a scalar g_gamma), one tile, and tops.utils.set_checkpoint_layout "full"."""
    return (q.dtype == torch.bfloat16 and mode in (GATE_K, GATE_S, GATE_GAMMA) and K <= 128
            and V <= 128 and checkpoint_layout() == "full")


def _states_like(hs):
    if isinstance(hs, States16):
        return States16(torch.empty_like(hs.h), torch.empty_like(hs.scale))
    return torch.empty_like(hs)


def states_fp32(hs):
    """Kept states as fp32 [chunks, H, K, V] (fp16 checkpoints scaled back)."""
    if not isinstance(hs, States16):
        return hs
    V = hs.h.shape[-1]
    f = hs.scale.repeat_interleave(64, dim=-1)[..., :V]
    return hs.h.to(torch.float32) * f[:, :, None, :]


def _sptr(hs):
    return N.ptr(hs.h if isinstance(hs, States16) else hs)


def pack_states(hs):
    """(tensor, scale or None) for ctx.save_for_backward."""
    return (hs.h, hs.scale) if isinstance(hs, States16) else (hs, None)


def unpack_states(h, scale):
    return h if scale is None else States16(h, scale)


def _fwd_tile(q, k, v, gate, h0, scale, output_final_state, plan: ChunkPlan, keep_states):
    """Run the forward chunk sweep on one tile (K <= 128).  gate = (mode, fp32 tensor).  Returns (o, ht, h_ckpt).
    Long or few sequences sweep as concurrent segments (plan.segments).  keep_states: False,
    True (every chunk's state) or PAIRED (the interleaved layout, bf16 only)."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    mode, gt = gate
    o = torch.empty_like(v)
    c16 = keep_states is True and _c16(q, mode, K, V)
    if c16:
        hs = States16(torch.empty(plan.total, H, K, V, device=q.device, dtype=torch.float16),
                      torch.empty(plan.total, H, cdiv(V, 64), device=q.device, dtype=torch.float32))
    else:
        hs = torch.empty(plan.total, H, K, V, device=q.device, dtype=torch.float32) \
            if keep_states else None
    sp = plan.segments(H, V)
    if sp is None:
        ht = torch.empty(plan.N, H, K, V, device=q.device, dtype=torch.float32) \
            if output_final_state else None
        s0, fin, cu, offs, Bx, Tx, Nx = h0, ht, plan.cu_dev, plan.offsets_dev, B, T, plan.N
    else:
        s0 = _segment_states(k, v, gate, h0, scale, sp, reverse=False)
        fin = torch.empty(sp.Nv, H, K, V, device=q.device, dtype=torch.float32) \
            if output_final_state else None
        cu, offs, Bx, Tx, Nx = sp.cu_dev, sp.offsets_dev, 1, B * T, sp.Nv
    tail = (N.ptr(s0), N.ptr(o), N.ptr(fin), _sptr(hs), N.ptr(cu), N.ptr(offs),
            Bx, Tx, H, K, V, Nx, N.chunk_dtype_code(q.dtype), float(scale), N.stream())
    if c16 and mode == GATE_K:
        N.call("tops_gla_chunk_fwd_c16", N.ptr(q), N.ptr(k), N.ptr(v), N.ptr(gt), N.ptr(s0),
               N.ptr(o), N.ptr(fin), N.ptr(hs.h), N.ptr(hs.scale), *tail[4:])
    elif c16:
        N.call("tops_simple_gla_chunk_fwd_c16", N.ptr(q), N.ptr(k), N.ptr(v), *_gate_ptrs(gate),
               N.ptr(s0), N.ptr(o), N.ptr(fin), N.ptr(hs.h), N.ptr(hs.scale), *tail[4:])
    elif keep_states == PAIRED:
        N.call("tops_chunk_fwd_paired", N.ptr(q), N.ptr(k), N.ptr(v), N.ptr(gt),
               _GATE_CODE[mode], *tail)
    elif mode == GATE_K:
        N.call("tops_gla_chunk_fwd", N.ptr(q), N.ptr(k), N.ptr(v), N.ptr(gt), *tail)
    elif mode == GATE_GAMMA_K:
        N.call("tops_gla_chunk_fwd_gamma", N.ptr(q), N.ptr(k), N.ptr(v), N.ptr(gt), *tail)
    else:
        N.call("tops_simple_gla_chunk_fwd", N.ptr(q), N.ptr(k), N.ptr(v), *_gate_ptrs(gate),
               *tail)
    ht = fin
    if sp is not None and fin is not None:
        ht = fin.index_select(0, sp.last_dev)
    return o, ht, hs


def _bwd_tile(q, k, v, gate, do, dht, hs, scale, plan: ChunkPlan, want_dh0: bool,
              want_dg: bool = True, h0=None, paired: bool = False):
    """Run the backward (reverse sweep + chunk-parallel dq/dk/dg) on one tile (K, V <= 128).
    Returns (dq, dk, dv, dg, dh0); dg is [B,T,H,K] for GATE_K (and for GATE_GAMMA_K when
    want_dg: the gradient of the per-token gate the constant stands for), [B,T,H] for GATE_S
    and None for GATE_GAMMA.  paired: hs is the interleaved buffer of chunk_fwd(PAIRED) (the
    reverse sweep fills in its odd chunks; h0 is then the forward's initial state)."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    if V > 128:
        raise NotImplementedError("tops-hip chunk backward needs V <= 128")
    mode, gt = gate
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    dg = None
    if mode == GATE_K or (mode == GATE_GAMMA_K and want_dg):
        dg = torch.empty(B, T, H, K, device=q.device, dtype=torch.float32)
    elif mode == GATE_S:
        dg = torch.empty(B, T, H, device=q.device, dtype=torch.float32)
    c16 = isinstance(hs, States16)
    dh_work = hs if paired else _states_like(hs)
    dt, st = N.chunk_dtype_code(q.dtype), N.stream()
    sp = plan.segments(H, V)
    if sp is None:
        dh0 = torch.empty(plan.N, H, K, V, device=q.device, dtype=torch.float32) \
            if want_dh0 else None
        s0, fin, cu, offs, Bx, Tx, Nx = dht, dh0, plan.cu_dev, plan.offsets_dev, B, T, plan.N
    else:
        s0 = _segment_states(q, do, gate, dht, scale, sp, reverse=True)
        fin = torch.empty(sp.Nv, H, K, V, device=q.device, dtype=torch.float32) \
            if want_dh0 else None
        cu, offs, Bx, Tx, Nx = sp.cu_dev, sp.offsets_dev, 1, B * T, sp.Nv
    dh_args = (N.ptr(do), N.ptr(s0), _sptr(dh_work), N.ptr(dv), N.ptr(fin), N.ptr(cu), N.ptr(offs),
               Bx, Tx, H, K, V, Nx, dt, float(scale), st)
    dqkg_tail = (N.ptr(do), _sptr(hs), _sptr(dh_work), N.ptr(dq), N.ptr(dk), N.ptr(dg),
                 N.ptr(plan.cu_dev), N.ptr(plan.offsets_dev), N.ptr(plan.chunk_map_dev),
                 plan.total, B, T, H, K, V, plan.N, dt, float(scale), st)
    if c16 and mode == GATE_K:
        N.call("tops_gla_chunk_bwd_dh_c16", N.ptr(q), N.ptr(k), N.ptr(gt), N.ptr(do), N.ptr(s0),
               N.ptr(dh_work.h), N.ptr(dh_work.scale), *dh_args[3:])
        N.call("tops_gla_chunk_bwd_dqkg_c16", N.ptr(q), N.ptr(k), N.ptr(v), N.ptr(gt), N.ptr(do),
               N.ptr(hs.h), N.ptr(hs.scale), N.ptr(dh_work.h), N.ptr(dh_work.scale),
               *dqkg_tail[3:])
    elif c16:
        N.call("tops_simple_gla_chunk_bwd_dh_c16", N.ptr(q), N.ptr(k), *_gate_ptrs(gate),
               N.ptr(do), N.ptr(s0), N.ptr(dh_work.h), N.ptr(dh_work.scale), *dh_args[3:])
        N.call("tops_simple_gla_chunk_bwd_dqkg_c16", N.ptr(q), N.ptr(k), N.ptr(v),
               *_gate_ptrs(gate), N.ptr(do), N.ptr(hs.h), N.ptr(hs.scale), N.ptr(dh_work.h),
               N.ptr(dh_work.scale), *dqkg_tail[3:])
    elif paired:
        code = _GATE_CODE[mode]
        N.call("tops_chunk_bwd_dh_paired", N.ptr(q), N.ptr(k), N.ptr(gt), code, *dh_args)
        N.call("tops_chunk_bwd_dqkg_paired", N.ptr(q), N.ptr(k), N.ptr(v), N.ptr(gt), code,
               N.ptr(do), N.ptr(h0), N.ptr(dht), N.ptr(hs), N.ptr(dq), N.ptr(dk), N.ptr(dg),
               *dqkg_tail[6:])
    elif mode == GATE_K:
        N.call("tops_gla_chunk_bwd_dh", N.ptr(q), N.ptr(k), N.ptr(gt), *dh_args)
        N.call("tops_gla_chunk_bwd_dqkg", N.ptr(q), N.ptr(k), N.ptr(v), N.ptr(gt), *dqkg_tail)
    elif mode == GATE_GAMMA_K:
        N.call("tops_gla_chunk_bwd_dh_gamma", N.ptr(q), N.ptr(k), N.ptr(gt), *dh_args)
        N.call("tops_gla_chunk_bwd_dqkg_gamma", N.ptr(q), N.ptr(k), N.ptr(v), N.ptr(gt),
               *dqkg_tail)
    else:
        N.call("tops_simple_gla_chunk_bwd_dh", N.ptr(q), N.ptr(k), *_gate_ptrs(gate), *dh_args)
        N.call("tops_simple_gla_chunk_bwd_dqkg", N.ptr(q), N.ptr(k), N.ptr(v), *_gate_ptrs(gate),
               *dqkg_tail)
    dh0 = fin
    if sp is not None and fin is not None:
        dh0 = fin.index_select(0, sp.first_dev)
    return dq, dk, dv, dg, dh0


_KERNEL_DTYPES = (torch.float32, torch.bfloat16, torch.float16)


def _direct(q, K, V, tile_v):
    return q.dtype in _KERNEL_DTYPES and K <= 128 and (V <= 128 or not tile_v)


def _k_gate(gate, k0: int, kw: int):
    """The gate of channel slice [k0, k0 + kw): a strided view for the per-channel forms."""
    mode, gt = gate
    if mode == GATE_K:
        return gt[..., k0:k0 + kw]
    if mode == GATE_GAMMA_K:
        return gt[:, k0:k0 + kw]
    return gt


def _acc(i: int, n: int) -> int:
    """acc_mode of slice i of n (include/tops_hip.h, the sliced entry points)."""
    return 0 if n == 1 else (1 if i == 0 else (3 if i == n - 1 else 2))


def _kv_view(x, k0, kw, v0=None, vw=None):
    """Rows [k0, k0 + kw) (and columns [v0, v0 + vw)) of a [.., K, V] state tensor, as a view."""
    if x is None:
        return None
    x = x[..., k0:k0 + kw, :]
    return x if v0 is None else x[..., v0:v0 + vw]


def _fwd_sliced(q, k, v, gate, h0, scale, output_final_state, plan: ChunkPlan, keep_states):
    """Forward of heads with K > 128 (bf16 / fp32): one sweep per channel slice of at most 128,
    reading strided views of q, k, g and the states (no copies); o is the fp32 sum of the
    slices' outputs, written in v's dtype by the last slice.  Checkpoints keep the whole
    [chunks, H, K, V] layout."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    nk, Kp, _, _ = tiling(K, V, False)
    mode, gt = gate
    dev = q.device
    o = torch.empty_like(v)
    o_sum = torch.empty(B, T, H, V, device=dev, dtype=torch.float32) if nk > 1 else None
    ht = torch.empty(plan.N, H, K, V, device=dev, dtype=torch.float32) if output_final_state else None
    hs = torch.empty(plan.total, H, K, V, device=dev, dtype=torch.float32) if keep_states else None
    code, dt, st = _GATE_CODE[mode], N.chunk_dtype_code(q.dtype), N.stream()
    for a in range(nk):
        k0 = a * Kp
        acc = _acc(a, nk)
        N.call("tops_chunk_fwd_slice", N.ptr(q[..., k0:k0 + Kp]), N.ptr(k[..., k0:k0 + Kp]),
               N.ptr(v), N.ptr(_k_gate(gate, k0, Kp)), code, N.ptr(_kv_view(h0, k0, Kp)),
               N.ptr(o) if acc in (0, 3) else None, N.ptr(o_sum), acc,
               N.ptr(_kv_view(ht, k0, Kp)), N.ptr(_kv_view(hs, k0, Kp)), N.ptr(plan.cu_dev),
               N.ptr(plan.offsets_dev), B, T, H, Kp, V, plan.N, K, dt, float(scale), st)
    return o, ht, hs


def _bwd_sliced(q, k, v, gate, do, dht, hs, scale, plan: ChunkPlan, want_dh0: bool,
                want_dg: bool):
    """Backward of heads beyond one tile (bf16 / fp32): the dh sweep per channel slice (dv
    summed over them in fp32), then dq / dk / dg per (channel slice, value slice) with dq,
    dk summed over the value slices in fp32 and dg accumulated in place."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    nk, Kp, nv, Vp = tiling(K, V, True)
    mode, gt = gate
    dev = q.device
    f32 = torch.float32
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    k_dg = mode == GATE_K or (mode == GATE_GAMMA_K and want_dg)
    dg = torch.empty(B, T, H, K, device=dev, dtype=f32) if k_dg else \
        torch.empty(B, T, H, device=dev, dtype=f32) if mode == GATE_S else None
    dh_work = torch.empty_like(hs)
    dh0 = torch.empty(plan.N, H, K, V, device=dev, dtype=f32) if want_dh0 else None
    dv_sum = torch.empty(B, T, H, V, device=dev, dtype=f32) if nk > 1 else None
    dq_sum = torch.empty(B, T, H, K, device=dev, dtype=f32) if nv > 1 else None
    dk_sum = torch.empty_like(dq_sum) if nv > 1 else None
    code, dt, st = _GATE_CODE[mode], N.chunk_dtype_code(q.dtype), N.stream()
    cu, offs = N.ptr(plan.cu_dev), N.ptr(plan.offsets_dev)
    for a in range(nk):
        k0 = a * Kp
        acc = _acc(a, nk)
        N.call("tops_chunk_bwd_dh_slice", N.ptr(q[..., k0:k0 + Kp]), N.ptr(k[..., k0:k0 + Kp]),
               N.ptr(_k_gate(gate, k0, Kp)), code, N.ptr(do), N.ptr(_kv_view(dht, k0, Kp)),
               N.ptr(_kv_view(dh_work, k0, Kp)), N.ptr(dv) if acc in (0, 3) else None,
               N.ptr(dv_sum), acc, N.ptr(_kv_view(dh0, k0, Kp)), cu, offs, B, T, H, Kp, V,
               plan.N, K, dt, float(scale), st)
    first = True
    for a in range(nk):
        k0 = a * Kp
        ks = slice(k0, k0 + Kp)
        for b in range(nv):
            v0 = b * Vp
            acc = _acc(b, nv)
            dga = None if dg is None else (dg[..., ks] if k_dg else dg)
            dg_accum = int(b > 0) if k_dg else int(not first)
            N.call("tops_chunk_bwd_dqkg_slice", N.ptr(q[..., ks]), N.ptr(k[..., ks]),
                   N.ptr(v[..., v0:v0 + Vp]), N.ptr(_k_gate(gate, k0, Kp)), code,
                   N.ptr(do[..., v0:v0 + Vp]), N.ptr(_kv_view(hs, k0, Kp, v0, Vp)),
                   N.ptr(_kv_view(dh_work, k0, Kp, v0, Vp)),
                   N.ptr(dq[..., ks]) if acc in (0, 3) else None,
                   N.ptr(dk[..., ks]) if acc in (0, 3) else None, N.ptr(dga),
                   N.ptr(None if dq_sum is None else dq_sum[..., ks]),
                   N.ptr(None if dk_sum is None else dk_sum[..., ks]), acc, dg_accum, cu, offs,
                   N.ptr(plan.chunk_map_dev), plan.total, B, T, H, Kp, Vp, plan.N, K, V, dt,
                   float(scale), st)
            first = False
    return dq, dk, dv, dg, dh0


def chunk_fwd(q, k, v, gate, h0, scale, output_final_state, plan: ChunkPlan, keep_states):
    """Forward of GLA / simple GLA.  Returns (o, ht, h_ckpt).  keep_states: False, True or
    PAIRED (the interleaved checkpoints where paired_states() holds, else every chunk's).

    K > 128 runs as channel slices on the strided entry points (the recurrence is separate
    per state entry, so o is the sum of the slices' outputs); V of any width is tiled by the
    sweep itself.  fp32, bf16 and fp16 inputs are read as they are (fp16 and fp32 split
    into bf16 hi / lo halves inside the kernels).  h_ckpt is always [chunks, H, K, V] (or the
    interleaved buffer)."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    if keep_states == PAIRED and not paired_states(q, K, V):
        keep_states = True
    if _direct(q, K, V, False):
        return _fwd_tile(q, k, v, gate, h0, scale, output_final_state, plan, keep_states)
    if q.dtype not in _KERNEL_DTYPES:
        raise TypeError(f"tops-hip chunk kernels take float32, bfloat16 or float16, got {q.dtype}")
    return _fwd_sliced(q, k, v, gate, h0, scale, output_final_state, plan, keep_states)


def chunk_bwd(q, k, v, gate, do, dht, hs, scale, plan: ChunkPlan, want_dh0: bool,
              want_dg: bool = True, h0=None, paired: bool = False):
    """Backward of GLA / simple GLA.  Returns (dq, dk, dv, dg, dh0); dg is [B,T,H,K] for
    GATE_K, [B,T,H] for GATE_S and None for GATE_GAMMA.  K or V > 128 run as slices
    (chunk_fwd); dq, dk, dv come back in the input dtype."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    if _direct(q, K, V, True):
        return _bwd_tile(q, k, v, gate, do, dht, hs, scale, plan, want_dh0, want_dg, h0, paired)
    return _bwd_sliced(q, k, v, gate, do, dht, hs, scale, plan, want_dh0, want_dg)

