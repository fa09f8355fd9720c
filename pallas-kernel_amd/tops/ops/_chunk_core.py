"""Host side of the chunk kernels shared by GLA and simple GLA: argument checks, output
allocation and the C-ABI calls (include/tops_hip.h)."""
from __future__ import annotations

import torch

from .. import _native as N
from ..utils import ChunkPlan

GATE_K, GATE_S, GATE_GAMMA = "k", "s", "gamma"


def check_qkv(q, k, v, initial_state, cu_seqlens):
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
    if K > 128 or K % 8 or V % 8:
        raise NotImplementedError(f"tops-hip chunk kernels need K <= 128 and K, V multiples of 8 "
                                  f"(got K={K}, V={V})")
    N.require_cuda(q, k, v, initial_state)


_GATE_CODE = {GATE_K: 0, GATE_S: 1, GATE_GAMMA: 2}


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
               pc.n, N.dtype_code(z.dtype), float(scale), int(reverse), N.stream())
    init = torch.empty(sp.Nv, H, K, V, device=dev, dtype=torch.float32)
    N.call("tops_chunk_state_combine", N.ptr(s_loc), N.ptr(dec), N.ptr(s_in), N.ptr(init),
           N.ptr(sp.seg_first_dev), N.ptr(pc.first_dev), N.ptr(pc.dst_dev),
           len(sp.seg_first) - 1, H, K, V, int(reverse), N.stream())
    return init


def chunk_fwd(q, k, v, gate, h0, scale, output_final_state, plan: ChunkPlan, keep_states: bool):
    """Run the forward chunk sweep.  gate = (mode, fp32 tensor).  Returns (o, ht, h_ckpt).
    Long or few sequences sweep as concurrent segments (plan.segments)."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    mode, gt = gate
    o = torch.empty_like(v)
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
    tail = (N.ptr(s0), N.ptr(o), N.ptr(fin), N.ptr(hs), N.ptr(cu), N.ptr(offs),
            Bx, Tx, H, K, V, Nx, N.dtype_code(q.dtype), float(scale), N.stream())
    if mode == GATE_K:
        N.call("tops_gla_chunk_fwd", N.ptr(q), N.ptr(k), N.ptr(v), N.ptr(gt), *tail)
    else:
        N.call("tops_simple_gla_chunk_fwd", N.ptr(q), N.ptr(k), N.ptr(v), *_gate_ptrs(gate),
               *tail)
    ht = fin
    if sp is not None and fin is not None:
        ht = fin.index_select(0, sp.last_dev)
    return o, ht, hs


def chunk_bwd(q, k, v, gate, do, dht, hs, scale, plan: ChunkPlan, want_dh0: bool):
    """Run the backward (reverse sweep + chunk-parallel dq/dk/dg).
    Returns (dq, dk, dv, dg, dh0); dg is [B,T,H,K] for GATE_K, [B,T,H] for GATE_S and None
    for GATE_GAMMA."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    if V > 128:
        raise NotImplementedError("tops-hip chunk backward needs V <= 128")
    mode, gt = gate
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    dg = None
    if mode == GATE_K:
        dg = torch.empty(B, T, H, K, device=q.device, dtype=torch.float32)
    elif mode == GATE_S:
        dg = torch.empty(B, T, H, device=q.device, dtype=torch.float32)
    dh_work = torch.empty_like(hs)
    dt, st = N.dtype_code(q.dtype), N.stream()
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
    dh_args = (N.ptr(do), N.ptr(s0), N.ptr(dh_work), N.ptr(dv), N.ptr(fin), N.ptr(cu), N.ptr(offs),
               Bx, Tx, H, K, V, Nx, dt, float(scale), st)
    dqkg_tail = (N.ptr(do), N.ptr(hs), N.ptr(dh_work), N.ptr(dq), N.ptr(dk), N.ptr(dg),
                 N.ptr(plan.cu_dev), N.ptr(plan.offsets_dev), N.ptr(plan.chunk_map_dev),
                 plan.total, B, T, H, K, V, plan.N, dt, float(scale), st)
    if mode == GATE_K:
        N.call("tops_gla_chunk_bwd_dh", N.ptr(q), N.ptr(k), N.ptr(gt), *dh_args)
        N.call("tops_gla_chunk_bwd_dqkg", N.ptr(q), N.ptr(k), N.ptr(v), N.ptr(gt), *dqkg_tail)
    else:
        N.call("tops_simple_gla_chunk_bwd_dh", N.ptr(q), N.ptr(k), *_gate_ptrs(gate), *dh_args)
        N.call("tops_simple_gla_chunk_bwd_dqkg", N.ptr(q), N.ptr(k), N.ptr(v), *_gate_ptrs(gate),
               *dqkg_tail)
    dh0 = fin
    if sp is not None and fin is not None:
        dh0 = fin.index_select(0, sp.first_dev)
    return dq, dk, dv, dg, dh0
