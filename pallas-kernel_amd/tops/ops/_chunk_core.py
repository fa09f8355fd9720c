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


def chunk_fwd(q, k, v, gate, h0, scale, output_final_state, plan: ChunkPlan, keep_states: bool):
    """Run the forward chunk sweep.  gate = (mode, fp32 tensor).  Returns (o, ht, h_ckpt)."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    mode, gt = gate
    o = torch.empty_like(v)
    ht = torch.empty(plan.N, H, K, V, device=q.device, dtype=torch.float32) \
        if output_final_state else None
    hs = torch.empty(plan.total, H, K, V, device=q.device, dtype=torch.float32) \
        if keep_states else None
    tail = (N.ptr(h0), N.ptr(o), N.ptr(ht), N.ptr(hs), N.ptr(plan.cu_dev), N.ptr(plan.offsets_dev),
            B, T, H, K, V, plan.N, N.dtype_code(q.dtype), float(scale), N.stream())
    if mode == GATE_K:
        N.call("tops_gla_chunk_fwd", N.ptr(q), N.ptr(k), N.ptr(v), N.ptr(gt), *tail)
    else:
        N.call("tops_simple_gla_chunk_fwd", N.ptr(q), N.ptr(k), N.ptr(v),
               N.ptr(gt) if mode == GATE_S else None, N.ptr(gt) if mode == GATE_GAMMA else None,
               *tail)
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
    dh0 = torch.empty(plan.N, H, K, V, device=q.device, dtype=torch.float32) if want_dh0 else None
    dh_work = torch.empty_like(hs)
    dt, st = N.dtype_code(q.dtype), N.stream()
    if mode == GATE_K:
        N.call("tops_gla_chunk_bwd_dh", N.ptr(q), N.ptr(k), N.ptr(gt), N.ptr(do), N.ptr(dht),
               N.ptr(dh_work), N.ptr(dv), N.ptr(dh0), N.ptr(plan.cu_dev), N.ptr(plan.offsets_dev),
               B, T, H, K, V, plan.N, dt, float(scale), st)
        N.call("tops_gla_chunk_bwd_dqkg", N.ptr(q), N.ptr(k), N.ptr(v), N.ptr(gt), N.ptr(do),
               N.ptr(hs), N.ptr(dh_work), N.ptr(dq), N.ptr(dk), N.ptr(dg),
               N.ptr(plan.cu_dev), N.ptr(plan.offsets_dev), N.ptr(plan.chunk_map_dev), plan.total,
               B, T, H, K, V, plan.N, dt, float(scale), st)
    else:
        N.call("tops_simple_gla_chunk_bwd", N.ptr(q), N.ptr(k), N.ptr(v),
               N.ptr(gt) if mode == GATE_S else None, N.ptr(gt) if mode == GATE_GAMMA else None,
               N.ptr(do), N.ptr(dht), N.ptr(hs), N.ptr(dh_work), N.ptr(dq), N.ptr(dk), N.ptr(dv),
               N.ptr(dg), N.ptr(dh0), N.ptr(plan.cu_dev), N.ptr(plan.offsets_dev),
               N.ptr(plan.chunk_map_dev), plan.total, B, T, H, K, V, plan.N, dt, float(scale), st)
    return dq, dk, dv, dg, dh0
