"""fused_chunk_simple_gla on MI355X (tops/ops/simple_gla/fused_chunk.py:28-555).

The reference's fused-chunk variant keeps the state on-chip across chunks (h never reaches
HBM in the forward, dh never in the backward).  The tops-hip forward sweep already keeps the
state in registers for every chunk op; this op is its own autograd function over the g_gamma
gate mode of those kernels with the reference custom_vjp's contract
(fused_chunk.py:435-500): o and the final state in q.dtype, dq / dk / dv / dh0 in dO's dtype,
and a zero gradient for g_gamma (a fixed per-head decay).  The state checkpoints of the
forward are kept for the backward, as the reference's residuals keep its inputs."""
from __future__ import annotations

import torch

from ...utils import ChunkPlan, inference_inputs
from .._chunk_core import (GATE_GAMMA, PAIRED, check_qkv, chunk_fwd as _core_fwd,
                           chunk_bwd as _core_bwd, pack_states, paired_states,
                           unpack_states)
from .chunk import chunk_simple_gla_fwd, chunk_simple_gla_bwd


class _FusedChunkSimpleGLA(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, g_gamma, h0, scale, output_final_state):
        dtype = q.dtype
        q, k, v = (x.contiguous() for x in (q, k, v))
        gg = g_gamma.detach().contiguous().to(torch.float32)
        h032 = None if h0 is None else h0.contiguous().to(torch.float32)
        plan = ChunkPlan.get(q.shape[0], q.shape[1], None, q.device)
        train = any(ctx.needs_input_grad[:5])
        o, ht, hs = _core_fwd(q, k, v, (GATE_GAMMA, gg), h032, scale, output_final_state, plan,
                              keep_states=PAIRED if train else False)
        if train:
            ctx.save_for_backward(q, k, v, gg, *pack_states(hs), h032)
            ctx.paired = paired_states(q, q.shape[-1], v.shape[-1])
            ctx.plan, ctx.scale, ctx.has_h0 = plan, scale, h0 is not None
            ctx.g_info = (g_gamma.dtype, g_gamma.shape)
        return o.to(dtype), (ht.to(dtype) if ht is not None else None)

    @staticmethod
    def backward(ctx, do, dht):
        q, k, v, gg, hs, hsc, h032 = ctx.saved_tensors
        hs = unpack_states(hs, hsc)
        qkv_dtype = do.dtype
        dht = None if dht is None else dht.contiguous().to(torch.float32)
        dq, dk, dv, _, dh0 = _core_bwd(q, k, v, (GATE_GAMMA, gg), do.contiguous().to(q.dtype), dht,
                                       hs, ctx.scale, ctx.plan, ctx.has_h0, h0=h032,
                                       paired=ctx.paired)
        dg = torch.zeros(ctx.g_info[1], device=q.device, dtype=torch.float32)
        if dh0 is not None:
            dh0 = dh0.to(qkv_dtype)
        return dq.to(qkv_dtype), dk.to(qkv_dtype), dv.to(qkv_dtype), dg, dh0, None, None


def fused_chunk_simple_gla(q, k, v, g_gamma, initial_state=None, scale=None,
                           output_final_state=False, chunk_size=64):
    """tops/ops/simple_gla/fused_chunk.py:503-555 (custom_vjp, nondiff scale /
    output_final_state / chunk_size; g_gamma [H]; initial_state [B, H, K, V]).

    Returns (o [B,T,H,V], final_state [B,H,K,V] or None), both in q.dtype.  The kernels tile
    by 64 whatever chunk_size is (the same result up to fp32 rounding)."""
    assert chunk_size > 0, "chunk_size must be positive"
    B, T, H, K = q.shape
    gg = torch.as_tensor(g_gamma, device=q.device)
    assert gg.numel() == H, f"g_gamma must have H={H} entries, got {tuple(gg.shape)}"
    check_qkv(q, k, v, initial_state, None, split_ok=True)
    if scale is None:
        scale = K ** -0.5
    q, k, v, gg, initial_state = inference_inputs(q, k, v, gg, initial_state)
    o, ht = _FusedChunkSimpleGLA.apply(q, k, v, gg, initial_state, float(scale),
                                       bool(output_final_state))
    return o, (ht if output_final_state else None)


def fused_chunk_simple_gla_fwd(q, k, v, g_gamma=None, scale=None, initial_state=None,
                               output_final_state=False, chunk_size=64, *, g=None, h0=None,
                               use_ht=None, cu_seqlens_cpu=None, cu_seqlens_dev=None,
                               interpret=None):
    """tops/ops/simple_gla/fused_chunk.py:28-60 forward: returns (o, ht).  Accepts the
    accelerator keywords (g, h0, use_ht, cu_seqlens_cpu / _dev) as chunk_simple_gla_fwd."""
    return chunk_simple_gla_fwd(q, k, v, g=g, g_gamma=g_gamma, scale=scale,
                                initial_state=initial_state, output_final_state=output_final_state,
                                chunk_size=chunk_size, h0=h0, use_ht=use_ht,
                                cu_seqlens_cpu=cu_seqlens_cpu, cu_seqlens_dev=cu_seqlens_dev,
                                interpret=interpret)


def fused_chunk_simple_gla_bwd(q, k, v, do, g_gamma=None, scale=None, h0=None, dht=None,
                               chunk_size=64, *, g=None, cu_seqlens_cpu=None,
                               cu_seqlens_dev=None, interpret=None):
    """tops/ops/simple_gla/fused_chunk.py:307-402 backward: returns (dq, dk, dv, dh0)."""
    assert g is None, "per-element gating not supported in fused_chunk_simple_gla_bwd"
    return chunk_simple_gla_bwd(q, k, v, do, g_gamma=g_gamma, scale=scale, h0=h0, dht=dht,
                                chunk_size=chunk_size, cu_seqlens_cpu=cu_seqlens_cpu,
                                cu_seqlens_dev=cu_seqlens_dev, interpret=interpret)
