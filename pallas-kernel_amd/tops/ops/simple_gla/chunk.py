"""Chunked simple GLA on MI355X: drop-in for tops.ops.simple_gla.chunk
(tops/ops/simple_gla/chunk.py) with the gate options of the reference's CPU tier
(tops/cpu/ops/simple_gla/chunk.py:796-889).

Simple GLA gates the whole K x V state with one log-gate per (token, head) -- g
[B,T,H] -- or with a constant per-head log-decay g_gamma [H]:
    S_t = exp(g_t) S_{t-1} + k_t v_t^T,   o_t = scale * S_t^T q_t.
The HIP chunk kernels run it as GLA with the gate shared by all K channels (a
runtime gate mode of the same kernels), so varlen (cu_seqlens), initial and final
states and the backward come with it.

As in the reference: `chunk_simple_gla` keeps the Pallas positional signature
(chunk.py:778-788, g_gamma 4th) with keyword-only g / cu_seqlens added; passing both
g and g_gamma is rejected (the reference backward rejects it,
tops/cpu/ops/simple_gla/chunk.py:724-728); the gradient w.r.t. g_gamma is zero (the
reference custom_vjp treats it as a fixed hyperparameter, chunk.py:762-765); dg for a
per-token g is [B,T,H] fp32.
"""
from __future__ import annotations

import torch

from ...utils import ChunkPlan, inference_inputs
from .._chunk_core import (GATE_S, GATE_GAMMA, PAIRED, check_qkv, chunk_fwd as _core_fwd,
                           chunk_bwd as _core_bwd, pack_states, paired_states,
                           unpack_states)


def _gate(q, g, g_gamma):
    B, T, H, K = q.shape
    if g is not None and g_gamma is not None:
        raise ValueError("chunk_simple_gla: pass only one of g or g_gamma "
                         "(the reference backward rejects both)")
    if g is not None:
        assert tuple(g.shape) == (B, T, H), f"g shape {tuple(g.shape)} != {(B, T, H)}"
        return GATE_S, g
    if g_gamma is not None:
        gg = torch.as_tensor(g_gamma, device=q.device)
        assert gg.numel() == H, f"g_gamma must have H={H} entries, got {tuple(gg.shape)}"
        return GATE_GAMMA, gg
    return GATE_GAMMA, torch.zeros(H, device=q.device, dtype=torch.float32)


class _ChunkSimpleGLA(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, gt, h0, mode, scale, output_final_state, cu_seqlens):
        q, k, v = (x.contiguous() for x in (q, k, v))
        g32 = gt.detach().contiguous().to(torch.float32)
        h032 = None if h0 is None else h0.contiguous().to(torch.float32)
        plan = ChunkPlan.get(q.shape[0], q.shape[1], cu_seqlens, q.device)
        train = any(ctx.needs_input_grad[:5])
        o, ht, hs = _core_fwd(q, k, v, (mode, g32), h032, scale, output_final_state, plan,
                              keep_states=PAIRED if train else False)
        if train:
            ctx.save_for_backward(q, k, v, g32, *pack_states(hs), h032)
            ctx.paired = paired_states(q, q.shape[-1], v.shape[-1])
            ctx.plan, ctx.scale, ctx.mode = plan, scale, mode
            ctx.g_info = (gt.dtype, gt.shape)
            ctx.h0_info = None if h0 is None else h0.dtype
        return o, ht

    @staticmethod
    def backward(ctx, do, dht):
        q, k, v, g32, hs, hsc, h032 = ctx.saved_tensors
        hs = unpack_states(hs, hsc)
        do = do.contiguous().to(q.dtype)
        dht = None if dht is None else dht.contiguous().to(torch.float32)
        dq, dk, dv, dg, dh0 = _core_bwd(q, k, v, (ctx.mode, g32), do, dht, hs, ctx.scale,
                                        ctx.plan, ctx.h0_info is not None, h0=h032,
                                        paired=ctx.paired)
        gdt, gshape = ctx.g_info
        if ctx.mode == GATE_GAMMA:
            dg = torch.zeros(gshape, device=q.device, dtype=gdt)
        else:
            dg = dg.to(gdt)
        if dh0 is not None:
            dh0 = dh0.to(ctx.h0_info)
        return dq, dk, dv, dg, dh0, None, None, None, None


def chunk_simple_gla(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g_gamma: torch.Tensor | None = None,
    initial_state: torch.Tensor | None = None,
    scale: float | None = None,
    output_final_state: bool = False,
    chunk_size: int = 64,
    *,
    g: torch.Tensor | None = None,
    cu_seqlens=None,
):
    """Chunked simple GLA (tops/ops/simple_gla/chunk.py:778-827, gate options of
    tops/cpu/ops/simple_gla/chunk.py:796-889).

    Returns (o [B,T,H,V] in q.dtype, final_state [N,H,K,V] fp32 or None)."""
    assert chunk_size > 0, "chunk_size must be positive"
    mode, gt = _gate(q, g, g_gamma)
    check_qkv(q, k, v, initial_state, cu_seqlens, split_ok=True)
    if scale is None:
        scale = q.shape[-1] ** -0.5
    q, k, v, gt, initial_state = inference_inputs(q, k, v, gt, initial_state)
    o, ht = _ChunkSimpleGLA.apply(q, k, v, gt, initial_state, mode, float(scale),
                                  bool(output_final_state), cu_seqlens)
    return o, (ht if output_final_state else None)


def _alias(new, old, name_new, name_old):
    if old is not None:
        if new is not None and new is not old:
            raise ValueError(f"pass either {name_new} or {name_old}, not both")
        return old
    return new


def chunk_simple_gla_fwd(q, k, v, g=None, g_gamma=None, scale=None, initial_state=None,
                         output_final_state=False, chunk_size: int = 64, cu_seqlens=None, *,
                         h0=None, use_ht=None, cu_seqlens_cpu=None, cu_seqlens_dev=None,
                         interpret=None):
    """Forward orchestrator (tops/cpu/ops/simple_gla/chunk.py:53-129; Pallas
    tops/ops/simple_gla/chunk.py:464-521).  Returns (o, ht).

    Takes both the CPU-reference keywords (initial_state, output_final_state, cu_seqlens)
    and the accelerator ones (h0, use_ht, cu_seqlens_cpu / cu_seqlens_dev; interpret is
    ignored)."""
    del interpret
    initial_state = _alias(initial_state, h0, "initial_state", "h0")
    if use_ht is not None:
        output_final_state = bool(use_ht)
    cu_seqlens = _alias(cu_seqlens, cu_seqlens_cpu if cu_seqlens_cpu is not None else cu_seqlens_dev,
                        "cu_seqlens", "cu_seqlens_cpu")
    mode, gt = _gate(q, g, g_gamma)
    check_qkv(q, k, v, initial_state, cu_seqlens, split_ok=True)
    if scale is None:
        scale = q.shape[-1] ** -0.5
    plan = ChunkPlan.get(q.shape[0], q.shape[1], cu_seqlens, q.device)
    h0 = None if initial_state is None else initial_state.contiguous().to(torch.float32)
    o, ht, _ = _core_fwd(q.contiguous(), k.contiguous(), v.contiguous(),
                         (mode, gt.contiguous().to(torch.float32)), h0, scale,
                         output_final_state, plan, keep_states=False)
    return o, ht


def chunk_simple_gla_fwd_varlen(q, k, v, g=None, g_gamma=None, scale=None, initial_state=None,
                                output_final_state=False, cu_seqlens=None, chunk_size: int = 64,
                                *, h0=None, use_ht=None, cu_seqlens_cpu=None, cu_seqlens_dev=None,
                                interpret=None):
    """Varlen forward (tops/ops/simple_gla/chunk.py:522-577): the same kernels with a
    cu_seqlens chunk map (keywords as chunk_simple_gla_fwd)."""
    del interpret
    initial_state = _alias(initial_state, h0, "initial_state", "h0")
    if use_ht is not None:
        output_final_state = bool(use_ht)
    cu_seqlens = _alias(cu_seqlens, cu_seqlens_cpu if cu_seqlens_cpu is not None else cu_seqlens_dev,
                        "cu_seqlens", "cu_seqlens_cpu")
    assert cu_seqlens is not None, "chunk_simple_gla_fwd_varlen needs cu_seqlens"
    return chunk_simple_gla_fwd(q, k, v, g=g, g_gamma=g_gamma, scale=scale,
                                initial_state=initial_state, output_final_state=output_final_state,
                                chunk_size=chunk_size, cu_seqlens=cu_seqlens)


def chunk_simple_gla_bwd(q, k, v, do, *, g=None, g_gamma=None, scale=None, h0=None, dht=None,
                         cu_seqlens=None, chunk_size: int = 64, cu_seqlens_cpu=None,
                         cu_seqlens_dev=None, interpret=None):
    """Backward orchestrator (tops/ops/simple_gla/chunk.py:579-674 keyword form).

    Returns (dq, dk, dv, dh0) as the reference does for g_gamma (dh0 when h0 is given,
    else None).  The reference rejects a per-token g here; this backend also accepts one
    (gate options of tops/cpu/ops/simple_gla/chunk.py:668-788) and then returns
    (dq, dk, dv, dh0, dg) with dg [B,T,H] fp32."""
    del interpret
    cu_seqlens = _alias(cu_seqlens, cu_seqlens_cpu if cu_seqlens_cpu is not None else cu_seqlens_dev,
                        "cu_seqlens", "cu_seqlens_cpu")
    dq, dk, dv, dg, dh0 = _bwd_all(q, k, v, do, g, g_gamma, scale, h0, dht, cu_seqlens)
    return (dq, dk, dv, dh0) if g is None else (dq, dk, dv, dh0, dg)


def _bwd_all(q, k, v, do, g, g_gamma, scale, h0, dht, cu_seqlens):
    mode, gt = _gate(q, g, g_gamma)
    check_qkv(q, k, v, h0, cu_seqlens, split_ok=True)
    if scale is None:
        scale = q.shape[-1] ** -0.5
    plan = ChunkPlan.get(q.shape[0], q.shape[1], cu_seqlens, q.device)
    q, k, v = (x.contiguous() for x in (q, k, v))
    g32 = gt.contiguous().to(torch.float32)
    h032 = None if h0 is None else h0.contiguous().to(torch.float32)
    _, _, hs = _core_fwd(q, k, v, (mode, g32), h032, scale, False, plan, keep_states=True)
    return _core_bwd(q, k, v, (mode, g32), do.contiguous().to(q.dtype),
                     None if dht is None else dht.contiguous().to(torch.float32), hs, scale, plan,
                     h0 is not None)
