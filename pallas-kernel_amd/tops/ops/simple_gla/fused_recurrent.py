"""fused_recurrent_simple_gla on MI355X (tops/ops/simple_gla/fused_recurrent.py:146-240).

The per-token simple-GLA recurrence h_t = h_{t-1} exp(g_t + g_gamma) + k_t v_t^T,
o_t = h_t^T (scale q_t) is GLA's with the gate shared by all K channels.  In forward time
order it runs on the chunk kernels' per-token scalar-gate mode (tops.ops.simple_gla
chunk_simple_gla with g [B,T,H]: the same sums grouped by 64-token chunks); g and g_gamma
are combined into that one [B,T,H] gate, g + g_gamma (tops/cpu/ops/simple_gla/naive.py:
113-125).  reverse=True (the recurrence iterated from the last token) runs on the reverse
chunk sweep when no gradient is wanted, else on every sequence reversed in time
(tops.ops.gla.fused_recurrent.reverse_chunk_native / _reversed_chunk).  Shapes the chunk kernels do not take run the per-token
kernels of tops.ops.gla.fused_recurrent_gla with the gate as a broadcast view over K.  Calls
of at most a few tokens per sequence that need no gradient (decode steps) run on the decode
kernel (tops.ops.gla.fused_recurrent.decode_native) with the gate broadcast over K, which at
that length costs a few KB.  Either way the combination is part of the
autograd graph, so the gradients w.r.t. g [B,T,H] and g_gamma [H] come back summed over the
broadcast axes: the gradient of the reference's lax.scan.
"""
from __future__ import annotations

import torch

from ..gla.fused_recurrent import (_reversed_chunk, decode_native, decode_sized,
                                   fused_recurrent_gla, reverse_chunk_native)
from .chunk import chunk_simple_gla


def fused_recurrent_simple_gla(q, k, v, g=None, g_gamma=None, scale=None, initial_state=None,
                               output_final_state=False, reverse=False, cu_seqlens=None):
    """Returns (o [B,T,H,V] in q.dtype, final_state [N,H,K,V] fp32 or None)."""
    B, T, H, K = q.shape
    assert g is None or tuple(g.shape) == (B, T, H), f"g shape {tuple(g.shape)} != {(B, T, H)}"
    assert g_gamma is None or tuple(g_gamma.shape) == (H,), f"g_gamma shape must be ({H},)"
    V = v.shape[-1]
    if decode_sized(T, cu_seqlens):
        gk = None
        if g is not None or g_gamma is not None:
            gk = torch.zeros(B, T, H, 1, device=q.device, dtype=torch.float32)
            if g is not None:
                gk = gk + g.to(torch.float32)[..., None]
            if g_gamma is not None:
                gk = gk + torch.as_tensor(g_gamma, device=q.device).to(torch.float32)[None, None, :, None]
            gk = gk.expand(B, T, H, K)
        sc = K ** -0.5 if scale is None else scale
        r = decode_native(q, k, v, gk, None, initial_state, sc, output_final_state, reverse,
                          cu_seqlens)
        if r is not None:
            return r
    if K % 8 == 0 and V % 8 == 0 and K <= 128 and V <= 128:
        gs = None
        if g is not None:
            gs = g.to(torch.float32)
        if g_gamma is not None:
            gg = torch.as_tensor(g_gamma, device=q.device).to(torch.float32)
            gs = gg.expand(B, T, H) if gs is None else gs + gg

        def run(q_, k_, v_, g_, cu_seqlens=None):
            return chunk_simple_gla(q_, k_, v_, None, initial_state=initial_state, scale=scale,
                                    output_final_state=output_final_state, g=g_,
                                    cu_seqlens=cu_seqlens)
        if reverse:
            sc = K ** -0.5 if scale is None else scale
            if g is None and g_gamma is not None:
                r = reverse_chunk_native(q, k, v, "gamma", gg, initial_state, sc,
                                         output_final_state, cu_seqlens)
            else:
                r = reverse_chunk_native(q, k, v, "s" if gs is not None else "gamma",
                                         gs if gs is not None else torch.zeros(H, device=q.device),
                                         initial_state, sc, output_final_state, cu_seqlens)
            if r is not None:
                return r
            return _reversed_chunk(run, q, k, v, gs, cu_seqlens)
        return run(q, k, v, gs, cu_seqlens)
    gk = None
    if g is not None:
        gk = g.to(torch.float32)[..., None]
    if g_gamma is not None:
        gg = torch.as_tensor(g_gamma, device=q.device).to(torch.float32)[None, None, :, None]
        gk = gg if gk is None else gk + gg
    if gk is not None:
        gk = gk.expand(B, T, H, K)
    return fused_recurrent_gla(q, k, v, gk, None, scale=scale, initial_state=initial_state,
                               output_final_state=output_final_state, reverse=reverse,
                               cu_seqlens=cu_seqlens)
