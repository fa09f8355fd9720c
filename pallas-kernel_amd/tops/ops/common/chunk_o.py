"""Simple-GLA chunk stages on MI355X (mirrors tops/ops/common/chunk_o.py): the output from
given states (chunk_fwd_o / chunk_fwd_o_ref), and the backward pieces chunk_bwd_dv,
chunk_bwd_dqkwg and chunk_simple_gla_bwd_o_pl.

The scalar gates (g [B,T,H], the chunk-local cumsum of a per-token log gate, and/or the
per-head constant g_gamma [H]) are the per-channel gate G[t, h, :] = g[t, h] +
g_gamma[h] * (t mod C + 1) shared by all K channels, so each stage runs the GLA stage
kernels of csrc/gla_stages.hip on that broadcast gate (fp32).  Sequences must be
chunk-aligned (as the reference requires), so varlen input is the plain token layout.
"""
from __future__ import annotations

import torch

from ..gla import stages as S
from ._stage import f32, finish, promoted, require
from .cumsum import chunk_local_cumsum  # noqa: F401  (exported here, as the reference does)


def _gate(q, g, g_gamma, C):
    """The per-channel gate [B,T,H,K] fp32 of scalar gates (zeros when neither is given)."""
    B, T, H, K = q.shape
    require(T % C == 0, f"T ({T}) must be a multiple of chunk_size ({C})")
    G = torch.zeros((B, T, H), device=q.device, dtype=torch.float32)
    if g is not None:
        require(tuple(g.shape) == (B, T, H), f"g must be {(B, T, H)}")
        G = G + g.to(torch.float32)
    if g_gamma is not None:
        require(tuple(g_gamma.shape) == (H,), f"g_gamma must be ({H},)")
        ramp = (torch.arange(T, device=q.device) % C + 1).to(torch.float32)
        G = G + ramp[None, :, None] * g_gamma.to(torch.float32)[None, None, :]
    return G[..., None].expand(B, T, H, K).contiguous()


def _states(h, B, T, H, K, V, C):
    NT = T // C
    require(h.numel() == B * NT * H * K * V, f"states must hold {(B, NT, H, K, V)} elements")
    return f32(h.reshape(B, NT, H, K, V))


def chunk_fwd_o(q, k, v, h, *, g=None, g_gamma=None, scale=None, cu_seqlens_cpu=None,
                cu_seqlens_dev=None, chunk_size: int = 64):
    """o [B,T,H,V] in v.dtype = scale * (q e^G h_c + causal(q k^T e^{G_i - G_j}) v) per chunk
    (tops/ops/common/chunk_o.py:443-586); h [B, NT, H, K, V] the state before each chunk."""
    del cu_seqlens_cpu, cu_seqlens_dev
    B, T, H, K = q.shape
    V = v.shape[-1]
    C = int(chunk_size)
    if scale is None:
        scale = K ** -0.5
    G = _gate(q, g, g_gamma, C)
    A = S.chunk_gla_fwd_intra_gk(q, k, G, scale, C)
    return finish(S.chunk_gla_fwd_o_gk(q, v, G, A, _states(h, B, T, H, K, V, C), scale,
                                       chunk_size=C), v.dtype)


chunk_fwd_o_ref = chunk_fwd_o


def chunk_bwd_dv(q, k, do, dh, *, g=None, g_gamma=None, scale=None, cu_seqlens_cpu=None,
                 chunk_size: int = 64):
    """dv = (k e^{G_last - G}) dh_c + causal(q k^T e^{G_i - G_j} scale)^T do per chunk
    (tops/ops/common/chunk_o.py:588-680); dh [B*NT, H, K, V] or [B, NT, H, K, V]."""
    del cu_seqlens_cpu
    B, T, H, K = q.shape
    V = do.shape[-1]
    C = int(chunk_size)
    if scale is None:
        scale = K ** -0.5
    G = _gate(q, g, g_gamma, C)
    A = S.chunk_gla_fwd_intra_gk(q, k, G, scale, C)
    dv = S.chunk_gla_bwd_dv_ref(k, G, A, do, _states(dh, B, T, H, K, V, C), chunk_size=C)
    return finish(dv, do.dtype)


def _dqk(q, k, v, G, h, do, dh, scale, C):
    B, T, H, K = q.shape
    V = v.shape[-1]
    dA = S.chunk_gla_bwd_dA_ref(v.float(), do.float(), scale, chunk_size=C)
    dqi, dki = S.chunk_gla_bwd_dqk_intra_ref(q, k, G, dA, chunk_size=C)
    return S.chunk_gla_bwd_dqkg_ref(q, k, v, _states(h, B, T, H, K, V, C), G, do,
                                    _states(dh, B, T, H, K, V, C), dqi, dki, scale, chunk_size=C)


def chunk_bwd_dqkwg(q, k, v, h, do, dh, *, w=None, g=None, g_gamma=None, dv=None, scale=None,
                    cu_seqlens=None, chunk_size: int = 64):
    """(dq, dk, dw, dg) of tops/ops/common/chunk_o.py:682-880:
      dq = scale (do h^T e^G + causal(do v^T e^{G_i - G_j}) k),
      dk = (v dh^T) e^{G_last - G} + causal(...)^T q,
      dw = -(dv h^T) when w and dv are given (delta rule), else None,
      dg [B,T,H] (per-token g only, else None): the raw per-position gate gradient with the
         chunk-end term folded into each chunk's last position, not reverse-cumsummed.
    dq, dk fp32."""
    del cu_seqlens
    B, T, H, K = q.shape
    V = v.shape[-1]
    C = int(chunk_size)
    if scale is None:
        scale = K ** -0.5
    G = _gate(q, g, g_gamma, C)
    dq, dk, dgc = _dqk(q, k, v, G, h, do, dh, scale, C)
    dw = None
    if w is not None and dv is not None:
        z = torch.zeros((B, T, H, K), device=q.device, dtype=torch.float32)
        zg = torch.zeros_like(z)
        dvh, _, _ = S.chunk_gla_bwd_dqkg_ref(z, z, v, h.reshape(B, T // C, H, K, V), zg,
                                             dv, torch.zeros_like(h).reshape(B, T // C, H, K, V),
                                             z, z, 1.0, chunk_size=C)
        dw = (-dvh).to(w.dtype)
    dg = None
    if g is not None:
        # the per-channel gate gradient is reverse-cumsummed within each chunk; undo that
        # (difference of neighbours, the chunk's last row kept) and sum the channels
        d5 = dgc.reshape(B, T // C, C, H, K)
        raw = d5.clone()
        raw[:, :, :-1] -= d5[:, :, 1:]
        dg = raw.sum(-1).reshape(B, T, H)
    return dq, dk, dw, dg


def chunk_simple_gla_bwd_o_pl(q, k, v, g_gamma, h, do, dh, scale, chunk_size,
                              cu_seqlens_cpu=None, cu_seqlens_dev=None):
    """(dq, dk, dv) in q/k/v dtypes for the constant per-head decay g_gamma, A recomputed
    from q, k (tops/ops/common/chunk_o.py:369-441)."""
    del cu_seqlens_cpu, cu_seqlens_dev
    B, T, H, K = q.shape
    V = v.shape[-1]
    C = int(chunk_size)
    G = _gate(q, None, g_gamma, C)
    dq, dk, _ = _dqk(q, k, v, G, h, do, dh, scale, C)
    A = S.chunk_gla_fwd_intra_gk(q, k, G, scale, C)
    dv = S.chunk_gla_bwd_dv_ref(k, G, A, do, _states(dh, B, T, H, K, V, C), chunk_size=C)
    return dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype)


__all__ = ["chunk_local_cumsum", "chunk_fwd_o", "chunk_fwd_o_ref", "chunk_bwd_dv",
           "chunk_bwd_dqkwg", "chunk_simple_gla_bwd_o_pl"]
