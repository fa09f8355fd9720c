"""chunk_kda_bwd_intra on MI355X (mirrors tops/ops/kda/chunk_intra.py:477-574): the
intra-chunk stage of the KDA backward, propagating dAqk and dAkk back to q, k, beta and
the gate, added to the incoming gradients of the earlier stages.

The fused KDA backward (tops_kda_chunk_bwd) computes this inside its WY kernel; this entry
point serves callers that drive the stages themselves (tops_kda_stage_intra_bwd, one
workgroup per (chunk, head), fp32 MFMA).
"""
from __future__ import annotations

import torch

from ... import _native as N
from ..common._stage import act, f32, require


def chunk_kda_bwd_intra(q, k, g, beta, dAqk, dAkk, dq=None, dk=None, db=None, dg=None,
                        cu_seqlens=None, chunk_indices=None, chunk_size: int = 64,
                        safe_gate: bool = False):
    """q, k [B,T,H,K]; g [B,T,H,K] chunk-local gate cumsum in log2 units; beta [B,T,H];
    dAqk, dAkk [B,T,H,BT] (used on i >= j); incoming dq, dk, dg [B,T,H,K] and db [B,T,H]
    (zeros when None).  Returns (dq, dk, db, dg) with the intra-chunk contributions added,
    each in the dtype of its incoming gradient (q's dtype when None).  cu_seqlens,
    chunk_indices and safe_gate are accepted and unused, as in the reference."""
    del cu_seqlens, chunk_indices, safe_gate
    B, T, H, K = q.shape
    C = int(chunk_size)
    require(C in (16, 32, 64), f"chunk_size must be 16, 32 or 64 on this backend, got {C}")
    for name, t, shp in (("k", k, (B, T, H, K)), ("g", g, (B, T, H, K)), ("beta", beta, (B, T, H)),
                         ("dAqk", dAqk, (B, T, H, C)), ("dAkk", dAkk, (B, T, H, C))):
        require(tuple(t.shape) == shp, f"{name} shape {tuple(t.shape)} != {shp}")
    require(T % C == 0, f"T={T} must be divisible by chunk_size={C}")
    (qk, kk), code = act(q, k)
    outs = [torch.empty((B, T, H, K), device=q.device, dtype=torch.float32) for _ in range(3)]
    dbi = torch.empty((B, T, H), device=q.device, dtype=torch.float32)
    dqi, dki, dgi = outs
    N.call("tops_kda_stage_intra_bwd", N.ptr(qk), N.ptr(kk), code, N.ptr(f32(g)), N.ptr(f32(beta)),
           N.ptr(f32(dAqk)), N.ptr(f32(dAkk)), N.ptr(dqi), N.ptr(dki), N.ptr(dbi), N.ptr(dgi),
           B, T, H, K, C, N.stream())

    def acc(inc, part, dtype):
        if inc is None:
            return part.to(dtype)
        return (inc.float() + part).to(inc.dtype)

    return (acc(dq, dqi, q.dtype), acc(dk, dki, q.dtype), acc(db, dbi, q.dtype),
            acc(dg, dgi, q.dtype))


__all__ = ["chunk_kda_bwd_intra"]
