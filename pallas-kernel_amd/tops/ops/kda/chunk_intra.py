"""The intra-chunk stages of KDA on MI355X (mirror tops/ops/kda/chunk_intra.py):

  kda_intra_chunk_fwd (:169-281): per chunk, Aqk, the (I + Akk)^-1 solve giving u, w and
      Akk_inv, and the gated qg, kg (tops_kda_stage_intra_fwd, csrc/kda_stages.hip: one
      workgroup per (batch, head, chunk), fp32);
  chunk_kda_bwd_intra (:477-574): dAqk and dAkk propagated back to q, k, beta and the gate,
      added to the incoming gradients of the earlier stages (tops_kda_stage_intra_bwd, one
      workgroup per (chunk, head), fp32 MFMA).

The fused KDA path (tops_kda_chunk_fwd / _bwd) computes both inside its own kernels; these
entry points serve callers that drive the stages themselves.
"""
from __future__ import annotations

import torch

from ... import _native as N
from ..common._stage import act, f32, require


def kda_intra_chunk_fwd(q, k, g, beta, v, segment_ids=None, scale: float = 1.0,
                        chunk_size: int = 128):
    """Head-first q, k, g [B,H,T,K] (g the chunk-local gate cumsum, log2 units), beta
    [B,H,T], v [B,H,T,V]; segment_ids [B,T] (tokens of different segments do not interact;
    None: one segment).  Returns (u [B,H,T,V], w, qg, kg [B,H,T,K], Aqk, Akk_inv
    [B,H,NC,C,C]), all in k.dtype, as the reference."""
    B, H, T, K = k.shape
    V = v.shape[-1]
    C = int(chunk_size)
    require(T % C == 0, "Sequence length must be divisible by chunk_size")
    for name, t, shp in (("q", q, (B, H, T, K)), ("g", g, (B, H, T, K)), ("beta", beta, (B, H, T)),
                         ("v", v, (B, H, T, V))):
        require(tuple(t.shape) == shp, f"{name} shape {tuple(t.shape)} != {shp}")
    if C not in (16, 32, 64, 128):
        raise NotImplementedError(f"tops-hip kda_intra_chunk_fwd takes chunk_size 16, 32, 64 or "
                                  f"128, got {C}")
    seg = None
    if segment_ids is not None:
        seg = torch.as_tensor(segment_ids, device=k.device).to(torch.int32).contiguous()
        require(tuple(seg.shape) == (B, T), f"segment_ids shape {tuple(seg.shape)} != {(B, T)}")
    (qq, kk, vv), code = act(q, k, v)
    dev, dt = k.device, kk.dtype
    u = torch.empty(B, H, T, V, device=dev, dtype=dt)
    w, qg, kg = (torch.empty(B, H, T, K, device=dev, dtype=dt) for _ in range(3))
    Aqk, Akk_inv = (torch.empty(B, H, T // C, C, C, device=dev, dtype=dt) for _ in range(2))
    N.call("tops_kda_stage_intra_fwd", N.ptr(qq), N.ptr(kk), N.ptr(f32(g)), N.ptr(f32(beta)),
           N.ptr(vv), N.ptr(seg), code, N.ptr(u), N.ptr(w), N.ptr(qg), N.ptr(kg), N.ptr(Aqk),
           N.ptr(Akk_inv), B, H, T, K, V, C, float(scale), N.stream())
    out = (u, w, qg, kg, Aqk, Akk_inv)
    return tuple(x if x.dtype == k.dtype else x.to(k.dtype) for x in out)


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


__all__ = ["kda_intra_chunk_fwd", "chunk_kda_bwd_intra"]
