"""torch-CPU float32 restatement of the reference's chunked GLA (test / baseline infrastructure).

The same algorithm as oracle/gla.py (tops/cpu/ops/gla/chunk.py: chunk-local gate cumsum,
inter-chunk state recurrence, intra-chunk attention, the backward's reverse state-gradient
recurrence and the dq / dk / dv / dg stages, chunk.py:52-156, 277-466, 551-607; the state
recurrences tops/cpu/ops/common/chunk_h.py:179-226, 387-427), in float32 torch, vectorised
over batch, heads and chunks so that a CPU run uses every core it is given
(torch.set_num_threads).  It is the CPU baseline that bench.py times; it is never the
product path.  Pinned against the float64 oracle by tests/test_oracle_torch_cpu.py.

Layout inside: [B, H, NT, C, D] (chunks contiguous per head) so every product is a batched
matrix product.  Fixed-length sequences with T % C == 0.
"""
from __future__ import annotations

import torch


def _chunks(x, C):
    B, T, H, D = x.shape
    return x.reshape(B, T // C, C, H, D).permute(0, 3, 1, 2, 4).contiguous()   # [B,H,NT,C,D]


def _unchunk(x):
    B, H, NT, C, D = x.shape
    return x.permute(0, 2, 3, 1, 4).reshape(B, NT * C, H, D)


def chunk_gla_fwd_bwd(q, k, v, g, h0, do, dht, scale, C=64, backward=True):
    """Forward (o, ht) and, when `backward`, the gradients (dq, dk, dv, dg, dh0) of
    L = <o, do> + <ht, dht>.  All float32 CPU tensors in the reference layout
    q, k, g [B,T,H,K]; v, do [B,T,H,V]; h0, dht [B,H,K,V]."""
    f = torch.float32
    q, k, v, g, do = (x.to(f) for x in (q, k, v, g, do))
    B, T, H, K = q.shape
    V = v.shape[-1]
    NT = T // C
    qc, kc, vc, gc_raw, doc = (_chunks(x, C) for x in (q, k, v, g, do))
    gc = gc_raw.cumsum(dim=3)                                  # chunk-local cumsum
    gl = gc[:, :, :, -1]                                       # [B,H,NT,K]  Gamma
    gn = gc[:, :, :, :1]                                       # first row: reference point
    qg = qc * torch.exp(gc - gn)
    kg = kc * torch.exp(gn - gc)
    mask = torch.tril(torch.ones(C, C, dtype=torch.bool))
    A = torch.matmul(qg, kg.transpose(-1, -2)) * scale        # [B,H,NT,C,C]
    A = A.masked_fill(~mask, 0.0)
    kdec = kc * torch.exp(gl[:, :, :, None] - gc)              # k * exp(Gamma - G)
    eg = torch.exp(gl)                                         # [B,H,NT,K]
    # state before every chunk
    hs = torch.empty(B, H, NT, K, V, dtype=f)
    h = torch.zeros(B, H, K, V, dtype=f) if h0 is None else h0.to(f).clone()
    kv = torch.matmul(kdec.transpose(-1, -2), vc)              # [B,H,NT,K,V]
    for i in range(NT):
        hs[:, :, i] = h
        h = h * eg[:, :, i, :, None] + kv[:, :, i]
    ht = h
    qe = qc * torch.exp(gc)
    o = torch.matmul(qe, hs) * scale + torch.matmul(A, vc)
    if not backward:
        return _unchunk(o), ht
    # reverse state gradient: dhs[:, :, i] = gradient w.r.t. the state after chunk i
    qd = torch.matmul((qe * scale).transpose(-1, -2), doc)     # [B,H,NT,K,V]
    dhs = torch.empty(B, H, NT, K, V, dtype=f)
    dh = torch.zeros(B, H, K, V, dtype=f) if dht is None else dht.to(f).clone()
    for i in range(NT - 1, -1, -1):
        dhs[:, :, i] = dh
        dh = dh * eg[:, :, i, :, None] + qd[:, :, i]
    dh0 = dh
    dv = torch.matmul(A.transpose(-1, -2), doc) + torch.matmul(kdec, dhs)
    dA = (torch.matmul(doc, vc.transpose(-1, -2)) * scale).masked_fill(~mask, 0.0)
    dq = torch.exp(gc) * torch.matmul(dA, kc * torch.exp(-gc))
    dk = torch.exp(-gc) * torch.matmul(dA.transpose(-1, -2), qe)
    dq = dq + scale * torch.exp(gc) * torch.matmul(doc, hs.transpose(-1, -2))
    dk_inter = torch.exp(gl[:, :, :, None] - gc) * torch.matmul(vc, dhs.transpose(-1, -2))
    dk = dk + dk_inter
    dgk_inter = eg * (hs * dhs).sum(dim=-1) + (dk_inter * kc).sum(dim=3)
    dg_raw = qc * dq - kc * dk
    dg = dg_raw.flip(3).cumsum(3).flip(3) + dgk_inter[:, :, :, None]
    return (_unchunk(o), ht, _unchunk(dq), _unchunk(dk), _unchunk(dv), _unchunk(dg), dh0)
