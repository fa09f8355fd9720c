"""torch-CPU float32 restatements of the reference's chunked GLA, simple GLA and KDA (test and
baseline infrastructure).

The same algorithm as oracle/gla.py (tops/cpu/ops/gla/chunk.py: chunk-local gate cumsum,
inter-chunk state recurrence, intra-chunk attention, the backward's reverse state-gradient
recurrence and the dq / dk / dv / dg stages, chunk.py:52-156, 277-466, 551-607; the state
recurrences tops/cpu/ops/common/chunk_h.py:179-226, 387-427), in float32 torch, vectorised
over batch, heads and chunks so that a CPU run uses every core it is given
(torch.set_num_threads).  It is the CPU baseline that bench.py times; it is never the
product path.  Pinned against the float64 oracle by tests/test_oracle_torch_cpu.py.

Also restated: simple GLA (tops/cpu/ops/simple_gla/chunk.py:53-129, 668-788: one log-gate per
token and head, varlen by per-sequence runs) and KDA (tops/cpu/ops/kda/naive.py:121-313, the
chunked WY form; its backward is torch autograd of that forward, i.e. the gradients of the same
function tops/cpu/ops/kda/chunk_bwd.py:525-668 computes by hand).

Layout inside: [B, H, NT, C, D] (chunks contiguous per head) so every product is a batched
matrix product.  chunk_gla_fwd_bwd takes fixed-length sequences with T % C == 0; the simple-GLA
and KDA entry points zero-pad a ragged tail (a zero token with a zero gate leaves the state as it
is and adds nothing).
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
    q, k, v, g = (x.to(f) for x in (q, k, v, g))
    B, T, H, K = q.shape
    V = v.shape[-1]
    NT = T // C
    qc, kc, vc, gc_raw = (_chunks(x, C) for x in (q, k, v, g))
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
    doc = _chunks(do.to(f), C)
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


def _pad_t(x, C):
    """Zero-pad axis 1 (time) to a multiple of C."""
    T = x.shape[1]
    Tp = -(-T // C) * C
    if Tp == T:
        return x
    return torch.nn.functional.pad(x, (0, 0) * (x.dim() - 2) + (0, Tp - T))


def _simple_seq(q, k, v, g, h0, do, dht, scale, C, backward):
    """One batch of fixed-length sequences (T % C == 0) of simple GLA, g [B,T,H] natural log.
    Inside a chunk the decay between rows i >= j is exp(G_i - G_j) <= 1, taken only on the
    causal side, so strong gates neither overflow nor underflow to NaN."""
    f = torch.float32
    B, T, H, K = q.shape
    V = v.shape[-1]
    NT = T // C
    qc, kc, vc = (_chunks(x.to(f), C) for x in (q, k, v))
    gc = g.to(f).reshape(B, NT, C, H).permute(0, 3, 1, 2).cumsum(-1)   # [B,H,NT,C]
    gl = gc[..., -1]                                                    # [B,H,NT]
    mask = torch.tril(torch.ones(C, C, dtype=torch.bool))
    diff = (gc[..., :, None] - gc[..., None, :]).masked_fill(~mask, 0.0)
    D = torch.exp(diff).masked_fill(~mask, 0.0)                         # [B,H,NT,C,C]
    A = torch.matmul(qc, kc.transpose(-1, -2)) * D * scale
    kdec = kc * torch.exp(gl[..., None] - gc)[..., None]
    hs = torch.empty(B, H, NT, K, V, dtype=f)
    h = torch.zeros(B, H, K, V, dtype=f) if h0 is None else h0.to(f).clone()
    kv = torch.matmul(kdec.transpose(-1, -2), vc)
    eg = torch.exp(gl)
    for i in range(NT):
        hs[:, :, i] = h
        h = h * eg[:, :, i, None, None] + kv[:, :, i]
    ht = h
    qe = qc * torch.exp(gc)[..., None]
    o = torch.matmul(qe, hs) * scale + torch.matmul(A, vc)
    if not backward:
        return _unchunk(o), ht
    doc = _chunks(do.to(f), C)
    qd = torch.matmul((qe * scale).transpose(-1, -2), doc)
    dhs = torch.empty(B, H, NT, K, V, dtype=f)
    dh = torch.zeros(B, H, K, V, dtype=f) if dht is None else dht.to(f).clone()
    for i in range(NT - 1, -1, -1):
        dhs[:, :, i] = dh
        dh = dh * eg[:, :, i, None, None] + qd[:, :, i]
    dh0 = dh
    dv = torch.matmul(A.transpose(-1, -2), doc) + torch.matmul(kdec, dhs)
    dAD = torch.matmul(doc, vc.transpose(-1, -2)) * scale * D          # dA with the decay
    dq = torch.matmul(dAD, kc) + scale * torch.exp(gc)[..., None] * torch.matmul(doc, hs.transpose(-1, -2))
    dk_inter = torch.exp(gl[..., None] - gc)[..., None] * torch.matmul(vc, dhs.transpose(-1, -2))
    dk = torch.matmul(dAD.transpose(-1, -2), qc) + dk_inter
    # per-token gate gradient: the channel sum of the per-channel form (reverse in-chunk
    # cumsum of q.dq - k.dk, plus the state terms, which every row of the chunk receives)
    dg_raw = (qc * dq - kc * dk).sum(-1)                                # [B,H,NT,C]
    inter = eg * (hs * dhs).sum((-1, -2)) + (dk_inter * kc).sum((-1, -2))
    dg = dg_raw.flip(-1).cumsum(-1).flip(-1) + inter[..., None]
    dg = dg.permute(0, 2, 3, 1).reshape(B, T, H)
    return (_unchunk(o), ht, _unchunk(dq), _unchunk(dk), _unchunk(dv), dg, dh0)


def chunk_simple_gla_fwd_bwd(q, k, v, g, scale, h0=None, do=None, dht=None, cu_seqlens=None,
                             C=64, backward=True):
    """Simple GLA (one natural-log gate per token and head, g [B,T,H]) forward (o, ht) and,
    when `backward`, the gradients (dq, dk, dv, dg [B,T,H], dh0) of <o, do> + <ht, dht>.
    cu_seqlens (B = 1): each sequence runs on its own; h0 / dht / ht / dh0 are [N,H,K,V]."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    spans = [(b, 0, T) for b in range(B)] if cu_seqlens is None else \
        [(0, int(cu_seqlens[i]), int(cu_seqlens[i + 1])) for i in range(len(cu_seqlens) - 1)]
    n = len(spans)
    f = torch.float32
    o = torch.zeros(B, T, H, V, dtype=f)
    ht = torch.zeros(n, H, K, V, dtype=f)
    grads = None
    if backward:
        grads = [torch.zeros(B, T, H, K, dtype=f), torch.zeros(B, T, H, K, dtype=f),
                 torch.zeros(B, T, H, V, dtype=f), torch.zeros(B, T, H, dtype=f),
                 torch.zeros(n, H, K, V, dtype=f)]
    if cu_seqlens is None:
        groups = [(list(range(n)), slice(0, B), 0, T)]
    else:
        groups = [([i], slice(0, 1), s, e) for i, (_, s, e) in enumerate(spans)]
    for idx, bs, s, e in groups:
        if e == s:
            if h0 is not None:
                ht[idx] = h0[idx].to(f)
            if backward and dht is not None:
                grads[4][idx] = dht[idx].to(f)
            continue
        sl = lambda x: _pad_t(x[bs, s:e], C)    # noqa: E731
        h0i = None if h0 is None else h0[idx]
        dhti = None if dht is None else dht[idx]
        out = _simple_seq(sl(q), sl(k), sl(v), sl(g), h0i, None if do is None else sl(do),
                          dhti, scale, C, backward)
        L = e - s
        o[bs, s:e] = out[0][:, :L]
        ht[idx] = out[1]
        if backward:
            for j, x in enumerate(out[2:6]):
                grads[j][bs, s:e] = x[:, :L]
            grads[4][idx] = out[6]
    if not backward:
        return o, ht
    return (o, ht, *grads)


def _kda_fwd_graph(q, k, v, g, beta, h0, scale, C):
    """KDA forward on float32 tensors that may require grad (T % C == 0).  Per chunk, with
    G the in-chunk cumsum of the natural-log gate and Gm = (G_first + G_last) / 2 per channel
    (every exponent below is at most half the chunk's total decay):
        Akk_ij = beta_i sum_d k_id k_jd exp(G_id - G_jd) (i > j),  T = (I + Akk)^-1
        u = T (beta v),  w = T (beta exp(G) k),  v_new = u - w S
        o = scale (q exp(G)) S + tril(scale q exp(G - Gm) (k exp(Gm - G))^T) v_new
        S <- exp(G_last) S + (k exp(G_last - G))^T v_new."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    NT = T // C
    qc, kc, vc, gc = (_chunks(x, C) for x in (q, k, v, g))
    bc = beta.reshape(B, NT, C, H).permute(0, 3, 1, 2)                 # [B,H,NT,C]
    G = gc.cumsum(3)
    Gl = G[:, :, :, -1:]                                                # [B,H,NT,1,K]
    Gm = 0.5 * (G[:, :, :, :1] + Gl)
    kp, km = kc * torch.exp(G - Gm), kc * torch.exp(Gm - G)
    qp = qc * torch.exp(G - Gm)
    low = torch.tril(torch.ones(C, C, dtype=torch.bool), -1)
    cau = torch.tril(torch.ones(C, C, dtype=torch.bool))
    Akk = (torch.matmul(kp, km.transpose(-1, -2)) * bc[..., None]).masked_fill(~low, 0.0)
    eye = torch.eye(C, dtype=q.dtype)
    Tm = torch.linalg.solve_triangular(eye + Akk, eye.expand_as(Akk), upper=False,
                                       unitriangular=True)
    u = torch.matmul(Tm, vc * bc[..., None])
    w = torch.matmul(Tm, kc * torch.exp(G) * bc[..., None])
    Aqk = (torch.matmul(qp, km.transpose(-1, -2)) * scale).masked_fill(~cau, 0.0)
    qe = qc * torch.exp(G) * scale
    kdec = kc * torch.exp(Gl - G)
    egl = torch.exp(Gl[:, :, :, 0])                                     # [B,H,NT,K]
    S = torch.zeros(B, H, K, V, dtype=q.dtype) if h0 is None else h0
    outs = []
    # per-chunk views by unbind: its backward stacks once, where indexing inside the loop
    # would give every chunk's gradient a full-size zero tensor
    per = zip(*(x.unbind(2) for x in (u, w, qe, Aqk, kdec, egl)))
    for un, wn, qn, an, kn, en in per:
        vn = un - torch.matmul(wn, S)
        outs.append(torch.matmul(qn, S) + torch.matmul(an, vn))
        S = S * en[..., None] + torch.matmul(kn.transpose(-1, -2), vn)
    o = torch.stack(outs, 2)                                            # [B,H,NT,C,V]
    return _unchunk(o), S


def chunk_kda_fwd_bwd(q, k, v, g, beta, scale, h0=None, do=None, dht=None, C=64,
                      backward=True):
    """KDA forward (o, ht) and, when `backward`, (dq, dk, dv, dbeta, dg, dh0): torch autograd
    of the chunked forward for L = <o, do> + <ht, dht> (dg w.r.t. the natural-log gate, dh0 only
    with h0).  q, k, g [B,T,H,K]; v, do [B,T,H,V]; beta [B,T,H]; h0, dht [B,H,K,V]."""
    f = torch.float32
    T = q.shape[1]
    xs = [_pad_t(x.detach().to(f), C) for x in (q, k, v, g, beta)]
    h = None if h0 is None else h0.detach().to(f)
    if not backward:
        with torch.no_grad():
            o, ht = _kda_fwd_graph(*xs, h, scale, C)
        return o[:, :T], ht
    leaves = [x.clone().requires_grad_() for x in xs]
    hl = None if h is None else h.clone().requires_grad_()
    with torch.enable_grad():
        o, ht = _kda_fwd_graph(*leaves, hl, scale, C)
        outs, cots = [o], [_pad_t(do.to(f), C)]
        if dht is not None:
            outs.append(ht)
            cots.append(dht.to(f))
        want = leaves + ([hl] if hl is not None else [])
        gr = torch.autograd.grad(outs, want, cots)
    dq, dk, dv, dg, db = (x[:, :T] for x in gr[:5])
    dh0 = gr[5] if hl is not None else None
    return o.detach()[:, :T], ht.detach(), dq, dk, dv, db, dg, dh0
