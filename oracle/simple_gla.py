"""Float64 oracle for simple GLA (test infrastructure only).

Restates tops/cpu/ops/simple_gla/{chunk.py, naive.py} in fp64 mode.  Layout
[B, T, H, D]; the gate is one log-value per (token, head): g [B, T, H], or a
constant per-head log-decay g_gamma [H].  The chunked form gates v inside the state
update (tops/cpu/ops/common/chunk_h.py:127-135, 192-197) and multiplies the
output terms by exp(G) (tops/cpu/ops/common/chunk_o.py:186-208).

Varlen (cu_seqlens, B == 1) runs every sequence as its own zero-padded B = 1
problem (tops/cpu/ops/simple_gla/chunk.py handles varlen per sequence and per chunk,
with read_chunk zero padding: the same computation).
"""

from __future__ import annotations

import numpy as np

from .common import F64, f64, pad_time, split_varlen


def _gates(B, T, H, g, g_gamma, valid_T):
    """Chunk-local inputs of the gate: per-token log-gates g_tok [B, T, H] (zero past
    valid_T), following the g / g_gamma branches of tops/cpu/ops/common/chunk_h.py:139-160
    (g_gamma: G_i = gamma * (i + 1) inside the chunk, Gamma = gamma * chunk_len)."""
    assert not (g is not None and g_gamma is not None), \
        "only one of g or g_gamma (tops/cpu/ops/simple_gla/chunk.py:724-728)"
    if g is not None:
        return f64(g)
    gt = np.zeros((B, T, H), F64)
    if g_gamma is not None:
        gt[:, :valid_T] = f64(g_gamma)[None, None, :]
    return gt


def _cumsum_chunks(gt, C):
    B, T, H = gt.shape
    return np.cumsum(gt.reshape(B, T // C, C, H), axis=2).reshape(B, T, H)


def _fwd_dense(q, k, v, gt, scale, h0, C):
    """Forward on T % C == 0 (tops/cpu/ops/simple_gla/chunk.py:53-129 with
    chunk_fwd_h common/chunk_h.py:179-226 and chunk_fwd_o common/chunk_o.py:115-259)."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    NT = T // C
    G = _cumsum_chunks(gt, C).reshape(B, NT, C, H)
    q5, k5, v5 = (x.reshape(B, NT, C, H, -1) for x in (q, k, v))
    h = np.zeros((B, H, K, V), F64) if h0 is None else f64(h0).copy()
    hs = np.empty((B, NT, H, K, V), F64)
    o = np.empty((B, NT, C, H, V), F64)
    mask = np.tril(np.ones((C, C), bool))
    for i in range(NT):
        hs[:, i] = h
        Gc = G[:, i]                                            # [B, C, H]
        Gl = Gc[:, -1]                                          # [B, H]
        # output: scale * [(q h) e^G + tril(q k^T e^(G_i - G_j)) v]
        o_inter = np.einsum("bchk,bhkv->bchv", q5[:, i], h) * np.exp(Gc)[..., None]
        qk = np.einsum("bihk,bjhk->bhij", q5[:, i], k5[:, i])
        dec = np.exp(np.transpose(Gc, (0, 2, 1))[:, :, :, None]
                     - np.transpose(Gc, (0, 2, 1))[:, :, None, :])
        A = np.where(mask, qk * dec, 0.0)
        o_intra = np.einsum("bhij,bjhv->bihv", A, v5[:, i])
        o[:, i] = scale * (o_inter + o_intra)
        # state: h * e^Gamma + k^T (v e^(Gamma - G))
        vd = v5[:, i] * np.exp(Gl[:, None, :] - Gc)[..., None]
        h = h * np.exp(Gl)[:, :, None, None] + np.einsum("bchk,bchv->bhkv", k5[:, i], vd)
    return o.reshape(B, T, H, V), hs, h


def chunk_simple_gla_fwd(q, k, v, g, g_gamma, scale, initial_state, output_final_state,
                         chunk_size=64, cu_seqlens=None):
    """tops/cpu/ops/simple_gla/chunk.py:53-129.  Returns (o, ht)."""
    q, k, v, h0 = map(f64, (q, k, v, initial_state))
    C = chunk_size
    B, T, H, K = q.shape
    if cu_seqlens is None:
        parts = [(q, k, v, None if g is None else f64(g), h0)]
    else:
        assert B == 1
        segs = [split_varlen(x, cu_seqlens) for x in (q, k, v)]
        gsegs = split_varlen(f64(g), cu_seqlens) if g is not None else [None] * len(segs[0])
        parts = [(segs[0][n], segs[1][n], segs[2][n], gsegs[n],
                  None if h0 is None else h0[n:n + 1]) for n in range(len(segs[0]))]
    outs, hts = [], []
    for (qq, kk, vv, gg, hh0) in parts:
        L = qq.shape[1]
        pq, pk, pv = (pad_time(x, C) for x in (qq, kk, vv))
        gt = _gates(1 if cu_seqlens is not None else B, pq.shape[1], H,
                    None if gg is None else pad_time(gg, C), g_gamma, L)
        o, _, ht = _fwd_dense(pq, pk, pv, gt, scale, hh0, C)
        outs.append(o[:, :L])
        hts.append(ht)
    o = np.concatenate(outs, axis=1)
    ht = np.concatenate(hts, axis=0) if output_final_state else None
    return o, ht


def chunk_simple_gla(q, k, v, g=None, g_gamma=None, scale=None, initial_state=None,
                     output_final_state=False, cu_seqlens=None, chunk_size=64):
    """Public oracle API (tops/cpu/ops/simple_gla/chunk.py:796-889)."""
    K = np.shape(q)[-1]
    if scale is None:
        scale = K ** -0.5
    return chunk_simple_gla_fwd(q, k, v, g, g_gamma, scale, initial_state, output_final_state,
                                chunk_size, cu_seqlens)


def _bwd_dense(q, k, v, gt, scale, h0, do, dht, C):
    """Backward on T % C == 0: chunk_bwd_dh (common/chunk_h.py:387-427), chunk_bwd_dqkwg
    (simple_gla/chunk.py:137-468), chunk_bwd_dv (:476-661), reverse cumsum of dg
    (:777-778).  Returns dq, dk, dv, dg (per token, before nothing else), dh0."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    NT = T // C
    _, hs, _ = _fwd_dense(q, k, v, gt, scale, h0, C)
    G = _cumsum_chunks(gt, C).reshape(B, NT, C, H)
    q5, k5, v5, do5 = (x.reshape(B, NT, C, H, -1) for x in (q, k, v, do))
    mask = np.tril(np.ones((C, C), bool))
    # reverse state-gradient recurrence: dhs[:, i] = dL/d(state after chunk i)
    dh = np.zeros((B, H, K, V), F64) if dht is None else f64(dht).copy()
    dhs = np.empty((B, NT, H, K, V), F64)
    for i in range(NT - 1, -1, -1):
        dhs[:, i] = dh
        Gc = G[:, i]
        qg = q5[:, i] * np.exp(Gc)[..., None] * scale
        dh = dh * np.exp(Gc[:, -1])[:, :, None, None] + np.einsum("bchk,bchv->bhkv", qg, do5[:, i])
    dh0 = dh
    dq = np.empty_like(q5)
    dk = np.empty_like(k5)
    dv = np.empty_like(v5)
    dg = np.empty((B, NT, C, H), F64)
    for i in range(NT):
        Gc = G[:, i]                                            # [B, C, H]
        Gl = Gc[:, -1]                                          # [B, H]
        h, dhc = hs[:, i], dhs[:, i]
        bq, bk, bv, bdo = q5[:, i], k5[:, i], v5[:, i], do5[:, i]
        GT = np.transpose(Gc, (0, 2, 1))                        # [B, H, C]
        dec = np.where(mask, np.exp(GT[:, :, :, None] - GT[:, :, None, :]), 0.0)  # [B,H,i,j]
        # dq, dk, dg (chunk_bwd_dqkwg, USE_G branch)
        ds = np.einsum("bihv,bjhv->bhij", bdo, bv) * dec * scale
        dq_i = np.einsum("bchv,bhkv->bchk", bdo, h) * np.exp(Gc)[..., None] * scale
        dk_i = np.einsum("bchv,bhkv->bchk", bv, dhc) * np.exp(Gl[:, None, :] - Gc)[..., None]
        dg_last = np.sum(h * dhc, axis=(-2, -1)) * np.exp(Gl) + np.sum(dk_i * bk, axis=(1, 3))
        dgc = np.sum(dq_i * bq, axis=-1) - np.sum(bk * dk_i, axis=-1)
        qk = np.einsum("bihk,bjhk->bhij", bq, bk)
        ds2 = ds * qk
        dgc = dgc + np.transpose(np.sum(ds2, axis=-1), (0, 2, 1)) \
            - np.transpose(np.sum(ds2, axis=-2), (0, 2, 1))
        dq[:, i] = dq_i + np.einsum("bhij,bjhk->bihk", ds, bk)
        dk[:, i] = dk_i + np.einsum("bhij,bihk->bjhk", ds, bq)
        dgc[:, -1] += dg_last
        dg[:, i] = dgc
        # dv (chunk_bwd_dv): A^T do + (k e^(Gamma - G)) dh
        A = np.einsum("bihk,bjhk->bhij", bq, bk) * dec * scale
        dv[:, i] = np.einsum("bhij,bihv->bjhv", A, bdo) + np.einsum(
            "bchk,bhkv->bchv", bk * np.exp(Gl[:, None, :] - Gc)[..., None], dhc)
    dg = np.flip(np.cumsum(np.flip(dg, 2), 2), 2)               # reverse cumsum per chunk
    return (dq.reshape(B, T, H, K), dk.reshape(B, T, H, K), dv.reshape(B, T, H, V),
            dg.reshape(B, T, H), dh0)


def chunk_simple_gla_bwd(q, k, v, g, g_gamma, initial_state, do, dht, scale, chunk_size=64,
                         cu_seqlens=None):
    """tops/cpu/ops/simple_gla/chunk.py:668-788.  Returns (dq, dk, dv, dg, dh0); dg is
    None unless g is given."""
    q, k, v, h0, do, dht = map(f64, (q, k, v, initial_state, do, dht))
    C = chunk_size
    B, T, H, K = q.shape
    if cu_seqlens is None:
        parts = [(q, k, v, None if g is None else f64(g), h0, do, dht)]
    else:
        assert B == 1
        segs = [split_varlen(x, cu_seqlens) for x in (q, k, v, do)]
        gsegs = split_varlen(f64(g), cu_seqlens) if g is not None else [None] * len(segs[0])
        parts = [(segs[0][n], segs[1][n], segs[2][n], gsegs[n],
                  None if h0 is None else h0[n:n + 1], segs[3][n],
                  None if dht is None else dht[n:n + 1]) for n in range(len(segs[0]))]
    res = [[], [], [], [], []]
    for (qq, kk, vv, gg, hh0, ddo, ddht) in parts:
        L = qq.shape[1]
        pq, pk, pv, pdo = (pad_time(x, C) for x in (qq, kk, vv, ddo))
        gt = _gates(pq.shape[0], pq.shape[1], H, None if gg is None else pad_time(gg, C),
                    g_gamma, L)
        dq, dk, dv, dg, dh0 = _bwd_dense(pq, pk, pv, gt, scale, hh0, pdo, ddht, C)
        for lst, x in zip(res, (dq[:, :L], dk[:, :L], dv[:, :L], dg[:, :L], dh0)):
            lst.append(x)
    out = [np.concatenate(r, axis=0 if i == 4 else 1) for i, r in enumerate(res)]
    if g is None:
        out[3] = None
    return tuple(out)


def naive_simple_gla(q, k, v, g=None, g_gamma=None, scale=None, initial_state=None,
                     output_final_state=False, cu_seqlens=None):
    """Per-token recurrence (tops/cpu/ops/simple_gla/naive.py:30-160):
    h_t = h_{t-1} exp(g_t [+ g_gamma]) + k_t v_t^T ; o_t = (scale q_t)^T h_t."""
    q, k, v, h0 = map(f64, (q, k, v, initial_state))
    B, T, H, K = q.shape
    V = v.shape[-1]
    if scale is None:
        scale = K ** -0.5
    lg = np.zeros((B, T, H), F64)
    if g is not None:
        lg = lg + f64(g)
    if g_gamma is not None:
        lg = lg + f64(g_gamma)[None, None, :]
    ranges = [(b, 0, T) for b in range(B)] if cu_seqlens is None else \
        [(0, int(cu_seqlens[n]), int(cu_seqlens[n + 1])) for n in range(len(cu_seqlens) - 1)]
    o = np.zeros((B, T, H, V), F64)
    hts = []
    for n, (b, bos, eos) in enumerate(ranges):
        h = np.zeros((H, K, V), F64) if h0 is None else h0[n].copy()
        for t in range(bos, eos):
            h = h * np.exp(lg[b, t])[:, None, None] + k[b, t][:, :, None] * v[b, t][:, None, :]
            o[b, t] = np.einsum("hkv,hk->hv", h, q[b, t] * scale)
        hts.append(h)
    return o, (np.stack(hts) if output_final_state else None)


def chunk_bwd_dqkwg_raw_dg(q, k, v, h, do, dh, g_cumsum, scale, C):
    """The raw per-position gate gradient of tops/ops/common/chunk_o.py:780-835 (per-token g):
    sum over channels of q dq_gate - k dk_gate, plus the row sums minus the column sums of
    ds2 = causal(do v^T e^{g_i - g_j}) scale * (q k^T), and the chunk-end term
    e^{g_last} sum(h dh) + sum(dk_gate k) added at each chunk's last position; not
    reverse-cumsummed.  g_cumsum [B,T,H]; h, dh [B,NT,H,K,V]."""
    q, k, v, h, do, dh, g = map(f64, (q, k, v, h, do, dh, g_cumsum))
    B, T, H, K = q.shape
    V = v.shape[-1]
    NT = T // C
    qc, kc = (x.reshape(B, NT, C, H, K) for x in (q, k))
    vc, dc = (x.reshape(B, NT, C, H, V) for x in (v, do))
    gc = g.reshape(B, NT, C, H)
    gl = gc[:, :, -1]                                              # [B,NT,H]
    dq_gate = np.einsum("bnchv,bnhkv->bnchk", dc, h) * np.exp(gc)[..., None] * scale
    dk_gate = np.einsum("bnchv,bnhkv->bnchk", vc, dh) * np.exp(gl[:, :, None] - gc)[..., None]
    last = np.exp(gl) * np.einsum("bnhkv,bnhkv->bnh", h, dh) + np.einsum("bnchk,bnchk->bnh", dk_gate, kc)
    m = np.tril(np.ones((C, C), bool))[None, None, :, :, None]
    ds = np.einsum("bnihv,bnjhv->bnijh", dc, vc) * np.exp(gc[:, :, :, None] - gc[:, :, None, :])
    ds2 = np.where(m, ds, 0.0) * scale * np.einsum("bnihk,bnjhk->bnijh", qc, kc)
    raw = (np.sum(dq_gate * qc, -1) - np.sum(kc * dk_gate, -1)
           + ds2.sum(axis=3) - ds2.sum(axis=2))
    raw[:, :, -1] += last
    return raw.reshape(B, T, H)
