"""Float64 oracle for GLA (test infrastructure only).

Restates tops/cpu/ops/gla/{chunk.py, fused_recurrent.py, naive.py, fused_chunk.py}
in fp64 mode.  Layout [B, T, H, D]; per-channel log-gates g: [B, T, H, K].

Varlen (cu_seqlens, B == 1): the reference gathers every sequence into
zero-padded chunks and restarts the state per sequence
(tops/cpu/ops/gla/chunk.py:179-221, 522-549; common/utils.py:36-85).  Zero rows
carry g = 0, so a padded chunk behaves exactly like its valid prefix; this
restatement therefore runs each sequence as its own zero-padded B=1 problem,
which is the same computation.
"""

from __future__ import annotations

import numpy as np

from .common import (F64, f64, cdiv, pad_time, chunk_local_cumsum, chunk_fwd_h,
                     chunk_bwd_dh, split_varlen)


# --------------------------------------------------------------------------
# forward sub-functions (tops/cpu/ops/gla/chunk.py:52-156)
# --------------------------------------------------------------------------

def chunk_gla_fwd_intra_gk(q, k, gc, scale, C):
    """A[b, t, h, j] for the chunk containing t (chunk.py:52-97).

    Reference point = first row of the chunk (chunk.py:83-88).  Full square;
    the caller applies the causal mask (chunk.py:245-250)."""
    B, T, H, K = q.shape
    NT = T // C
    q5 = q.reshape(B, NT, C, H, K)
    k5 = k.reshape(B, NT, C, H, K)
    g5 = gc.reshape(B, NT, C, H, K)
    gn = g5[:, :, 0:1]
    A = np.einsum("bnihk,bnjhk->bnihj", q5 * np.exp(g5 - gn), k5 * np.exp(gn - g5)) * scale
    return A.reshape(B, T, H, C)


def causal_mask_A(A, C):
    B, T, H, _ = A.shape
    A5 = A.reshape(B, T // C, C, H, C)
    m = np.tril(np.ones((C, C), bool))[None, None, :, None, :]
    return np.where(m, A5, 0.0).reshape(B, T, H, C)


def chunk_gla_fwd_o_gk(q, v, gc, A, h, scale, C):
    """o = scale * (q*exp(G)) @ h_c + tril(A) @ v  (chunk.py:100-156)."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    NT = T // C
    q5 = q.reshape(B, NT, C, H, K)
    g5 = gc.reshape(B, NT, C, H, K)
    v5 = v.reshape(B, NT, C, H, V)
    A5 = A.reshape(B, NT, C, H, C)
    o_inter = scale * np.einsum("bnchk,bnhkv->bnchv", q5 * np.exp(g5), h)
    o_intra = np.einsum("bnihj,bnjhv->bnihv", A5, v5)
    return (o_inter + o_intra).reshape(B, T, H, V)


def _fwd_dense(q, k, v, g, scale, h0, C):
    """Non-varlen forward on T % C == 0 (chunk.py:222-254)."""
    gc = chunk_local_cumsum(g, C)
    h, ht = chunk_fwd_h(k, v, gk=gc, h0=h0, C=C)
    A = causal_mask_A(chunk_gla_fwd_intra_gk(q, k, gc, scale, C), C)
    o = chunk_gla_fwd_o_gk(q, v, gc, A, h, scale, C)
    return gc, A, h, ht, o


def chunk_gla_fwd(q, k, v, g, scale, initial_state, output_final_state, chunk_size=64,
                  cu_seqlens=None):
    """Forward orchestrator (chunk.py:159-269).  Returns (o, ht)."""
    q, k, v, g, h0 = map(f64, (q, k, v, g, initial_state))
    C = chunk_size
    B, T, H, K = q.shape
    V = v.shape[-1]
    if cu_seqlens is None:
        parts = [(q, k, v, g, h0)]
    else:
        assert B == 1
        segs = [split_varlen(x, cu_seqlens) for x in (q, k, v, g)]
        parts = [(segs[0][n], segs[1][n], segs[2][n], segs[3][n],
                  None if h0 is None else h0[n:n + 1]) for n in range(len(segs[0]))]
    outs, hts = [], []
    for (qq, kk, vv, gg, hh0) in parts:
        L = qq.shape[1]
        _, _, _, ht, o = _fwd_dense(*(pad_time(x, C) for x in (qq, kk, vv, gg)), scale, hh0, C)
        outs.append(o[:, :L])
        hts.append(ht)
    o = np.concatenate(outs, axis=1)
    ht = np.concatenate(hts, axis=0) if output_final_state else None
    return o, ht


def chunk_gla(q, k, v, g=None, scale=None, initial_state=None, output_final_state=False,
              cu_seqlens=None, chunk_size=16):
    """Public oracle API (tops/cpu/ops/gla/chunk.py:649-718)."""
    q = f64(q)
    B, T, H, K = q.shape
    V = np.shape(v)[-1]
    if cu_seqlens is not None:
        assert B == 1, f"B must be 1 for varlen, got {B}"
        lens = np.diff(np.asarray(cu_seqlens))
        assert np.all(lens > 0), "Empty segments not supported"
        if initial_state is not None:
            assert np.shape(initial_state) == (len(cu_seqlens) - 1, H, K, V)
    if g is None:
        g = np.zeros_like(q)
    if scale is None:
        scale = K ** -0.5
    return chunk_gla_fwd(q, k, v, g, scale, initial_state, output_final_state,
                         chunk_size=chunk_size, cu_seqlens=cu_seqlens)


def fused_chunk_gla(q, k, v, g, scale=None, initial_state=None, output_final_state=False,
                    cu_seqlens=None, chunk_size=16):
    """tops/cpu/ops/gla/fused_chunk.py:4-44 -- delegates to chunk_gla."""
    return chunk_gla(q, k, v, g=g, scale=scale, initial_state=initial_state,
                     output_final_state=output_final_state, cu_seqlens=cu_seqlens,
                     chunk_size=chunk_size)


# --------------------------------------------------------------------------
# backward sub-functions (tops/cpu/ops/gla/chunk.py:277-466)
# --------------------------------------------------------------------------

def chunk_gla_bwd_dA(v, do, scale, C):
    """dA = scale * tril(do @ v^T) per chunk (chunk.py:277-307)."""
    B, T, H, V = v.shape
    NT = T // C
    dA = np.einsum("bnihv,bnjhv->bnihj", do.reshape(B, NT, C, H, V),
                   v.reshape(B, NT, C, H, V)) * scale
    return causal_mask_A(dA.reshape(B, T, H, C), C)


def chunk_gla_bwd_dv(k, gc, A, do, dh, C):
    """dv = A^T do + (k*exp(G_last - G)) dh (chunk.py:310-354)."""
    B, T, H, K = k.shape
    V = do.shape[-1]
    NT = T // C
    k5 = k.reshape(B, NT, C, H, K)
    g5 = gc.reshape(B, NT, C, H, K)
    dv_intra = np.einsum("bnihj,bnihv->bnjhv", A.reshape(B, NT, C, H, C),
                         do.reshape(B, NT, C, H, V))
    kd = k5 * np.exp(g5[:, :, -1:] - g5)
    dv_inter = np.einsum("bnchk,bnhkv->bnchv", kd, dh)
    return (dv_intra + dv_inter).reshape(B, T, H, V)


def chunk_gla_bwd_dqk_intra(q, k, gc, dA, C):
    """Intra-chunk dq, dk from dA (chunk.py:357-393)."""
    B, T, H, K = q.shape
    NT = T // C
    q5 = q.reshape(B, NT, C, H, K)
    k5 = k.reshape(B, NT, C, H, K)
    g5 = gc.reshape(B, NT, C, H, K)
    dA5 = dA.reshape(B, NT, C, H, C)
    dq = np.exp(g5) * np.einsum("bnihj,bnjhk->bnihk", dA5, k5 * np.exp(-g5))
    dk = np.exp(-g5) * np.einsum("bnihj,bnihk->bnjhk", dA5, q5 * np.exp(g5))
    return dq.reshape(B, T, H, K), dk.reshape(B, T, H, K)


def chunk_gla_bwd_dqkg(q, k, v, h, gc, do, dh, dq, dk, scale, C):
    """Inter-chunk dq, dk and the gate gradient (chunk.py:396-466)."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    NT = T // C
    q5 = q.reshape(B, NT, C, H, K)
    k5 = k.reshape(B, NT, C, H, K)
    v5 = v.reshape(B, NT, C, H, V)
    g5 = gc.reshape(B, NT, C, H, K)
    do5 = do.reshape(B, NT, C, H, V)
    gn = g5[:, :, -1]                                             # [B,NT,H,K]
    dq_inter = scale * np.exp(g5) * np.einsum("bnchv,bnhkv->bnchk", do5, h)
    dk_inter = np.exp(gn[:, :, None] - g5) * np.einsum("bnchv,bnhkv->bnchk", v5, dh)
    dq_t = dq.reshape(B, NT, C, H, K) + dq_inter
    dk_t = dk.reshape(B, NT, C, H, K) + dk_inter
    dgk_inter = np.exp(gn) * np.einsum("bnhkv,bnhkv->bnhk", h, dh) + np.sum(dk_inter * k5, axis=2)
    dg_raw = q5 * dq_t - k5 * dk_t
    dg = np.flip(np.cumsum(np.flip(dg_raw, 2), 2), 2) + dgk_inter[:, :, None]
    return dq_t.reshape(B, T, H, K), dk_t.reshape(B, T, H, K), dg.reshape(B, T, H, K)


def _bwd_dense(q, k, v, g, scale, h0, do, dht, C):
    """Non-varlen backward on T % C == 0 (chunk.py:551-607)."""
    gc = chunk_local_cumsum(g, C)
    h, _ = chunk_fwd_h(k, v, gk=gc, h0=h0, C=C)
    dh, dh0 = chunk_bwd_dh(q, do, gk=gc, dht=dht, scale=scale, C=C)
    A = causal_mask_A(chunk_gla_fwd_intra_gk(q, k, gc, scale, C), C)
    dv = chunk_gla_bwd_dv(k, gc, A, do, dh, C)
    dA = chunk_gla_bwd_dA(v, do, scale, C)
    dq, dk = chunk_gla_bwd_dqk_intra(q, k, gc, dA, C)
    dq, dk, dg = chunk_gla_bwd_dqkg(q, k, v, h, gc, do, dh, dq, dk, scale, C)
    return dq, dk, dv, dg, dh0


def chunk_gla_bwd(q, k, v, g, scale, initial_state, do, dht, chunk_size=64, cu_seqlens=None):
    """Backward orchestrator (chunk.py:469-640).  Returns (dq, dk, dv, dg, dh0).

    dh0 is the gradient w.r.t. the initial state (zero-state gradient when no
    h0 is given; the reference returns it whenever it is requested)."""
    q, k, v, g, h0, do, dht = map(f64, (q, k, v, g, initial_state, do, dht))
    C = chunk_size
    B = q.shape[0]
    if g is None:
        g = np.zeros_like(q)
    if cu_seqlens is None:
        parts = [(q, k, v, g, h0, do, dht)]
    else:
        assert B == 1
        segs = [split_varlen(x, cu_seqlens) for x in (q, k, v, g, do)]
        N = len(segs[0])
        parts = [(segs[0][n], segs[1][n], segs[2][n], segs[3][n],
                  None if h0 is None else h0[n:n + 1], segs[4][n],
                  None if dht is None else dht[n:n + 1]) for n in range(N)]
    res = [[], [], [], [], []]
    for (qq, kk, vv, gg, hh0, ddo, ddht) in parts:
        L = qq.shape[1]
        pq, pk, pv, pg, pdo = (pad_time(x, C) for x in (qq, kk, vv, gg, ddo))
        dq, dk, dv, dg, dh0 = _bwd_dense(pq, pk, pv, pg, scale, hh0, pdo, ddht, C)
        for lst, x in zip(res, (dq[:, :L], dk[:, :L], dv[:, :L], dg[:, :L], dh0)):
            lst.append(x)
    return tuple(np.concatenate(r, axis=0 if i == 4 else 1) for i, r in enumerate(res))


# --------------------------------------------------------------------------
# recurrent forms (tops/cpu/ops/gla/fused_recurrent.py, naive.py)
# --------------------------------------------------------------------------

def _seq_ranges(B, T, cu_seqlens):
    if cu_seqlens is None:
        return [(b, 0, T) for b in range(B)]
    cu = [int(c) for c in cu_seqlens]
    return [(0, cu[n], cu[n + 1]) for n in range(len(cu) - 1)]


def fused_recurrent_fwd(q, k, v, gk=None, gv=None, scale=None, initial_state=None,
                        output_final_state=False, reverse=False, cu_seqlens=None):
    """Per-token recurrence (tops/cpu/ops/gla/fused_recurrent.py:51-167).

    h <- h*exp(gk_t)[:,None]*exp(gv_t)[None,:] + k_t v_t^T ; o_t = scale * h^T q_t."""
    q, k, v, gk, gv, h0 = map(f64, (q, k, v, gk, gv, initial_state))
    B, T, H, K = q.shape
    V = v.shape[-1]
    if scale is None:
        scale = K ** -0.5
    o = np.zeros((B, T, H, V), F64)
    hts = []
    for n, (b, bos, eos) in enumerate(_seq_ranges(B, T, cu_seqlens)):
        h = np.zeros((H, K, V), F64) if h0 is None else h0[n].copy()
        ts = range(eos - 1, bos - 1, -1) if reverse else range(bos, eos)
        for t in ts:
            if gk is not None:
                h = h * np.exp(gk[b, t])[:, :, None]
            if gv is not None:
                h = h * np.exp(gv[b, t])[:, None, :]
            h = h + k[b, t][:, :, None] * v[b, t][:, None, :]
            o[b, t] = np.einsum("hkv,hk->hv", h, q[b, t] * scale)
        hts.append(h)
    return o, (np.stack(hts) if output_final_state else None)


def fused_recurrent_gla(q, k, v, gk=None, gv=None, scale=None, initial_state=None,
                        output_final_state=False, reverse=False, cu_seqlens=None):
    """Public API (tops/cpu/ops/gla/fused_recurrent.py:362-422)."""
    return fused_recurrent_fwd(q, k, v, gk, gv, scale, initial_state, output_final_state,
                               reverse, cu_seqlens)


def fused_recurrent_bwd(q, k, v, gk=None, gv=None, o=None, do=None, dht=None, scale=None,
                        initial_state=None, reverse=False, cu_seqlens=None):
    """Two-pass backward (tops/cpu/ops/gla/fused_recurrent.py:171-358).

    Returns (dq, dk, dv, dgk, dgv, dh0); dgk/dgv are running suffix sums
    plus the h_T*dht boundary term."""
    q, k, v, gk, gv, o, do, dht, h0 = map(f64, (q, k, v, gk, gv, o, do, dht, initial_state))
    B, T, H, K = q.shape
    V = v.shape[-1]
    if scale is None:
        scale = K ** -0.5
    dq = np.zeros((B, T, H, K), F64)
    dk = np.zeros((B, T, H, K), F64)
    dv = np.zeros((B, T, H, V), F64)
    dgk = np.zeros((B, T, H, K), F64) if gk is not None else None
    dgv = np.zeros((B, T, H, V), F64) if gv is not None else None
    dh0s = []
    for n, (b, bos, eos) in enumerate(_seq_ranges(B, T, cu_seqlens)):
        h = np.zeros((H, K, V), F64) if h0 is None else h0[n].copy()
        fwd = range(eos - 1, bos - 1, -1) if reverse else range(bos, eos)
        for t in fwd:
            if gk is not None:
                h = h * np.exp(gk[b, t])[:, :, None]
            if gv is not None:
                h = h * np.exp(gv[b, t])[:, None, :]
            h = h + k[b, t][:, :, None] * v[b, t][:, None, :]
            dq[b, t] = scale * np.einsum("hkv,hv->hk", h, do[b, t])
        dh = np.zeros((H, K, V), F64) if dht is None else dht[n].copy()
        if gk is not None:
            rk = np.sum(h * dh, axis=2)
        if gv is not None:
            rv = np.sum(h * dh, axis=1)
        bwd = range(bos, eos) if reverse else range(eos - 1, bos - 1, -1)
        for t in bwd:
            dh = dh + (q[b, t] * scale)[:, :, None] * do[b, t][:, None, :]
            dk[b, t] = np.einsum("hkv,hv->hk", dh, v[b, t])
            dv[b, t] = np.einsum("hkv,hk->hv", dh, k[b, t])
            if gk is not None:
                rk = rk + q[b, t] * dq[b, t] - k[b, t] * dk[b, t]
                dgk[b, t] = rk
                dh = dh * np.exp(gk[b, t])[:, :, None]
            if gv is not None:
                rv = rv + o[b, t] * do[b, t] - v[b, t] * dv[b, t]
                dgv[b, t] = rv
                dh = dh * np.exp(gv[b, t])[:, None, :]
        dh0s.append(dh)
    dh0 = np.stack(dh0s) if h0 is not None else None
    return dq, dk, dv, dgk, dgv, dh0


def naive_recurrent_gla(q, k, v, gk, initial_state=None, output_final_state=False):
    """tops/cpu/ops/gla/naive.py:30-105 (scale fixed to K^-0.5)."""
    q, k, v, gk, h0 = map(f64, (q, k, v, gk, initial_state))
    B, T, H, K = q.shape
    V = v.shape[-1]
    scale = K ** -0.5
    h = np.zeros((B, H, K, V), F64) if h0 is None else h0.copy()
    o = np.zeros((B, T, H, V), F64)
    for t in range(T):
        h = h * np.exp(gk[:, t])[..., None] + k[:, t][..., None] * v[:, t][..., None, :]
        o[:, t] = np.einsum("bhkv,bhk->bhv", h, q[:, t] * scale)
    return o, (h if output_final_state else None)
