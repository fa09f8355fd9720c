"""Float64 oracle for KDA, the gated delta rule with per-channel gates (test infrastructure
only).

Restates tops/cpu/ops/kda/naive.py (naive_recurrent_kda :10-118, naive_chunk_kda
:121-313) and the chunked forward / backward of tops/cpu/ops/kda/chunk_bwd.py:525-668
(stages: recompute w, u, h, v_new; dAv; the reverse state-gradient pass dhu; the WY /
dqkg and intra backward; the reverse gate cumsum), with every intermediate exposed so
the HIP kernels can be checked stage by stage.  Per head, natural-log gates:

    S' = S_{t-1} * exp(g_t)[:, None]
    S_t = S' + beta_t k_t (v_t - S'^T k_t)^T
    o_t = S_t^T (scale q_t)

Chunked (chunk c, Gn = in-chunk inclusive cumsum of g, Gam = Gn[last], S_c the state
before the chunk):
    Akk_ij = beta_i sum_d k_id k_jd exp(Gn_id - Gn_jd)  (i > j),  T = (I + Akk)^-1
    u = T (beta v),  w = T (beta exp(Gn) k),  v_new = u - w S_c
    Aqk_ij = sum_d (scale q_id) k_jd exp(Gn_id - Gn_jd)  (j <= i)
    o = (scale q exp(Gn)) S_c + Aqk v_new
    S_{c+1} = exp(Gam) S_c + (k exp(Gam - Gn))^T v_new
The reference keeps the gates in log2 units (tops/ops/kda/gate.py:42-51) and divides dg
by ln 2 at the end (tops/ops/kda/chunk.py:245-248); natural-log units give the same
numbers without the two conversions.
"""

from __future__ import annotations

import numpy as np

from .common import F64, f64, pad_time


def naive_recurrent_kda(q, k, v, g, beta, scale=None, initial_state=None,
                        output_final_state=False):
    """tops/cpu/ops/kda/naive.py:10-118."""
    q, k, v, g, beta, h0 = map(f64, (q, k, v, g, beta, initial_state))
    B, T, H, K = q.shape
    V = v.shape[-1]
    if scale is None:
        scale = K ** -0.5
    S = np.zeros((B, H, K, V), F64) if h0 is None else h0.copy()
    o = np.zeros((B, T, H, V), F64)
    for t in range(T):
        S = S * np.exp(g[:, t])[..., None]
        pred = np.einsum("bhk,bhkv->bhv", k[:, t], S)
        S = S + np.einsum("bhk,bhv->bhkv", beta[:, t][..., None] * k[:, t], v[:, t] - pred)
        o[:, t] = np.einsum("bhk,bhkv->bhv", q[:, t] * scale, S)
    return o, (S if output_final_state else None)


def _chunks(x, C):
    B, T, H = x.shape[:3]
    return x.reshape(B, T // C, C, H, *x.shape[3:])


def chunk_kda_fwd_parts(q, k, v, g, beta, scale, initial_state, C=64):
    """Chunked forward with every intermediate (T % C == 0): the naive chunk form of
    tops/cpu/ops/kda/naive.py:121-313 (same algebra; Akk inverted exactly).
    Returns a dict of [B, NT, C, H, ...] arrays plus S (state before each chunk,
    [B, NT, H, K, V]), ht and o [B, T, H, V]."""
    q, k, v, g, beta, h0 = map(f64, (q, k, v, g, beta, initial_state))
    B, T, H, K = q.shape
    V = v.shape[-1]
    NT = T // C
    qc, kc, vc, gc, bc = (_chunks(x, C) for x in (q, k, v, g, beta))
    Gn = np.cumsum(gc, axis=2)                                   # [B,NT,C,H,K]
    E = np.exp(Gn[:, :, :, None] - Gn[:, :, None, :])            # [B,NT,i,j,H,K]
    lower = np.tril(np.ones((C, C), bool), -1)[None, None, :, :, None]
    causal = np.tril(np.ones((C, C), bool))[None, None, :, :, None]
    Akk = np.where(lower, np.einsum("bnihd,bnjhd,bnijhd->bnijh", kc, kc, E), 0.0) \
        * bc[:, :, :, None, :]                                   # [B,NT,i,j,H]
    I = np.eye(C)[None, None, :, :, None]
    Tm = np.moveaxis(np.linalg.inv(np.moveaxis(I + Akk, 4, 2)), 2, 4)   # (I + Akk)^-1
    bv = bc[..., None] * vc
    bk = bc[..., None] * np.exp(Gn) * kc
    u = np.einsum("bnijh,bnjhv->bnihv", Tm, bv)
    w = np.einsum("bnijh,bnjhk->bnihk", Tm, bk)
    Aqk = np.where(causal, np.einsum("bnihd,bnjhd,bnijhd->bnijh", qc * scale, kc, E), 0.0)
    S = np.zeros((B, H, K, V), F64) if h0 is None else h0.copy()
    Ss = np.empty((B, NT, H, K, V), F64)
    vnew = np.empty_like(vc)
    o = np.empty_like(vc)
    for n in range(NT):
        Ss[:, n] = S
        vn = u[:, n] - np.einsum("bihk,bhkv->bihv", w[:, n], S)
        vnew[:, n] = vn
        o[:, n] = np.einsum("bihk,bhkv->bihv", qc[:, n] * scale * np.exp(Gn[:, n]), S) \
            + np.einsum("bijh,bjhv->bihv", Aqk[:, n], vn)
        Gl = Gn[:, n, -1]                                        # [B,H,K]
        S = S * np.exp(Gl)[..., None] + np.einsum(
            "bjhk,bjhv->bhkv", kc[:, n] * np.exp(Gl[:, None] - Gn[:, n]), vn)
    return dict(Gn=Gn, Akk=Akk, T=Tm, u=u, w=w, Aqk=Aqk, S=Ss, v_new=vnew, ht=S,
                o=o.reshape(B, T, H, V))


def chunk_kda(q, k, v, g, beta, scale=None, initial_state=None, output_final_state=False,
              chunk_size=64):
    """Public oracle (tops/ops/kda/chunk.py:193-217 semantics): ragged T is zero-padded,
    which is exact (a padded token has k = 0, g = 0)."""
    q = f64(q)
    T = q.shape[1]
    K = q.shape[-1]
    if scale is None:
        scale = K ** -0.5
    C = chunk_size
    pq, pk, pv, pg, pb = (pad_time(f64(x), C) for x in (q, k, v, g, beta))
    P = chunk_kda_fwd_parts(pq, pk, pv, pg, pb, scale, initial_state, C)
    return P["o"][:, :T], (P["ht"] if output_final_state else None)


def chunk_kda_bwd(q, k, v, g, beta, scale, initial_state, do, dht, chunk_size=64,
                  return_parts=False):
    """Chunked backward (tops/cpu/ops/kda/chunk_bwd.py:525-668, restated).

    Per chunk c (last to first), with dS the gradient w.r.t. S_{c+1}:
      dv_new = Aqk^T dO + (k exp(Gam - Gn)) dS                       (dAv + dhu)
      dS_c   = exp(Gam) dS + (scale q exp(Gn))^T dO - w^T dv_new       (dhu)
    then the GLA-shaped terms of o and the state update (with v := v_new, h := S_c) and the
    WY terms (du = dv_new, dw = -dv_new S_c^T, through T, Akk, beta v, beta exp(Gn) k):
      dAkk = -(T^T (du (beta v)^T + dw (beta exp(Gn) k)^T) T^T), strictly lower.
    dg is the gradient w.r.t. the natural-log gate: the reverse in-chunk cumsum of the
    gradient w.r.t. Gn.  Returns (dq, dk, dv, dbeta, dg, dh0) [+ parts]."""
    q0 = f64(q)
    B, T, H, K = q0.shape
    C = chunk_size
    pq, pk, pv, pg, pb, pdo = (pad_time(f64(x), C) for x in (q, k, v, g, beta, do))
    Tp = pq.shape[1]
    V = pv.shape[-1]
    NT = Tp // C
    P = chunk_kda_fwd_parts(pq, pk, pv, pg, pb, scale, initial_state, C)
    Gn, Tm, u, w, Aqk, Ss, vnew = (P[x] for x in ("Gn", "T", "u", "w", "Aqk", "S", "v_new"))
    qc, kc, vc, bc, doc = (_chunks(x, C) for x in (pq, pk, pv, pb, pdo))
    E = np.exp(Gn[:, :, :, None] - Gn[:, :, None, :])
    lower = np.tril(np.ones((C, C), bool), -1)[None, :, :, None]
    causal = np.tril(np.ones((C, C), bool))[None, :, :, None]
    # ---- reverse state-gradient pass
    dS = np.zeros((B, H, K, V), F64) if dht is None else f64(dht).copy()
    dSs = np.empty_like(Ss)
    dvn = np.empty_like(vc)
    for n in range(NT - 1, -1, -1):
        dSs[:, n] = dS
        Gl = Gn[:, n, -1]
        kd = kc[:, n] * np.exp(Gl[:, None] - Gn[:, n])
        dv_n = np.einsum("bijh,bihv->bjhv", Aqk[:, n], doc[:, n]) + np.einsum("bjhk,bhkv->bjhv", kd, dS)
        dvn[:, n] = dv_n
        qg = qc[:, n] * scale * np.exp(Gn[:, n])
        dS = dS * np.exp(Gl)[..., None] + np.einsum("bihk,bihv->bhkv", qg, doc[:, n]) \
            - np.einsum("bihk,bihv->bhkv", w[:, n], dv_n)
    dh0 = dS
    dq = np.empty_like(qc)
    dk = np.empty_like(kc)
    dv = np.empty_like(vc)
    dbeta = np.empty_like(bc)
    dGn = np.empty_like(Gn)
    for n in range(NT):
        Gc, Gl = Gn[:, n], Gn[:, n, -1]
        qs = qc[:, n] * scale
        kk, vn, S, dSn, dvn_n, bb = kc[:, n], vnew[:, n], Ss[:, n], dSs[:, n], dvn[:, n], bc[:, n]
        En = E[:, n]                                             # [B,i,j,H,K]
        # --- GLA-shaped part (o and the state update, v := v_new)
        dA = np.where(causal, np.einsum("bihv,bjhv->bijh", doc[:, n], vn), 0.0)
        eG = np.exp(Gc)
        dq_n = eG * np.einsum("bihv,bhkv->bihk", doc[:, n], S) * scale \
            + np.einsum("bijh,bjhk,bijhk->bihk", dA, kk, En) * scale
        dk_n = np.einsum("bijh,bihk,bijhk->bjhk", dA, qs, En)
        kint = np.exp(Gl[:, None] - Gc) * np.einsum("bjhv,bhkv->bjhk", vn, dSn)
        dk_n = dk_n + kint
        dG = qs * (eG * np.einsum("bihv,bhkv->bihk", doc[:, n], S)) \
            + np.einsum("bijh,bihk,bjhk,bijhk->bihk", dA, qs, kk, En) \
            - np.einsum("bijh,bihk,bjhk,bijhk->bjhk", dA, qs, kk, En) \
            - kk * kint
        dGl = np.exp(Gl) * np.einsum("bhkv,bhkv->bhk", S, dSn) + np.sum(kk * kint, axis=1)
        # --- WY part
        bv = bb[..., None] * vc[:, n]
        bk = bb[..., None] * eG * kk
        Tn = Tm[:, n]                                            # [B,i,j,H]
        du = dvn_n
        dw = -np.einsum("bihv,bhkv->bihk", dvn_n, S)
        dbv = np.einsum("bijh,bihv->bjhv", Tn, du)
        dbk = np.einsum("bijh,bihk->bjhk", Tn, dw)
        dT = np.einsum("bihv,bjhv->bijh", du, bv) + np.einsum("bihk,bjhk->bijh", dw, bk)
        dAkk = -np.einsum("bmih,bmnh,bjnh->bijh", Tn, dT, Tn)    # -T^T dT T^T
        dAkk = np.where(lower, dAkk, 0.0)
        dv[:, n] = bb[..., None] * dbv
        db = np.sum(vc[:, n] * dbv, axis=-1) + np.sum(eG * kk * dbk, axis=-1)
        dk_n = dk_n + bb[..., None] * eG * dbk
        dG = dG + bk * dbk
        Pm = bb[:, :, None, :] * dAkk                            # beta_i dAkk_ij
        dk_n = dk_n + np.einsum("bijh,bjhk,bijhk->bihk", Pm, kk, En) \
            + np.einsum("bijh,bihk,bijhk->bjhk", Pm, kk, En)
        t3 = np.einsum("bijh,bihk,bjhk,bijhk->bijhk", Pm, kk, kk, En)
        dG = dG + np.sum(t3, axis=2) - np.sum(t3, axis=1)
        db = db + np.einsum("bijh,bihk,bjhk,bijhk->bih", dAkk, kk, kk, En)
        dq[:, n] = dq_n
        dk[:, n] = dk_n
        dbeta[:, n] = db
        dG[:, -1] = dG[:, -1] + dGl
        dGn[:, n] = dG
    dg = np.flip(np.cumsum(np.flip(dGn, 2), 2), 2)
    out = [x.reshape(B, Tp, H, -1)[:, :T] for x in (dq, dk, dv)]
    out += [dbeta.reshape(B, Tp, H)[:, :T], dg.reshape(B, Tp, H, K)[:, :T], dh0]
    if return_parts:
        P.update(dS=dSs, dv_new=dvn)
        return tuple(out), P
    return tuple(out)


def chunk_kda_bwd_intra(q, k, g, beta, dAqk, dAkk, C=64):
    """Intra-chunk backward through Aqk and Akk (tops/ops/kda/chunk_intra.py:283-386 and
    :477-574; tops/cpu/ops/kda/chunk_intra.py:16-200).  g is the chunk-local cumsum in log2
    units, Aqk_ij = sum_d q_id k_jd 2^(g_id - g_jd), Akk_ij = beta_i sum_d k_id k_jd
    2^(g_id - g_jd); both upstream gradients are used on i >= j (the accelerator kernel's
    mask).  Returns the intra parts (dq, dk, db, dg); dg is taken w.r.t. g as if the
    exponentials were natural (no ln 2 factor), as the reference does."""
    q, k, g, beta, dAqk, dAkk = map(f64, (q, k, g, beta, dAqk, dAkk))
    B, T, H, K = q.shape
    NT = T // C
    qc, kc, gc = (x.reshape(B, NT, C, H, K) for x in (q, k, g))
    bc = beta.reshape(B, NT, C, H)
    m = np.tril(np.ones((C, C), bool))[None, None, :, None, :]
    aq = np.where(m, dAqk.reshape(B, NT, C, H, C), 0.0)
    ak = np.where(m, dAkk.reshape(B, NT, C, H, C), 0.0)
    E = np.exp2(gc[:, :, :, None] - gc[:, :, None, :])            # [B,NT,i,j,H,K]
    dq = np.einsum("bnihj,bnjhk,bnijhk->bnihk", aq, kc, E)
    row = np.einsum("bnihj,bnjhk,bnijhk->bnihk", ak, kc, E)
    db = np.sum(row * kc, axis=-1)
    dkrow = bc[..., None] * row
    dkcol = np.einsum("bnihj,bnihk,bnijhk->bnjhk", aq, qc, E) \
        + np.einsum("bnihj,bnih,bnihk,bnijhk->bnjhk", ak, bc, kc, E)
    dg = qc * dq + kc * dkrow - kc * dkcol
    return (dq.reshape(B, T, H, K), (dkrow + dkcol).reshape(B, T, H, K), db.reshape(B, T, H),
            dg.reshape(B, T, H, K))


def kda_intra_chunk_fwd(q, k, g, beta, v, segment_ids=None, scale=1.0, chunk_size=128):
    """tops/ops/kda/chunk_intra.py:91-166 (kernel) and :169-281 (wrapper).  Head-first
    [B, H, T, .] inputs, g the chunk-local gate cumsum in log2 units, segment_ids [B, T] (None:
    one segment).  Per chunk (i, j rows; masks also require equal segment ids):
        Aqk[i][j] = scale sum_d q_id k_jd 2^(g_id - g_jd)    (j <= i)
        Akk[i][j] = beta_i sum_d k_id k_jd 2^(g_id - g_jd)   (j < i)
        [u | w | Akk_inv] solves (I + Akk) X = [beta v | beta k 2^g | I] by forward
        substitution (the reference's solve_unit_lower_triangular, :28-88)
        qg = q 2^g,  kg = k 2^(g_last - g)
    Returns (u [B,H,T,V], w, qg, kg [B,H,T,K], Aqk, Akk_inv [B,H,NC,C,C])."""
    q, k, g, beta, v = map(f64, (q, k, g, beta, v))
    B, H, T, K = k.shape
    V = v.shape[-1]
    C = chunk_size
    NC = T // C
    seg = np.zeros((B, T), np.int64) if segment_ids is None else np.asarray(segment_ids)
    qc, kc, gc, vc = (x.reshape(B, H, NC, C, -1) for x in (q, k, g, v))
    bc = beta.reshape(B, H, NC, C)
    sc = seg.reshape(B, 1, NC, C)
    same = sc[..., :, None] == sc[..., None, :]                     # [B,1,NC,C,C]
    i = np.arange(C)
    lower_qk = i[:, None] >= i[None, :]
    lower = i[:, None] > i[None, :]
    gd = np.where(lower_qk[..., None], gc[..., :, None, :] - gc[..., None, :, :], 0.0)
    E = np.exp2(gd)                                                  # [B,H,NC,C,C,K]
    Aqk = np.where(lower_qk & same, scale * np.einsum("...id,...jd,...ijd->...ij", qc, kc, E), 0.0)
    Akk = np.where(lower & same, bc[..., :, None] * np.einsum("...id,...jd,...ijd->...ij", kc, kc, E),
                   0.0)
    rhs = np.concatenate([vc * bc[..., None], kc * np.exp2(gc) * bc[..., None],
                          np.broadcast_to(np.eye(C), (B, H, NC, C, C))], axis=-1)
    X = np.empty_like(rhs)
    for r in range(C):
        X[..., r, :] = rhs[..., r, :] - np.einsum("...j,...jc->...c", Akk[..., r, :r], X[..., :r, :])
    u = X[..., :V].reshape(B, H, T, V)
    w = X[..., V:V + K].reshape(B, H, T, K)
    Akk_inv = X[..., V + K:]
    qg = (qc * np.exp2(gc)).reshape(B, H, T, K)
    kg = (kc * np.exp2(gc[..., -1:, :] - gc)).reshape(B, H, T, K)
    return u, w, qg, kg, Aqk, Akk_inv


def _delta_h_seq(k, w, u, g, gk, S, C):
    """One sequence [L, H, .] of the delta-rule state pass; returns (h [NT, H, K, V], v_new, S)."""
    L = k.shape[0]
    NT = -(-L // C)
    hs = np.empty((NT,) + S.shape, F64)
    vn_all = np.empty_like(u)
    for c in range(NT):
        t0, t1 = c * C, min(L, (c + 1) * C)
        hs[c] = S
        vn = u[t0:t1] - np.einsum("thk,hkv->thv", w[t0:t1], S)
        vn_all[t0:t1] = vn
        if g is not None:
            gl = g[t1 - 1]                                              # [H]
            S = S * np.exp2(gl)[:, None, None]
            vn = vn * np.exp2(gl[None] - g[t0:t1])[..., None]
        if gk is not None:
            S = S * np.exp2(gk[t1 - 1])[..., None]
        S = S + np.einsum("thk,thv->hkv", k[t0:t1], vn)
    return hs, vn_all, S


def chunk_gated_delta_rule_fwd_h(k, w, u, g=None, gk=None, initial_state=None,
                                 output_final_state=False, chunk_size=64, save_new_value=True,
                                 use_exp2=True, cu_seqlens=None):
    """tops/cpu/ops/common/chunk_delta_h.py:22-118 (per chunk: h = S; v_new = u - w S;
    S *= 2^gk_last; S += k^T v_new, k already gated) with the scalar gate of
    tops/ops/common/chunk_delta_h.py:44-166 (S *= 2^g_last; the update uses
    v_new 2^(g_last - g), the returned v_new is ungated), and the varlen form of
    :388-560 (chunks per sequence, a short last chunk gated at its last token).  Gates are
    chunk-local cumsums, log2 units (natural with use_exp2=False).  Returns
    (h [B, NT, H, K, V], v_new [B, T, H, V] or None, ht [N, H, K, V] or None)."""
    k, w, u = f64(k), f64(w), f64(u)
    f = 1.0 if use_exp2 else 1.0 / np.log(2.0)
    g = None if g is None else f64(g) * f
    gk = None if gk is None else f64(gk) * f
    B, T, H, K = k.shape
    V = u.shape[-1]
    C = chunk_size
    if cu_seqlens is None:
        bounds = [(b, 0, T) for b in range(B)]
    else:
        cu = [int(x) for x in cu_seqlens]
        bounds = [(0, cu[n], cu[n + 1]) for n in range(len(cu) - 1)]
    N = len(bounds)
    h0 = None if initial_state is None else f64(initial_state)
    hs_all, vn = [], np.zeros((B, T, H, V), F64)
    ht = np.empty((N, H, K, V), F64)
    hb = [[] for _ in range(B)]
    for n, (b, s0, s1) in enumerate(bounds):
        S = np.zeros((H, K, V), F64) if h0 is None else h0[n].copy()
        hs, vseq, S = _delta_h_seq(k[b, s0:s1], w[b, s0:s1], u[b, s0:s1],
                                   None if g is None else g[b, s0:s1],
                                   None if gk is None else gk[b, s0:s1], S, C)
        hb[b].append(hs)
        vn[b, s0:s1] = vseq
        ht[n] = S
    h = np.stack([np.concatenate(x, axis=0) for x in hb], axis=0)
    return h, (vn if save_new_value else None), (ht if output_final_state else None)
