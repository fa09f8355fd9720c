"""Pins of the oracle pieces behind the GLA stage functions (CPU only).

chunk_local_cumsum_segments is checked against a brute-force double loop (each output the
explicit sum over its chunk up to / from that row), for forward and reverse, head_first,
ragged T and varlen boundaries; chunk_fwd_h / chunk_bwd_dh with the scalar gate against
the same recurrences with that gate broadcast over K as a per-channel gate (an identity
of the algebra), and the g_gamma ramp against an explicit scalar-gate cumsum.
"""
import numpy as np
import pytest

from oracle import common as OC


def _brute(g, C, reverse, cu, head_first, scale):
    x = np.swapaxes(g, 1, 2) if head_first else g
    B, T = x.shape[:2]
    out = np.zeros_like(x)
    bounds = [(0, T)] if cu is None else list(zip(cu[:-1], cu[1:]))
    for b in range(B):
        for s0, s1 in bounds:
            for t in range(s0, s1):
                c0 = s0 + ((t - s0) // C) * C
                c1 = min(c0 + C, s1)
                rows = range(t, c1) if reverse else range(c0, t + 1)
                out[b, t] = sum(x[b, s] for s in rows) * (1.0 if scale is None else scale)
    return np.swapaxes(out, 1, 2) if head_first else out


@pytest.mark.parametrize("case", [
    dict(B=2, T=32, H=2, S=3, C=8, reverse=False, cu=None, hf=False, scale=None),
    dict(B=2, T=30, H=1, S=2, C=8, reverse=True, cu=None, hf=False, scale=0.5),
    dict(B=1, T=33, H=2, S=2, C=16, reverse=False, cu=[0, 17, 33], hf=False, scale=0.75),
    dict(B=1, T=33, H=2, S=2, C=16, reverse=True, cu=[0, 17, 33], hf=False, scale=None),
    dict(B=2, T=24, H=3, S=2, C=8, reverse=True, cu=None, hf=True, scale=0.25),
    dict(B=1, T=56, H=1, S=2, C=16, reverse=False, cu=[0, 8, 40, 56], hf=False, scale=None),
])
def test_chunk_local_cumsum_segments_brute_force(case):
    rng = np.random.default_rng(case["T"] + case["S"])
    shape = ((case["B"], case["H"], case["T"], case["S"]) if case["hf"]
             else (case["B"], case["T"], case["H"], case["S"]))
    g = rng.standard_normal(shape)
    got = OC.chunk_local_cumsum_segments(g, case["C"], case["reverse"], case["cu"], case["hf"],
                                         case["scale"])
    ref = _brute(g, case["C"], case["reverse"], case["cu"], case["hf"], case["scale"])
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)


def test_chunk_local_cumsum_segments_matches_dense_form():
    g = np.random.default_rng(3).standard_normal((2, 64, 2, 4))
    for rev in (False, True):
        np.testing.assert_allclose(OC.chunk_local_cumsum_segments(g, 16, rev),
                                   OC.chunk_local_cumsum(g, 16, rev), rtol=1e-13, atol=1e-13)


def test_scalar_gate_equals_broadcast_channel_gate():
    rng = np.random.default_rng(11)
    B, T, H, K, V, C = 2, 64, 2, 8, 6, 16
    k, q = rng.standard_normal((2, B, T, H, K))
    v, do = rng.standard_normal((2, B, T, H, V))
    g = -np.abs(rng.standard_normal((B, T, H))) * 0.2
    gc = OC.chunk_local_cumsum(g, C)
    gk = np.repeat(gc[..., None], K, axis=-1)
    h0 = rng.standard_normal((B, H, K, V))
    hs1, ht1 = OC.chunk_fwd_h(k, v, g=gc, h0=h0, C=C)
    hs2, ht2 = OC.chunk_fwd_h(k, v, gk=gk, h0=h0, C=C)
    np.testing.assert_allclose(hs1, hs2, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(ht1, ht2, rtol=1e-12, atol=1e-12)
    d1, d01 = OC.chunk_bwd_dh(q, do, g=gc, dht=h0, scale=0.3, C=C)
    d2, d02 = OC.chunk_bwd_dh(q, do, gk=gk, dht=h0, scale=0.3, C=C)
    np.testing.assert_allclose(d1, d2, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(d01, d02, rtol=1e-12, atol=1e-12)
    # a constant per-head decay is the scalar gate gamma on every token
    gam = np.array([-0.1, -0.3])
    ramp = np.broadcast_to(gam, (B, T, H))
    np.testing.assert_allclose(OC.chunk_local_cumsum(ramp, C).reshape(B, T // C, C, H)[:, 0, :, 1],
                               np.outer(np.ones(B), (np.arange(C) + 1) * gam[1]), rtol=1e-13)


def test_kda_bwd_intra_against_autograd():
    """chunk_kda_bwd_intra = the float64 autograd of L = sum(dAqk * Aqk) + sum(dAkk * Akk)
    (with the i >= j masks), dg scaled by 1 / ln 2 (the reference drops that factor)."""
    import torch
    from oracle import kda as KO
    rng = np.random.default_rng(5)
    B, T, H, K, C = 1, 32, 2, 8, 16
    q, k = rng.standard_normal((2, B, T, H, K)) * 0.5
    g = OC.chunk_local_cumsum(-np.abs(rng.standard_normal((B, T, H, K))) * 0.3, C)
    beta = 1 / (1 + np.exp(-rng.standard_normal((B, T, H))))
    dAqk, dAkk = rng.standard_normal((2, B, T, H, C))
    tq, tk, tg, tb = (torch.tensor(x, requires_grad=True) for x in (q, k, g, beta))
    NT = T // C
    mask = torch.tril(torch.ones(C, C, dtype=torch.bool))[None, None, :, None, :]
    q5, k5, g5 = (x.reshape(B, NT, C, H, K) for x in (tq, tk, tg))
    b5 = tb.reshape(B, NT, C, H)
    E = torch.exp2(g5[:, :, :, None] - g5[:, :, None, :])
    Aqk = torch.einsum("bnihk,bnjhk,bnijhk->bnihj", q5, k5, E)
    Akk = b5[..., None] * torch.einsum("bnihk,bnjhk,bnijhk->bnihj", k5, k5, E)
    uq = torch.tensor(dAqk).reshape(B, NT, C, H, C)
    uk = torch.tensor(dAkk).reshape(B, NT, C, H, C)
    L = (torch.where(mask, uq, 0.0) * Aqk).sum() + (torch.where(mask, uk, 0.0) * Akk).sum()
    gq, gk_, gg, gb = torch.autograd.grad(L, (tq, tk, tg, tb))
    dq, dk, db, dg = KO.chunk_kda_bwd_intra(q, k, g, beta, dAqk, dAkk, C)
    np.testing.assert_allclose(dq, gq.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dk, gk_.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(db, gb.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dg, gg.numpy() / np.log(2.0), rtol=1e-10, atol=1e-12)
    # a planted mistake (beta on the column instead of the row) is caught
    bad = KO.chunk_kda_bwd_intra(q, k, g, np.roll(beta, 1, axis=1), dAqk, dAkk, C)[1]
    assert np.abs(bad - gk_.numpy()).max() > 1e-3


def test_simple_gla_raw_dg_reverse_cumsum_is_the_gla_gate_gradient():
    """Reverse-cumsumming the raw per-position dg of chunk_bwd_dqkwg inside each chunk gives
    the GLA gate gradient (autograd-pinned oracle) of the same gate broadcast over K, summed
    over the channels."""
    from oracle import gla as O
    from oracle import simple_gla as SO
    rng = np.random.default_rng(21)
    B, T, H, K, V, C = 1, 64, 2, 8, 4, 16
    q, k = rng.standard_normal((2, B, T, H, K))
    v, do = rng.standard_normal((2, B, T, H, V))
    h, dh = rng.standard_normal((2, B, T // C, H, K, V)) * 0.3
    g = OC.chunk_local_cumsum(-np.abs(rng.standard_normal((B, T, H))) * 0.2, C)
    G = np.repeat(g[..., None], K, axis=-1)
    dA = O.chunk_gla_bwd_dA(v, do, 0.5, C)
    dqi, dki = O.chunk_gla_bwd_dqk_intra(q, k, G, dA, C)
    _, _, dgc = O.chunk_gla_bwd_dqkg(q, k, v, h, G, do, dh, dqi, dki, 0.5, C)
    raw = SO.chunk_bwd_dqkwg_raw_dg(q, k, v, h, do, dh, g, 0.5, C)
    rc = OC.chunk_local_cumsum(raw, C, reverse=True)
    np.testing.assert_allclose(rc, dgc.sum(-1), rtol=1e-10, atol=1e-10)
