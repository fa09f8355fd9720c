"""Pin the float64 oracle of the two KDA forward stages (CPU only).

  kda_intra_chunk_fwd           (tops/ops/kda/chunk_intra.py:91-281)
  chunk_gated_delta_rule_fwd_h  (tops/cpu/ops/common/chunk_delta_h.py:22-118,
                                 tops/ops/common/chunk_delta_h.py:44-166, 898-993)

Independent forms: the chunk parts of oracle.kda.chunk_kda_fwd_parts (natural-log gates,
(I + Akk)^-1 by numpy.linalg.inv, the state recurrence written on the un-split formulas),
the GLA state recurrence oracle.common.chunk_fwd_h (the delta pass with w = 0 and a scalar
gate), per-segment inverses by numpy.linalg.inv (segment masks), and per-sequence calls
(varlen).  Each check has a planted mistake that it must catch.
"""
import numpy as np
import pytest

from oracle import common as OC
from oracle import kda as KD
from _closed_forms import rel
from _inputs import kda_inputs

TOL = 1e-10
LN2 = np.log(2.0)


def _log2_cumsum(g, C):
    """Chunk-local cumsum of natural-log gates [B,T,H,K], in log2 units."""
    B, T = g.shape[:2]
    return (np.cumsum(g.reshape(B, T // C, C, *g.shape[2:]), axis=2) / LN2).reshape(g.shape)


def _hf(x):
    """[B,T,H,...] -> head-first [B,H,T,...]."""
    return np.ascontiguousarray(np.swapaxes(x, 1, 2))


@pytest.mark.parametrize("B,T,H,K,V,C", [(1, 128, 2, 16, 32, 64), (2, 64, 1, 8, 8, 16),
                                         (1, 96, 2, 32, 16, 32)])
def test_intra_matches_chunk_parts(B, T, H, K, V, C):
    d = kda_inputs(B, T, H, K, V, seed=T + K + C, gate_div=2.0)
    scale = K ** -0.5
    P = KD.chunk_kda_fwd_parts(d["q"], d["k"], d["v"], d["g"], d["beta"], scale, None, C)
    G = _log2_cumsum(np.float64(d["g"]), C)
    u, w, qg, kg, Aqk, Akk_inv = KD.kda_intra_chunk_fwd(
        _hf(d["q"]), _hf(d["k"]), _hf(G), _hf(d["beta"]), _hf(d["v"]), scale=scale, chunk_size=C)
    NT = T // C
    # parts: [B, NT, C, H, .] and [B, NT, i, j, H]
    hf = lambda x: np.moveaxis(x, 3, 1).reshape(B, H, T, -1)       # noqa: E731
    sq = lambda x: np.moveaxis(x, 4, 1)                              # noqa: E731
    assert rel(u, hf(P["u"])) < TOL and rel(w, hf(P["w"])) < TOL
    assert rel(Aqk, sq(P["Aqk"])) < TOL and rel(Akk_inv, sq(P["T"])) < TOL
    Gn = P["Gn"]
    assert rel(qg, hf(np.float64(d["q"]).reshape(B, NT, C, H, K) * np.exp(Gn))) < TOL
    assert rel(kg, hf(np.float64(d["k"]).reshape(B, NT, C, H, K) * np.exp(Gn[:, :, -1:] - Gn))) < TOL
    # planted: the gate difference taken the other way round
    _, _, _, _, bad, _ = KD.kda_intra_chunk_fwd(_hf(d["q"]), _hf(d["k"]), -_hf(G), _hf(d["beta"]),
                                                _hf(d["v"]), scale=scale, chunk_size=C)
    assert rel(bad, sq(P["Aqk"])) > 1e-3


def test_intra_segments_are_block_diagonal():
    """Two segments inside one chunk: Akk_inv is the block diagonal of the per-segment
    inverses, u = Akk_inv (beta v), and Aqk has no cross-segment entries."""
    B, T, H, K, V, C = 1, 32, 1, 8, 8, 32
    d = kda_inputs(B, T, H, K, V, seed=5, gate_div=2.0)
    G = _log2_cumsum(np.float64(d["g"]), C)
    seg = np.array([[0] * 12 + [1] * 20])
    args = (_hf(d["q"]), _hf(d["k"]), _hf(G), _hf(d["beta"]), _hf(d["v"]))
    u, w, qg, kg, Aqk, Akk_inv = KD.kda_intra_chunk_fwd(*args, segment_ids=seg, scale=0.5,
                                                        chunk_size=C)
    k = np.float64(d["k"][0, :, 0])
    beta = np.float64(d["beta"][0, :, 0])
    g = G[0, :, 0]
    want = np.zeros((C, C))
    for a, b in ((0, 12), (12, 32)):
        Akk = np.zeros((b - a, b - a))
        for i in range(b - a):
            for j in range(i):
                Akk[i, j] = beta[a + i] * np.sum(k[a + i] * k[a + j] * 2.0 ** (g[a + i] - g[a + j]))
        want[a:b, a:b] = np.linalg.inv(np.eye(b - a) + Akk)
    assert rel(Akk_inv[0, 0, 0], want) < TOL
    assert rel(u[0, 0], want @ (beta[:, None] * np.float64(d["v"][0, :, 0]))) < TOL
    assert np.all(Aqk[0, 0, 0, 12:, :12] == 0.0)
    # planted: the segment ids ignored
    _, _, _, _, _, bad = KD.kda_intra_chunk_fwd(*args, segment_ids=None, scale=0.5, chunk_size=C)
    assert rel(bad[0, 0, 0], want) > 1e-3


@pytest.mark.parametrize("B,T,H,K,V,C", [(1, 128, 2, 16, 32, 64), (2, 64, 2, 8, 8, 16)])
def test_delta_h_matches_chunk_parts(B, T, H, K, V, C):
    d = kda_inputs(B, T, H, K, V, seed=11 + T, gate_div=2.0, h0=True)
    P = KD.chunk_kda_fwd_parts(d["q"], d["k"], d["v"], d["g"], d["beta"], 1.0, d["h0"], C)
    Gn = P["Gn"]
    kg = (np.float64(d["k"]).reshape(P["u"].shape[:-1] + (K,)) * np.exp(Gn[:, :, -1:] - Gn))
    flat = lambda x: x.reshape(B, T, H, -1)                           # noqa: E731
    G = _log2_cumsum(np.float64(d["g"]), C)
    h, vn, ht = KD.chunk_gated_delta_rule_fwd_h(flat(kg), flat(P["w"]), flat(P["u"]), gk=G,
                                                initial_state=d["h0"], output_final_state=True,
                                                chunk_size=C)
    assert rel(h, P["S"]) < TOL and rel(vn, flat(P["v_new"])) < TOL and rel(ht, P["ht"]) < TOL
    # natural-log gates with use_exp2=False are the same recurrence
    h2, _, _ = KD.chunk_gated_delta_rule_fwd_h(flat(kg), flat(P["w"]), flat(P["u"]), gk=G * LN2,
                                               initial_state=d["h0"], chunk_size=C,
                                               use_exp2=False)
    assert rel(h2, P["S"]) < TOL
    # planted: the state decayed with the first token's gate instead of the last
    Gbad = np.repeat(G.reshape(B, T // C, C, H, K)[:, :, :1], C, axis=2).reshape(G.shape)
    hb, _, _ = KD.chunk_gated_delta_rule_fwd_h(flat(kg), flat(P["w"]), flat(P["u"]), gk=Gbad,
                                               initial_state=d["h0"], chunk_size=C)
    assert rel(hb, P["S"]) > 1e-3


def test_delta_h_scalar_gate_is_gla_recurrence():
    """w = 0: the pass is the GLA state recurrence with a scalar gate, u the values."""
    B, T, H, K, V, C = 2, 128, 2, 8, 16, 32
    rng = np.random.default_rng(3)
    k, u = rng.standard_normal((B, T, H, K)), rng.standard_normal((B, T, H, V))
    gn = -np.abs(rng.standard_normal((B, T, H))) / 4
    gc = np.cumsum(gn.reshape(B, T // C, C, H), axis=2).reshape(B, T, H)     # natural log
    h0 = rng.standard_normal((B, H, K, V))
    hs, hfin = OC.chunk_fwd_h(k, u, g=gc, h0=h0, C=C)
    h, vn, ht = KD.chunk_gated_delta_rule_fwd_h(k, np.zeros_like(k), u, g=gc / LN2,
                                                initial_state=h0, output_final_state=True,
                                                chunk_size=C)
    assert rel(h, hs) < TOL and rel(ht, hfin) < TOL and rel(vn, u) < TOL
    # planted: the update's v_new left ungated
    hb, _, _ = KD.chunk_gated_delta_rule_fwd_h(k, np.zeros_like(k), u, g=None, gk=None,
                                               initial_state=h0, chunk_size=C)
    assert rel(hb, hs) > 1e-3


def test_delta_h_varlen_is_per_sequence():
    H, K, V, C = 2, 8, 8, 16
    cu = [0, 20, 21, 64, 100]
    T = cu[-1]
    rng = np.random.default_rng(9)
    k, w = rng.standard_normal((2, 1, T, H, K)) * 0.3
    u = rng.standard_normal((1, T, H, V))
    gk = -np.abs(rng.standard_normal((1, T, H, K))) / 4
    g = -np.abs(rng.standard_normal((1, T, H))) / 4
    h0 = rng.standard_normal((len(cu) - 1, H, K, V))
    h, vn, ht = KD.chunk_gated_delta_rule_fwd_h(k, w, u, g=g, gk=gk, initial_state=h0,
                                                output_final_state=True, chunk_size=C,
                                                cu_seqlens=cu)
    hs = []
    for n in range(len(cu) - 1):
        a, b = cu[n], cu[n + 1]
        Tn = b - a
        pad = -(-Tn // C) * C - Tn
        z = lambda x: np.concatenate([x[:, a:b], np.zeros((1, pad) + x.shape[2:])], 1)  # noqa
        # a padded tail (zero k, w, u) must not decay the state: repeat the last gate
        rep = lambda x: np.concatenate([x[:, a:b], np.repeat(x[:, b - 1:b], pad, 1)], 1)  # noqa
        hn, vnn, htn = KD.chunk_gated_delta_rule_fwd_h(z(k), z(w), z(u), g=rep(g), gk=rep(gk),
                                                       initial_state=h0[n:n + 1],
                                                       output_final_state=True, chunk_size=C)
        hs.append(hn[0])
        assert rel(vn[0, a:b], vnn[0, :Tn]) < TOL and rel(ht[n], htn[0]) < TOL
    assert rel(h[0], np.concatenate(hs, 0)) < TOL
