"""Pin the float64 KDA oracle against independent formulations (CPU only).

Mirrors the reference's self-validation of tops/cpu KDA:
  naive vs chunk at fp64                tests/ref/kda/test_naive_kda.py:195-218
  autograd gradients                    tests/ref/kda/test_naive_kda.py:253-293
  beta = 0 / zero-gate properties       tests/ref/kda/test_chunk_kda.py:179-400
Gradients are pinned by torch float64 autograd of a per-token recurrence written
independently in tests/_closed_forms.py.
"""
import numpy as np
import pytest

from oracle import kda as KD
from _closed_forms import kda_grads, rel
from _inputs import kda_inputs

TOL = 1e-10


@pytest.mark.parametrize("B,T,H,K,V,C,h0", [
    (1, 64, 2, 8, 16, 16, False),
    (2, 37, 1, 16, 8, 16, True),      # ragged T
    (1, 70, 2, 16, 16, 64, True),
    (1, 1, 2, 8, 8, 16, True),        # T = 1
])
def test_chunk_matches_naive(B, T, H, K, V, C, h0):
    d = kda_inputs(B, T, H, K, V, seed=T + K, gate_div=1.0, h0=h0)
    o, ht = KD.chunk_kda(d["q"], d["k"], d["v"], d["g"], d["beta"], initial_state=d["h0"],
                         output_final_state=True, chunk_size=C)
    on, hn = KD.naive_recurrent_kda(d["q"], d["k"], d["v"], d["g"], d["beta"],
                                    initial_state=d["h0"], output_final_state=True)
    assert rel(o, on) < TOL and rel(ht, hn) < TOL


def test_naive_matches_torch_recurrence():
    d = kda_inputs(1, 20, 2, 8, 8, seed=3, gate_div=1.0, h0=True, grads=True)
    on, hn = KD.naive_recurrent_kda(d["q"], d["k"], d["v"], d["g"], d["beta"],
                                    initial_state=d["h0"], output_final_state=True)
    ref = kda_grads(d["q"], d["k"], d["v"], d["g"], d["beta"], d["h0"], d["do"], d["dht"])
    assert rel(on, ref["o"]) < TOL and rel(hn, ref["ht"]) < TOL


def test_beta_zero_only_decays():
    """beta = 0: S_t = S_0 * exp(cumsum g), o_t = scale (q_t exp(cumsum g_t)) S_0."""
    d = kda_inputs(1, 40, 1, 8, 8, seed=4, gate_div=1.0, h0=True)
    d["beta"] = np.zeros_like(d["beta"])
    o, ht = KD.chunk_kda(d["q"], d["k"], d["v"], d["g"], d["beta"], initial_state=d["h0"],
                         output_final_state=True, chunk_size=16)
    Gc = np.cumsum(d["g"].astype(np.float64), axis=1)[0, :, 0]        # [T, K]
    S0 = d["h0"][0, 0].astype(np.float64)
    ref = (d["q"][0, :, 0].astype(np.float64) * 8 ** -0.5 * np.exp(Gc)) @ S0
    assert rel(o[0, :, 0], ref) < TOL
    assert rel(ht[0, 0], S0 * np.exp(Gc[-1])[:, None]) < TOL


@pytest.mark.parametrize("B,T,H,K,V,C", [(1, 48, 2, 8, 8, 16), (2, 37, 1, 16, 8, 16),
                                         (1, 40, 1, 8, 16, 32)])
def test_chunk_bwd_matches_autograd(B, T, H, K, V, C):
    d = kda_inputs(B, T, H, K, V, seed=100 + T, gate_div=2.0, h0=True, grads=True)
    dq, dk, dv, db, dg, dh0 = KD.chunk_kda_bwd(d["q"], d["k"], d["v"], d["g"], d["beta"],
                                               K ** -0.5, d["h0"], d["do"], d["dht"], chunk_size=C)
    ref = kda_grads(d["q"], d["k"], d["v"], d["g"], d["beta"], d["h0"], d["do"], d["dht"])
    for name, x in dict(dq=dq, dk=dk, dv=dv, dbeta=db, dg=dg, dh0=dh0).items():
        assert rel(x, ref[name]) < 1e-9, name


def test_planted_mistake_is_caught():
    """Dropping the -w^T dv_new term of the state gradient (a plausible bug) must fail the
    autograd pin: the recursion is rerun here without it."""
    d = kda_inputs(1, 48, 1, 8, 8, seed=9, gate_div=2.0, h0=True, grads=True)
    (_, _, _, _, _, dh0), P = KD.chunk_kda_bwd(d["q"], d["k"], d["v"], d["g"], d["beta"],
                                               8 ** -0.5, d["h0"], d["do"], d["dht"],
                                               chunk_size=16, return_parts=True)
    ref = kda_grads(d["q"], d["k"], d["v"], d["g"], d["beta"], d["h0"], d["do"], d["dht"])
    assert rel(dh0, ref["dh0"]) < 1e-9
    # recompute the reverse pass without the delta-rule term
    C, s = 16, 8 ** -0.5
    Gn, Aqk = P["Gn"], P["Aqk"]
    qc = d["q"].astype(np.float64).reshape(1, 3, C, 1, 8)
    kc = d["k"].astype(np.float64).reshape(1, 3, C, 1, 8)
    doc = d["do"].astype(np.float64).reshape(1, 3, C, 1, 8)
    dS = d["dht"].astype(np.float64)
    for n in range(2, -1, -1):
        Gl = Gn[:, n, -1]
        dS = dS * np.exp(Gl)[..., None] + np.einsum("bihk,bihv->bhkv", qc[:, n] * s * np.exp(Gn[:, n]), doc[:, n])
    assert rel(dS, ref["dh0"]) > 1e-3
