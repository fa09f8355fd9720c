"""Pin the float64 GLA oracle against independent formulations (CPU only).

Mirrors the reference's own self-validation of tops/cpu:
  chunk vs naive at fp64 1e-10           tests/ref/gla/test_chunk_gla.py:372-391
  fused recurrent vs naive / chunk       tests/ref/gla/test_fused_recurrent_gla.py:170-232
  varlen == independent sequences        tests/ref/gla/test_chunk_gla_varlen.py:145-198
  state split == full run                tests/ops/gla/test_pallas_chunk_gla.py:223-248
  reverse                                tests/ref/gla/test_fused_recurrent_gla.py:492-501
Gradients are pinned by torch float64 autograd of the parallel form.
"""
import numpy as np
import pytest
import torch

from oracle import gla as O
from _closed_forms import gla_parallel_grads, rel
from _inputs import gla_inputs

TOL = 1e-10


def _pf(d, scale=None, h0=None, do=None, dht=None):
    B, T, H, V = d["v"].shape
    if do is None:
        do = np.zeros((B, T, H, V))
    return gla_parallel_grads(d["q"], d["k"], d["v"], d["g"], h0, do, dht, scale=scale)


@pytest.mark.parametrize("B,T,H,K,V,C,h0,scale", [
    (2, 64, 2, 16, 32, 16, False, None),
    (1, 37, 3, 8, 16, 16, True, None),       # ragged T (chunk padding)
    (2, 50, 2, 32, 16, 32, True, 0.1),       # K != V, custom scale
    (1, 1, 2, 8, 8, 16, True, None),         # T = 1
    (1, 130, 1, 16, 16, 64, False, None),
])
def test_chunk_fwd_matches_parallel_form(B, T, H, K, V, C, h0, scale):
    d = gla_inputs(B, T, H, K, V, seed=T * 7 + K, gate_div=1.0, h0=h0)
    o, ht = O.chunk_gla(d["q"], d["k"], d["v"], d["g"], scale=scale, initial_state=d["h0"],
                        output_final_state=True, chunk_size=C)
    ref = _pf(d, scale=scale, h0=d["h0"])
    assert rel(o, ref["o"]) < TOL
    assert rel(ht, ref["ht"]) < TOL


def test_zero_gate_is_causal_linear_attention():
    """g = 0, h0 = 0: o = scale * tril(Q K^T) V, a plain matmul (textbook)."""
    d = gla_inputs(2, 70, 2, 16, 24, seed=5)
    o, ht = O.chunk_gla(d["q"], d["k"], d["v"], None, output_final_state=True, chunk_size=16)
    q, k, v = (d[x].astype(np.float64) for x in "qkv")
    s = 16 ** -0.5
    for b in range(2):
        for h in range(2):
            A = np.tril(q[b, :, h] @ k[b, :, h].T)
            assert np.allclose(o[b, :, h], s * A @ v[b, :, h], rtol=1e-12, atol=1e-12)
            assert np.allclose(ht[b, h], k[b, :, h].T @ v[b, :, h], rtol=1e-12, atol=1e-12)


def test_single_token_closed_form():
    """T = 1: o = scale * (h0*exp(g0)[:,None] + k0 v0^T)^T q0."""
    d = gla_inputs(1, 1, 1, 4, 3, seed=9, gate_div=1.0, h0=True)
    o, ht = O.chunk_gla(d["q"], d["k"], d["v"], d["g"], initial_state=d["h0"],
                        output_final_state=True)
    q0, k0, v0, g0 = (d[x][0, 0, 0].astype(np.float64) for x in "qkvg")
    S = d["h0"][0, 0].astype(np.float64) * np.exp(g0)[:, None] + np.outer(k0, v0)
    assert np.allclose(o[0, 0, 0], 0.5 * S.T @ q0, rtol=1e-13)
    assert np.allclose(ht[0, 0], S, rtol=1e-13)


@pytest.mark.parametrize("C", [16, 64])
def test_chunk_vs_naive(C):
    d = gla_inputs(2, 100, 2, 16, 16, seed=3, gate_div=1.0, h0=True)
    o, ht = O.chunk_gla(d["q"], d["k"], d["v"], d["g"], initial_state=d["h0"],
                        output_final_state=True, chunk_size=C)
    on, hn = O.naive_recurrent_gla(d["q"], d["k"], d["v"], d["g"], d["h0"], True)
    assert rel(o, on) < TOL and rel(ht, hn) < TOL


def test_fused_recurrent_vs_parallel_form_and_chunk():
    d = gla_inputs(2, 45, 2, 8, 16, seed=11, gate_div=1.0, h0=True)
    o, ht = O.fused_recurrent_gla(d["q"], d["k"], d["v"], d["g"], initial_state=d["h0"],
                                  output_final_state=True)
    ref = _pf(d, h0=d["h0"])
    assert rel(o, ref["o"]) < TOL and rel(ht, ref["ht"]) < TOL
    oc, hc = O.chunk_gla(d["q"], d["k"], d["v"], d["g"], initial_state=d["h0"],
                         output_final_state=True, chunk_size=16)
    assert rel(o, oc) < TOL and rel(ht, hc) < TOL


def test_fused_recurrent_gv_vs_parallel_form():
    rng = np.random.default_rng(4)
    d = gla_inputs(1, 20, 2, 8, 8, seed=12, gate_div=1.0, h0=True)
    gv = -np.abs(rng.standard_normal((1, 20, 2, 8))) * 0.3
    o, ht = O.fused_recurrent_gla(d["q"], d["k"], d["v"], d["g"], gv, initial_state=d["h0"],
                                  output_final_state=True)
    t = {n: torch.tensor(np.asarray(x, np.float64)) for n, x in
         dict(q=d["q"], k=d["k"], v=d["v"], g=d["g"], h0=d["h0"], gv=gv).items()}
    from _closed_forms import gla_parallel_torch
    po, pht = gla_parallel_torch(t["q"], t["k"], t["v"], t["g"], t["h0"], None, t["gv"])
    assert rel(o, po.numpy()) < TOL and rel(ht, pht.numpy()) < TOL


def test_reverse_equals_flipped_sequence():
    d = gla_inputs(1, 33, 2, 8, 8, seed=13, gate_div=1.0, h0=True)
    o_r, ht_r = O.fused_recurrent_gla(d["q"], d["k"], d["v"], d["g"], initial_state=d["h0"],
                                      output_final_state=True, reverse=True)
    fl = {x: d[x][:, ::-1] for x in "qkvg"}
    o_f, ht_f = O.fused_recurrent_gla(fl["q"], fl["k"], fl["v"], fl["g"],
                                      initial_state=d["h0"], output_final_state=True)
    assert rel(o_r, o_f[:, ::-1]) < TOL and rel(ht_r, ht_f) < TOL
    o_n, _ = O.fused_recurrent_gla(d["q"], d["k"], d["v"], d["g"], initial_state=d["h0"])
    assert rel(o_r, o_n) > 1e-3


def test_varlen_equals_independent_sequences():
    cu = [0, 13, 64, 65, 140]
    d = gla_inputs(1, 140, 2, 16, 8, seed=21, gate_div=1.0, h0=True, N=4)
    o, ht = O.chunk_gla(d["q"], d["k"], d["v"], d["g"], initial_state=d["h0"],
                        output_final_state=True, cu_seqlens=cu, chunk_size=16)
    for n in range(4):
        s = slice(cu[n], cu[n + 1])
        on, hn = O.naive_recurrent_gla(d["q"][:, s], d["k"][:, s], d["v"][:, s], d["g"][:, s],
                                       d["h0"][n:n + 1], True)
        assert rel(o[:, s], on) < TOL and rel(ht[n:n + 1], hn) < TOL
    of, hf = O.fused_recurrent_gla(d["q"], d["k"], d["v"], d["g"], initial_state=d["h0"],
                                   output_final_state=True, cu_seqlens=cu)
    assert rel(o, of) < TOL and rel(ht, hf) < TOL


def test_state_split():
    d = gla_inputs(1, 40, 2, 16, 32, seed=77, gate_div=1.0)
    _, hfull = O.chunk_gla(d["q"], d["k"], d["v"], d["g"], output_final_state=True)
    _, h1 = O.chunk_gla(*(d[x][:, :20] for x in "qkvg"), output_final_state=True)
    _, h2 = O.chunk_gla(*(d[x][:, 20:] for x in "qkvg"), initial_state=h1,
                        output_final_state=True)
    assert rel(h2, hfull) < TOL


@pytest.mark.parametrize("B,T,H,K,V,C,h0", [
    (1, 64, 2, 8, 16, 16, True),
    (2, 45, 1, 16, 8, 16, True),      # ragged
    (1, 96, 2, 16, 16, 32, False),
])
def test_chunk_bwd_matches_autograd(B, T, H, K, V, C, h0):
    d = gla_inputs(B, T, H, K, V, seed=101 + T, gate_div=1.0, h0=True, grads=True)
    if not h0:
        d["h0"] = np.zeros_like(d["h0"])
    dq, dk, dv, dg, dh0 = O.chunk_gla_bwd(d["q"], d["k"], d["v"], d["g"], K ** -0.5, d["h0"],
                                          d["do"], d["dht"], chunk_size=C)
    ref = gla_parallel_grads(d["q"], d["k"], d["v"], d["g"], d["h0"], d["do"], d["dht"])
    for name, x in dict(dq=dq, dk=dk, dv=dv, dg=dg, dh0=dh0).items():
        assert rel(x, ref[name]) < 1e-9, name


def test_chunk_bwd_varlen_matches_autograd_per_sequence():
    cu = [0, 20, 21, 70]
    d = gla_inputs(1, 70, 2, 8, 8, seed=202, gate_div=1.0, h0=True, N=3, grads=True)
    dq, dk, dv, dg, dh0 = O.chunk_gla_bwd(d["q"], d["k"], d["v"], d["g"], 8 ** -0.5, d["h0"],
                                          d["do"], d["dht"], chunk_size=16, cu_seqlens=cu)
    for n in range(3):
        s = slice(cu[n], cu[n + 1])
        ref = gla_parallel_grads(d["q"][:, s], d["k"][:, s], d["v"][:, s], d["g"][:, s],
                                 d["h0"][n:n + 1], d["do"][:, s], d["dht"][n:n + 1])
        for name, x in dict(dq=dq, dk=dk, dv=dv, dg=dg).items():
            assert rel(x[:, s], ref[name]) < 1e-9, (n, name)
        assert rel(dh0[n:n + 1], ref["dh0"]) < 1e-9


@pytest.mark.parametrize("reverse", [False, True])
def test_fused_recurrent_bwd_matches_autograd(reverse):
    rng = np.random.default_rng(8)
    d = gla_inputs(2, 30, 2, 8, 8, seed=303, gate_div=1.0, h0=True, grads=True)
    gv = -np.abs(rng.standard_normal((2, 30, 2, 8))) * 0.2
    if reverse:
        flip = lambda x: np.ascontiguousarray(x[:, ::-1])
    else:
        flip = lambda x: x
    o, _ = O.fused_recurrent_fwd(d["q"], d["k"], d["v"], d["g"], gv, initial_state=d["h0"],
                                 reverse=reverse)
    dq, dk, dv, dgk, dgv, dh0 = O.fused_recurrent_bwd(
        d["q"], d["k"], d["v"], d["g"], gv, o, d["do"], d["dht"], initial_state=d["h0"],
        reverse=reverse)
    ref = gla_parallel_grads(flip(d["q"]), flip(d["k"]), flip(d["v"]), flip(d["g"]), d["h0"],
                             flip(d["do"]), d["dht"], gv=flip(gv))
    assert rel(dq, flip(ref["dq"])) < 1e-9
    assert rel(dk, flip(ref["dk"])) < 1e-9
    assert rel(dv, flip(ref["dv"])) < 1e-9
    assert rel(dgk, flip(ref["dg"])) < 1e-9
    assert rel(dgv, flip(ref["dgv"])) < 1e-9
    assert rel(dh0, ref["dh0"]) < 1e-9


def test_planted_mistake_is_caught():
    """A dropped boundary term in dg (a plausible bug) must fail the autograd pin."""
    d = gla_inputs(1, 64, 1, 8, 8, seed=404, gate_div=1.0, h0=True, grads=True)
    C = 16
    q, k, v, g, h0, do, dht = (np.asarray(d[x], np.float64)
                               for x in ("q", "k", "v", "g", "h0", "do", "dht"))
    gc = O.chunk_local_cumsum(g, C)
    h, _ = O.chunk_fwd_h(k, v, gk=gc, h0=h0, C=C)
    dh, _ = O.chunk_bwd_dh(q, do, gk=gc, dht=dht, scale=8 ** -0.5, C=C)
    A = O.causal_mask_A(O.chunk_gla_fwd_intra_gk(q, k, gc, 8 ** -0.5, C), C)
    dA = O.chunk_gla_bwd_dA(v, do, 8 ** -0.5, C)
    dq, dk = O.chunk_gla_bwd_dqk_intra(q, k, gc, dA, C)
    _, _, dg = O.chunk_gla_bwd_dqkg(q, k, v, h * 0.0, gc, do, dh, dq, dk, 8 ** -0.5, C)
    ref = gla_parallel_grads(q, k, v, g, h0, do, dht)
    assert rel(dg, ref["dg"]) > 1e-3
