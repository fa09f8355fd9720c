"""Pin the float64 simple-GLA oracle against independent formulations (CPU only).

Mirrors the reference's own self-validation of tops/cpu simple GLA:
  chunk vs naive at fp64                  tests/ref/simple_gla (chunk vs naive)
  varlen bwd vs per-sequence autograd     tests/ref/simple_gla/test_chunk_simple_gla_varlen.py:341-420
Gradients are pinned by torch float64 autograd of the parallel form with the scalar
gate broadcast over K inside the autograd graph (so dg [B,T,H] comes out summed over K),
and the chunked oracle is cross-checked against the GLA oracle with broadcast gates.
"""
import numpy as np
import pytest
import torch

from oracle import simple_gla as S
from oracle import gla as O
from _closed_forms import gla_parallel_torch, rel
from _inputs import simple_gla_inputs, varlen_cu

TOL = 1e-10


def _autograd(d, gate, h0, do, dht, scale=None):
    """o, ht and gradients of sum(o*do) + sum(ht*dht) through the parallel form."""
    t = {n: torch.tensor(np.asarray(d[n], np.float64), requires_grad=True) for n in "qkv"}
    K = d["q"].shape[-1]
    if gate == "g":
        gs = torch.tensor(np.asarray(d["g"], np.float64), requires_grad=True)
        gk = gs[..., None].expand(*gs.shape, K)
    else:
        gs = None
        B, T, H = d["g"].shape
        gk = torch.tensor(np.asarray(d["g_gamma"], np.float64))[None, None, :, None].expand(B, T, H, K)
    h0t = None if h0 is None else torch.tensor(np.asarray(h0, np.float64), requires_grad=True)
    o, ht = gla_parallel_torch(t["q"], t["k"], t["v"], gk, h0t, scale)
    loss = (o * torch.tensor(np.asarray(do, np.float64))).sum()
    if dht is not None:
        loss = loss + (ht * torch.tensor(np.asarray(dht, np.float64))).sum()
    loss.backward()
    out = dict(o=o.detach().numpy(), ht=ht.detach().numpy(), dq=t["q"].grad.numpy(),
               dk=t["k"].grad.numpy(), dv=t["v"].grad.numpy())
    if gs is not None:
        out["dg"] = gs.grad.numpy()
    if h0t is not None:
        out["dh0"] = h0t.grad.numpy()
    return out


@pytest.mark.parametrize("gate", ["g", "gamma"])
@pytest.mark.parametrize("B,T,H,K,V,C,h0", [
    (2, 64, 2, 16, 32, 16, False),
    (1, 37, 3, 8, 16, 16, True),      # ragged T
    (2, 50, 2, 32, 16, 32, True),
    (1, 1, 2, 8, 8, 16, True),        # T = 1
])
def test_chunk_matches_naive(gate, B, T, H, K, V, C, h0):
    d = simple_gla_inputs(B, T, H, K, V, seed=T + 13 * K, h0=h0)
    g, gg = (d["g"], None) if gate == "g" else (None, d["g_gamma"])
    o, ht = S.chunk_simple_gla(d["q"], d["k"], d["v"], g=g, g_gamma=gg, initial_state=d["h0"],
                               output_final_state=True, chunk_size=C)
    on, hn = S.naive_simple_gla(d["q"], d["k"], d["v"], g=g, g_gamma=gg, initial_state=d["h0"],
                                output_final_state=True)
    assert rel(o, on) < TOL and rel(ht, hn) < TOL


def test_gamma_partial_last_chunk_uses_valid_length():
    """g_gamma with T % C != 0: the last chunk decays by gamma * valid_len
    (tops/cpu/ops/common/chunk_h.py:213-216), which the naive recurrence fixes."""
    d = simple_gla_inputs(1, 70, 2, 8, 8, seed=4, h0=True)
    o, ht = S.chunk_simple_gla(d["q"], d["k"], d["v"], g_gamma=d["g_gamma"], initial_state=d["h0"],
                               output_final_state=True, chunk_size=64)
    on, hn = S.naive_simple_gla(d["q"], d["k"], d["v"], g_gamma=d["g_gamma"], initial_state=d["h0"],
                                output_final_state=True)
    assert rel(ht, hn) < TOL and rel(o, on) < TOL


@pytest.mark.parametrize("gate", ["g", "gamma"])
@pytest.mark.parametrize("B,T,H,K,V,C", [(2, 48, 2, 8, 16, 16), (1, 37, 2, 16, 8, 16),
                                         (1, 70, 1, 8, 8, 32)])
def test_bwd_matches_autograd(gate, B, T, H, K, V, C):
    d = simple_gla_inputs(B, T, H, K, V, seed=T * 3 + V, h0=True, grads=True)
    g, gg = (d["g"], None) if gate == "g" else (None, d["g_gamma"])
    dq, dk, dv, dg, dh0 = S.chunk_simple_gla_bwd(d["q"], d["k"], d["v"], g, gg, d["h0"], d["do"],
                                                 d["dht"], K ** -0.5, chunk_size=C)
    ref = _autograd(d, gate, d["h0"], d["do"], d["dht"])
    for name, x in (("dq", dq), ("dk", dk), ("dv", dv), ("dh0", dh0)):
        assert rel(x, ref[name]) < 1e-9, name
    if gate == "g":
        assert rel(dg, ref["dg"]) < 1e-9
    else:
        assert dg is None


def test_matches_gla_oracle_with_broadcast_gate():
    """Simple GLA == GLA with the scalar gate on every K channel; dg == sum_K dg_GLA."""
    B, T, H, K, V = 1, 90, 2, 16, 16
    d = simple_gla_inputs(B, T, H, K, V, seed=21, h0=True, grads=True)
    gk = np.broadcast_to(d["g"][..., None], (B, T, H, K))
    o, ht = S.chunk_simple_gla(d["q"], d["k"], d["v"], g=d["g"], initial_state=d["h0"],
                               output_final_state=True)
    og, htg = O.chunk_gla(d["q"], d["k"], d["v"], gk, initial_state=d["h0"], output_final_state=True,
                          chunk_size=64)
    assert rel(o, og) < TOL and rel(ht, htg) < TOL
    r = S.chunk_simple_gla_bwd(d["q"], d["k"], d["v"], d["g"], None, d["h0"], d["do"], d["dht"],
                               K ** -0.5)
    rg = O.chunk_gla_bwd(d["q"], d["k"], d["v"], gk, K ** -0.5, d["h0"], d["do"], d["dht"])
    for a, b in zip(r[:3], rg[:3]):
        assert rel(a, b) < TOL
    assert rel(r[3], rg[3].sum(-1)) < TOL
    assert rel(r[4], rg[4]) < TOL


@pytest.mark.parametrize("gate", ["g", "gamma"])
def test_varlen_equals_independent(gate):
    T, H, K, V = 150, 2, 8, 16
    cu = varlen_cu(T, 4, seed=8)
    d = simple_gla_inputs(1, T, H, K, V, seed=8, h0=True, N=4, grads=True)
    g, gg = (d["g"], None) if gate == "g" else (None, d["g_gamma"])
    o, ht = S.chunk_simple_gla(d["q"], d["k"], d["v"], g=g, g_gamma=gg, initial_state=d["h0"],
                               output_final_state=True, cu_seqlens=cu)
    r = S.chunk_simple_gla_bwd(d["q"], d["k"], d["v"], g, gg, d["h0"], d["do"], d["dht"],
                               K ** -0.5, cu_seqlens=cu)
    for n in range(4):
        a, b = cu[n], cu[n + 1]
        sl = lambda x: x[:, a:b]
        on, hn = S.naive_simple_gla(sl(d["q"]), sl(d["k"]), sl(d["v"]),
                                    g=None if g is None else sl(g), g_gamma=gg,
                                    initial_state=d["h0"][n:n + 1], output_final_state=True)
        assert rel(o[:, a:b], on) < TOL and rel(ht[n:n + 1], hn) < TOL
        rn = S.chunk_simple_gla_bwd(sl(d["q"]), sl(d["k"]), sl(d["v"]),
                                    None if g is None else sl(g), gg, d["h0"][n:n + 1],
                                    sl(d["do"]), d["dht"][n:n + 1], K ** -0.5)
        for i in range(3):
            assert rel(r[i][:, a:b], rn[i]) < TOL
        if g is not None:
            assert rel(r[3][:, a:b], rn[3]) < TOL
        assert rel(r[4][n:n + 1], rn[4]) < TOL


def test_both_gates_rejected():
    d = simple_gla_inputs(1, 8, 1, 8, 8, seed=1, grads=True)
    with pytest.raises(AssertionError):
        S.chunk_simple_gla_bwd(d["q"], d["k"], d["v"], d["g"], d["g_gamma"], None, d["do"], None, 1.0)
