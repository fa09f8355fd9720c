"""Pin the float64 KDA gate / L2-norm oracle (oracle/kda_gate.py) on the CPU.

Mirrors the reference's checks of tops/cpu/ops/kda/gate.py:
  gate formula at fp64 (manual formula, both modes)      tests/ref/kda/test_fused_recurrent_kda.py:133-150
  kda_gate_chunk_cumsum == chunk cumsum of the gate      tests/ref/kda/test_fused_recurrent_kda.py:158-175
and adds what the mathematics fixes independently of the oracle's own formulas:
  * special values (softplus(0) = ln 2, sigmoid(0) = 1/2, large-argument limits);
  * the activation against torch.nn.functional.softplus / torch.sigmoid with the head
    broadcast written as an explicit loop over heads;
  * every gradient (dg, dA_log, dt_bias for base and expanded bias, both modes; the L2 norm)
    against torch float64 autograd of an independently written forward;
  * the cumsum against exp2(out) == running product of exp(g) within each chunk, and varlen
    against per-sequence calls.
"""
import math

import numpy as np
import pytest
import torch

from oracle import kda_gate as G

TOL = 1e-12


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def _inputs(B, T, H, K, Ha, bias, seed):
    rng = np.random.Generator(np.random.PCG64(seed))
    g = rng.standard_normal((B, T, H, K)) * 2.0
    A_log = np.log(rng.uniform(1.0, 4.0, Ha))
    b = None
    if bias == "base":
        b = rng.standard_normal(Ha * K)
    elif bias == "full":
        b = rng.standard_normal(H * K)
    return g, A_log, b


def _torch_gate(g, A_log, b, H, K, lb):
    """Independent torch formulation: explicit per-head loop over the parameter rows."""
    Ha = A_log.shape[0]
    outs = []
    for h in range(H):
        a = A_log[h // (H // Ha)]
        x = g[..., h, :]
        if b is not None:
            nb = b.shape[0] // K
            x = x + b.reshape(nb, K)[h // (H // nb)]
        if lb is None:
            outs.append(-torch.exp(a) * torch.nn.functional.softplus(x))
        else:
            outs.append(lb * torch.sigmoid(torch.exp(a) * x))
    return torch.stack(outs, -2)


def test_special_values():
    g = np.zeros((1, 1, 2, 4))
    A0 = np.zeros(2)
    np.testing.assert_allclose(G.kda_gate(g, A0), -math.log(2.0), rtol=1e-15)
    np.testing.assert_allclose(G.kda_gate(g, A0, lower_bound=-5.0), -2.5, rtol=1e-15)
    # softplus(x) -> x for large x, -> exp(x) for very negative x
    big = np.full((1, 1, 1, 4), 40.0)
    np.testing.assert_allclose(G.kda_gate(big, np.zeros(1)), -40.0, rtol=1e-15)
    neg = np.full((1, 1, 1, 4), -30.0)
    np.testing.assert_allclose(G.kda_gate(neg, np.zeros(1)), -math.exp(-30.0), rtol=1e-12)
    # A_log scales the standard gate by exp(A_log)
    np.testing.assert_allclose(G.kda_gate(g, np.log([2.0, 3.0]))[..., 1, :], -3 * math.log(2.0),
                               rtol=1e-15)


@pytest.mark.parametrize("H,Ha,bias", [(4, 4, None), (4, 4, "base"), (4, 2, "base"),
                                       (4, 2, "full"), (6, 3, None), (4, 1, "full")])
@pytest.mark.parametrize("lb", [None, -5.0, -2.0])
def test_gate_forward_and_backward_vs_torch_autograd(H, Ha, bias, lb):
    B, T, K = 2, 5, 8
    g, A_log, b = _inputs(B, T, H, K, Ha, bias, seed=H * 7 + Ha + (0 if lb is None else 1))
    y = G.kda_gate(g, A_log, b, lower_bound=lb)
    gt = torch.tensor(g, requires_grad=True)
    At = torch.tensor(A_log, requires_grad=True)
    bt = None if b is None else torch.tensor(b, requires_grad=True)
    yt = _torch_gate(gt, At, bt, H, K, lb)
    assert _rel(y, yt.detach().numpy()) < TOL
    dy = np.random.Generator(np.random.PCG64(5)).standard_normal(y.shape)
    (yt * torch.tensor(dy)).sum().backward()
    dg, dA, db = G.kda_gate_bwd(g, A_log, b, dy, lower_bound=lb)
    assert _rel(dg, gt.grad.numpy()) < TOL
    assert _rel(dA, At.grad.numpy()) < 1e-11
    if b is None:
        assert db is None
    else:
        assert db.shape == b.shape
        assert _rel(db, bt.grad.numpy()) < 1e-11


def test_gate_backward_without_batch_axes():
    """[H, K] inputs (no leading axes) reduce over nothing but the head repeats."""
    g, A_log, b = _inputs(1, 1, 4, 8, 2, "base", seed=9)
    g = g[0, 0]
    dy = np.ones_like(g)
    dg, dA, db = G.kda_gate_bwd(g, A_log, b, dy)
    gt = torch.tensor(g, requires_grad=True)
    At = torch.tensor(A_log, requires_grad=True)
    bt = torch.tensor(b, requires_grad=True)
    _torch_gate(gt, At, bt, 4, 8, None).sum().backward()
    assert _rel(dg, gt.grad.numpy()) < TOL
    assert _rel(dA, At.grad.numpy()) < TOL and _rel(db, bt.grad.numpy()) < TOL


@pytest.mark.parametrize("C", [4, 8, 64])
def test_chunk_cumsum_is_a_running_product(C):
    rng = np.random.Generator(np.random.PCG64(C))
    g = -np.abs(rng.standard_normal((2, 19, 2, 4))) / 4
    out = G.kda_gate_chunk_cumsum(g, C)
    for b in range(2):
        for t in range(19):
            c0 = (t // C) * C
            prod = np.prod(np.exp(g[b, c0:t + 1]), axis=0)
            np.testing.assert_allclose(np.exp2(out[b, t]), prod, rtol=1e-13)


def test_chunk_cumsum_varlen_matches_per_sequence():
    rng = np.random.Generator(np.random.PCG64(3))
    g = rng.standard_normal((1, 19, 2, 8))
    cu = [0, 7, 19]
    out = G.kda_gate_chunk_cumsum(g, 8, cu_seqlens=cu)
    for s, e in zip(cu[:-1], cu[1:]):
        np.testing.assert_allclose(out[:, s:e], G.kda_gate_chunk_cumsum(g[:, s:e], 8), rtol=0, atol=0)


def test_fla_form_of_the_cumsum_equals_cumsum_of_the_gate():
    """tests/ref/kda/test_fused_recurrent_kda.py:158-175: the FLA-form cumsum is the natural-log
    chunk cumsum of the activated gate; the accelerator form divides by ln 2."""
    g, A_log, b = _inputs(1, 19, 2, 8, 2, "full", seed=1)
    y = G.kda_gate(g, A_log, b)
    nat = G.kda_gate_chunk_cumsum(y, 8, cu_seqlens=[0, 7, 19]) * math.log(2.0)
    for s, e in ((0, 7), (7, 19)):
        for c0 in range(s, e, 8):
            c1 = min(c0 + 8, e)
            np.testing.assert_allclose(nat[:, c0:c1], np.cumsum(y[:, c0:c1], axis=1), rtol=1e-13)


@pytest.mark.parametrize("D", [1, 8, 64, 130])
def test_l2norm_and_its_gradient(D):
    rng = np.random.Generator(np.random.PCG64(D))
    x = rng.standard_normal((3, 5, D))
    y = G.l2norm(x)
    ss = (x * x).sum(-1)
    np.testing.assert_allclose((y * y).sum(-1), ss / (ss + 1e-6), rtol=1e-13)
    np.testing.assert_allclose(y * np.sqrt(ss + 1e-6)[..., None], x, rtol=1e-13)
    xt = torch.tensor(x, requires_grad=True)
    dy = rng.standard_normal(x.shape)
    (xt / torch.sqrt((xt * xt).sum(-1, keepdim=True) + 1e-6) * torch.tensor(dy)).sum().backward()
    assert _rel(G.l2norm_bwd(x, dy), xt.grad.numpy()) < TOL


def test_planted_mistakes_are_caught():
    """A dropped bias, a dropped exp(A) or a mis-folded head broadcast changes the results the
    checks above compare."""
    g, A_log, b = _inputs(1, 3, 4, 8, 2, "base", seed=4)
    y = G.kda_gate(g, A_log, b)
    assert _rel(G.kda_gate(g, A_log, None), y) > 1e-3
    assert _rel(-np.logaddexp(g + np.repeat(b.reshape(2, 8), 2, 0), 0.0), y) > 1e-3
    wrong_b = np.tile(b.reshape(2, 8), (2, 1)).reshape(-1)   # tiled instead of repeated heads
    assert _rel(G.kda_gate(g, A_log, wrong_b), y) > 1e-3
