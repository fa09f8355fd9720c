"""Pin the float64 oracle of the layer-side modules (oracle/modules.py) on the CPU.

Mirrors the reference's module checks (tests/modules/test_modules.py: RMSNorm and
FusedRMSNormGated against the manual formula, ShortConvolution causality, packed varlen ==
separate sequences, decode step shapes) and pins every function against independent library
routines: torch.nn.functional.rms_norm / silu and torch.nn.functional.conv1d (depthwise,
groups = D) in float64, their autograd for the backward, and decode steps chained after a
prefill against the prefill of the longer sequence.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import modules as M

TOL = 1e-12


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


@pytest.mark.parametrize("gate", [False, True])
@pytest.mark.parametrize("affine", [False, True])
@pytest.mark.parametrize("D", [1, 7, 64, 300])
def test_rmsnorm_gated_vs_torch(D, affine, gate):
    rng = np.random.Generator(np.random.PCG64(D))
    x = rng.standard_normal((3, 5, D))
    g = rng.standard_normal((3, 5, D)) if gate else None
    w = rng.standard_normal(D) if affine else None
    xt = torch.tensor(x, requires_grad=True)
    gt = None if g is None else torch.tensor(g, requires_grad=True)
    wt = None if w is None else torch.tensor(w, requires_grad=True)
    yt = F.rms_norm(xt, (D,), wt, eps=1e-5)
    if gt is not None:
        yt = yt * F.silu(gt)
    y = M.rmsnorm_gated(x, g, w, eps=1e-5)
    assert _rel(y, yt.detach().numpy()) < TOL
    dy = rng.standard_normal(x.shape)
    (yt * torch.tensor(dy)).sum().backward()
    dx, dg, dw = M.rmsnorm_gated_bwd(x, g, w, dy, eps=1e-5)
    assert _rel(dx, xt.grad.numpy()) < 1e-11
    if gate:
        assert _rel(dg, gt.grad.numpy()) < TOL
    else:
        assert dg is None
    if affine:
        assert _rel(dw, wt.grad.numpy()) < TOL
    else:
        assert dw is None


def _torch_conv(x, w, b, act):
    """Depthwise causal conv1d through torch: [B,T,D] -> [B,T,D]."""
    D, W = w.shape
    y = F.conv1d(F.pad(x.transpose(1, 2), (W - 1, 0)), w.unsqueeze(1), b, groups=D)
    y = y.transpose(1, 2)
    return F.silu(y) if act == "silu" else y


@pytest.mark.parametrize("act", ["silu", None])
@pytest.mark.parametrize("W", [1, 2, 4, 7])
@pytest.mark.parametrize("bias", [False, True])
def test_short_conv_vs_torch_conv1d(W, act, bias):
    rng = np.random.Generator(np.random.PCG64(W))
    B, T, D = 2, 11, 6
    x = rng.standard_normal((B, T, D))
    w = rng.standard_normal((D, W))
    b = rng.standard_normal(D) if bias else None
    xt, wt = torch.tensor(x, requires_grad=True), torch.tensor(w, requires_grad=True)
    bt = None if b is None else torch.tensor(b, requires_grad=True)
    yt = _torch_conv(xt, wt, bt, act)
    assert _rel(M.short_conv(x, w, b, act), yt.detach().numpy()) < TOL
    dy = rng.standard_normal(x.shape)
    (yt * torch.tensor(dy)).sum().backward()
    dx, dw, db = M.short_conv_bwd(x, w, b, dy, act)
    assert _rel(dx, xt.grad.numpy()) < TOL
    assert _rel(dw, wt.grad.numpy()) < TOL
    if bias:
        assert _rel(db, bt.grad.numpy()) < TOL
    else:
        assert db is None


def test_short_conv_causal_and_varlen():
    rng = np.random.Generator(np.random.PCG64(2))
    D, W = 8, 3
    w, b = rng.standard_normal((D, W)), rng.standard_normal(D)
    x1 = rng.standard_normal((1, 16, D))
    x2 = x1.copy()
    x2[:, 10:] = rng.standard_normal((1, 6, D))
    y1, y2 = M.short_conv(x1, w, b), M.short_conv(x2, w, b)
    np.testing.assert_array_equal(y1[:, :10], y2[:, :10])
    assert np.abs(y1[:, 10:] - y2[:, 10:]).max() > 1e-3
    s1, s2 = rng.standard_normal((1, 6, D)), rng.standard_normal((1, 10, D))
    yp = M.short_conv(np.concatenate([s1, s2], 1), w, b, cu_seqlens=[0, 6, 16])
    np.testing.assert_allclose(yp[:, :6], M.short_conv(s1, w, b), rtol=1e-15)
    np.testing.assert_allclose(yp[:, 6:], M.short_conv(s2, w, b), rtol=1e-15)
    dy = rng.standard_normal(yp.shape)
    dxp, dwp, dbp = M.short_conv_bwd(np.concatenate([s1, s2], 1), w, b, dy, cu_seqlens=[0, 6, 16])
    a = M.short_conv_bwd(s1, w, b, dy[:, :6])
    c = M.short_conv_bwd(s2, w, b, dy[:, 6:])
    np.testing.assert_allclose(dxp, np.concatenate([a[0], c[0]], 1), rtol=1e-13)
    np.testing.assert_allclose(dwp, a[1] + c[1], rtol=1e-13)
    np.testing.assert_allclose(dbp, a[2] + c[2], rtol=1e-13)


@pytest.mark.parametrize("T", [1, 2, 5, 9])
def test_decode_steps_continue_the_prefill(T):
    """prefill(x[:T]) -> final state; steps with x[T], x[T+1], ... reproduce prefill of the
    longer sequence at those positions (cache semantics of convolution.py:82-173)."""
    rng = np.random.Generator(np.random.PCG64(T))
    D, W = 5, 4
    w, b = rng.standard_normal((D, W)), rng.standard_normal(D)
    x = rng.standard_normal((2, T + 3, D))
    full = M.short_conv(x, w, b)
    cache = M.short_conv_final_state(x[:, :T], W)
    assert cache.shape == (2, D, W)
    for t in range(T, T + 3):
        y, cache = M.short_conv_step(x[:, t], cache, w, b)
        np.testing.assert_allclose(y, full[:, t], rtol=1e-13)
    np.testing.assert_allclose(cache, M.short_conv_final_state(x, W), rtol=0)
    # no cache: the step is the conv of a one-token sequence
    y0, c0 = M.short_conv_step(x[:, 0], None, w, b)
    assert c0 is None
    np.testing.assert_allclose(y0, M.short_conv(x[:, :1], w, b)[:, 0], rtol=1e-15)


def test_planted_mistakes_are_caught():
    rng = np.random.Generator(np.random.PCG64(9))
    D, W = 4, 3
    x, w = rng.standard_normal((1, 7, D)), rng.standard_normal((D, W))
    ref = _torch_conv(torch.tensor(x), torch.tensor(w), None, "silu").numpy()
    assert _rel(M.short_conv(x, w[:, ::-1].copy()), ref) > 1e-3      # taps reversed
    xx = rng.standard_normal((2, 3, 16))
    ref_n = F.rms_norm(torch.tensor(xx), (16,), eps=1e-5).numpy()
    summed = xx / np.sqrt((xx * xx).sum(-1, keepdims=True) + 1e-5)   # mean taken as sum
    assert _rel(M.rmsnorm_gated(xx, eps=1e-5), ref_n) < TOL and _rel(summed, ref_n) > 0.5
