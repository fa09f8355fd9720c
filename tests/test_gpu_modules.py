"""RMSNorm / FusedRMSNormGated / ShortConvolution on MI355X against the float64 oracle
(oracle/modules.py restating tops/modules/layernorm.py, fused_norm_gate.py and
convolution.py).

Covers fp32 and bf16 inputs, D from 64 to 2048 (not only multiples of 64), with and without
gate / affine weight / bias, 1 <= W <= 8 taps, SiLU and identity, packed varlen sequences
including one-token sequences, the final-state window, decode steps chained after a prefill
and the module-level decode switch (B*T == N); backward: dx, dg, the weight and bias
gradients (reduced over many workgroups, bit-identical across calls).
Tolerances (relative L2): fp32 results 2e-6, fp32 reductions 1e-5, results stored in bf16
4e-3 (one bf16 rounding).
"""
import numpy as np
import pytest
import torch

from oracle import modules as M
from _gpu import to_dev, seen, host, rel

pytestmark = pytest.mark.gpu

EW, RED, BF = 2e-6, 1e-5, 4e-3


def _lim(dtype):
    return EW if dtype == torch.float32 else BF


@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("gate,affine", [(False, True), (True, True), (True, False),
                                         (False, False)], ids=["norm", "gated", "gated-noaff",
                                                               "plain"])
@pytest.mark.parametrize("D", [64, 100, 128, 300, 1024, 2048])
def test_rmsnorm_gated(D, gate, affine, xdt, cuda_device):
    from tops.modules import rms_norm_gated
    rng = np.random.Generator(np.random.PCG64(D + 7 * gate + 3 * affine))
    x = rng.standard_normal((3, 37, D)).astype(np.float32)
    g = rng.standard_normal(x.shape).astype(np.float32) if gate else None
    w = (1 + 0.5 * rng.standard_normal(D)).astype(np.float32) if affine else None
    dy = rng.standard_normal(x.shape).astype(np.float32)
    print(f"rmsnorm D={D} gate={gate} affine={affine} {xdt}", flush=True)
    xt = to_dev(x, xdt, cuda_device).requires_grad_()
    gt = None if g is None else to_dev(g, xdt, cuda_device).requires_grad_()
    wt = None if w is None else to_dev(w, torch.float32, cuda_device).requires_grad_()
    y = rms_norm_gated(xt, gt, wt, eps=1e-5)
    assert y.dtype == xdt
    y.backward(to_dev(dy, xdt, cuda_device))
    sx, sg, sdy = seen(x, xdt), seen(g, xdt), seen(dy, xdt)
    ry = M.rmsnorm_gated(sx, sg, w, eps=1e-5)
    rdx, rdg, rdw = M.rmsnorm_gated_bwd(sx, sg, w, sdy, eps=1e-5)
    e = dict(y=rel(host(y), ry), dx=rel(host(xt.grad), rdx))
    if gate:
        e["dg"] = rel(host(gt.grad), rdg)
    if affine:
        e["dw"] = rel(host(wt.grad), rdw)
    print(" ".join(f"{k}={v:.2e}" for k, v in e.items()))
    for k, v in e.items():
        assert v < (RED if k == "dw" else _lim(xdt) if k != "dx" or xdt != torch.float32 else 1e-5), (k, v)


def test_norm_modules_and_deterministic_weight_grad(cuda_device):
    from tops.modules import FusedRMSNormGated, RMSNorm
    rng = np.random.Generator(np.random.PCG64(5))
    D = 128
    x = rng.standard_normal((8, 1250, D)).astype(np.float32)      # 10000 rows
    g = rng.standard_normal(x.shape).astype(np.float32)
    dy = rng.standard_normal(x.shape).astype(np.float32)
    fn = FusedRMSNormGated(D, eps=1e-5).to(cuda_device)
    nm = RMSNorm(D, eps=1e-6).to(cuda_device)
    with torch.no_grad():
        fn.weight.copy_(to_dev(1 + 0.3 * rng.standard_normal(D), torch.float32, cuda_device))
        nm.weight.copy_(fn.weight)
    xt, gt = to_dev(x, torch.float32, cuda_device), to_dev(g, torch.float32, cuda_device)
    dyt = to_dev(dy, torch.float32, cuda_device)
    w = host(fn.weight)
    grads = []
    for _ in range(2):
        fn.zero_grad()
        fn(xt, gt).backward(dyt)
        grads.append(fn.weight.grad.clone())
    assert torch.equal(grads[0], grads[1])
    rdw = M.rmsnorm_gated_bwd(x, g, w, dy, eps=1e-5)[2]
    assert rel(host(grads[0]), rdw) < RED
    y = nm(xt)
    assert rel(host(y), M.rmsnorm_gated(x, None, w, eps=1e-6)) < EW


CONV_CASES = [
    dict(B=2, T=300, D=300, W=4, bias=True, act="silu"),
    dict(B=1, T=1, D=64, W=4, bias=True, act="silu", module=False),
    dict(B=3, T=17, D=40, W=1, bias=False, act=None),
    dict(B=2, T=129, D=512, W=3, bias=True, act=None),
    dict(B=1, T=600, D=96, W=8, bias=True, act="silu", cu=[0, 1, 2, 300, 301, 600]),
    dict(B=1, T=200, D=256, W=5, bias=False, act="swish", cu=[0, 7, 200]),
    dict(B=2, T=5000, D=128, W=4, bias=True, act="silu"),
    # odd D (one column per lane, forward and backward) and D = 2 mod 4 (two-column lanes,
    # a half-empty last lane pair), W = 3 and 8, varlen with short sequences, and runs long
    # enough for both the interior and the edge walks of the backward
    dict(B=2, T=1000, D=301, W=3, bias=True, act="silu"),
    dict(B=1, T=700, D=301, W=8, bias=False, act=None, cu=[0, 1, 5, 350, 700]),
    dict(B=2, T=777, D=302, W=4, bias=True, act="silu"),
    dict(B=1, T=520, D=302, W=8, bias=True, act="silu", cu=[0, 3, 4, 260, 520]),
    dict(B=1, T=2049, D=302, W=3, bias=False, act="silu", cu=[0, 2, 2049]),
]


def _cid(c):
    s = f"B{c['B']}-T{c['T']}-D{c['D']}-W{c['W']}-{'b' if c['bias'] else 'nb'}-{c['act']}"
    return s + ("-varlen" if "cu" in c else "")


@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("cfg", CONV_CASES, ids=_cid)
def test_short_conv_fwd_bwd(cfg, xdt, cuda_device):
    from tops.modules import short_conv
    B, T, D, W = (cfg[k] for k in "BTDW")
    cu = cfg.get("cu")
    print(f"conv {_cid(cfg)} {xdt}", flush=True)
    rng = np.random.Generator(np.random.PCG64(T + D + W))
    x = rng.standard_normal((B, T, D)).astype(np.float32)
    w = (rng.standard_normal((D, W)) / np.sqrt(W)).astype(np.float32)
    b = rng.standard_normal(D).astype(np.float32) if cfg["bias"] else None
    dy = rng.standard_normal((B, T, D)).astype(np.float32)
    xt = to_dev(x, xdt, cuda_device).requires_grad_()
    wt = to_dev(w.reshape(D, 1, W), torch.float32, cuda_device).requires_grad_()
    bt = None if b is None else to_dev(b, torch.float32, cuda_device).requires_grad_()
    y, fs = short_conv(xt, wt, bt, cfg["act"], cu, output_final_state=True)
    assert y.dtype == torch.float32 and fs.dtype == xdt
    y.backward(to_dev(dy, torch.float32, cuda_device))
    sx = seen(x, xdt)
    ry = M.short_conv(sx, w, b, cfg["act"], cu)
    rdx, rdw, rdb = M.short_conv_bwd(sx, w, b, dy, cfg["act"], cu)
    e = dict(y=rel(host(y), ry), fs=rel(host(fs), M.short_conv_final_state(sx, W, cu)),
             dx=rel(host(xt.grad), rdx), dw=rel(host(wt.grad).reshape(D, W), rdw))
    if b is not None:
        e["db"] = rel(host(bt.grad), rdb)
    print(" ".join(f"{k}={v:.2e}" for k, v in e.items()))
    assert e["y"] < EW and e["fs"] == 0.0
    assert e["dx"] < (RED if xdt == torch.float32 else BF)
    assert e["dw"] < RED and e.get("db", 0.0) < RED


def test_short_conv_module_decode_continues_prefill(cuda_device):
    """Prefill with output_final_state, then decode steps through the module (B*T == N) and
    through step(): each step equals the prefill of the longer sequence at that position."""
    from tops.modules import ShortConvolution
    rng = np.random.Generator(np.random.PCG64(17))
    B, T, D, W = 2, 9, 48, 4
    conv = ShortConvolution(D, W, bias=True, activation="silu").to(cuda_device)
    w = host(conv.weight).reshape(D, W)
    b = host(conv.bias)
    x = rng.standard_normal((B, T + 3, D)).astype(np.float32)
    full = M.short_conv(x, w, b, "silu")
    xt = to_dev(x, torch.float32, cuda_device)
    y, cache = conv(xt[:, :T], output_final_state=True)
    assert cache.shape == (B, D, W)
    assert rel(host(y), full[:, :T]) < EW
    for t in range(T, T + 3):
        yt, cache = conv(xt[:, t:t + 1], cache=cache, output_final_state=True)
        assert yt.shape == (B, 1, D)
        assert rel(host(yt)[:, 0], full[:, t]) < EW
    assert rel(host(cache), M.short_conv_final_state(x, W)) == 0.0
    # varlen decode: one token per sequence, [1, N, D]
    x1 = rng.standard_normal((1, 3, D)).astype(np.float32)
    c0 = rng.standard_normal((3, D, W)).astype(np.float32)
    ys, cs = conv(to_dev(x1, torch.float32, cuda_device), cache=to_dev(c0, torch.float32, cuda_device),
                  cu_seqlens=[0, 1, 2, 3])
    ry, rc = M.short_conv_step(x1[0], c0, w, b, "silu")
    assert rel(host(ys)[0], ry) < EW and rel(host(cs), rc) == 0.0
    # no cache and no final state: y = act(x w[-1] + b), cache stays None
    y0, c0n = conv.step(to_dev(x1, torch.float32, cuda_device)[:, :1], None)
    assert c0n is None
    assert rel(host(y0)[:, 0], M.short_conv_step(x1[:, 0], None, w, b, "silu")[0]) < EW
