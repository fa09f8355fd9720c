"""chunk_gla on MI355X vs the float64 oracle (the reference's tops/cpu restated).

Cases mirror tests/ops/gla/test_pallas_chunk_gla.py:24-126 of the reference
(shapes, T = 1/3/odd, K != V, h0, custom scale, varlen incl. non-chunk-aligned
segments) plus the BASELINE configs.  Error metric: ||x - x_ref||_2 / ||x_ref||_2
with x_ref the fp64 oracle on exactly the (bf16-rounded) inputs the kernel saw.
Tolerance (stated by the north star): fp32 1e-4, bf16 2e-3.
"""
import numpy as np
import pytest
import torch

from oracle import gla as O
from _inputs import gla_inputs
from _gpu import to_dev, seen, host, rel, tol

pytestmark = pytest.mark.gpu

CASES = [
    dict(B=2, T=32, H=4, K=32, V=64, seed=42),
    dict(B=2, T=32, H=4, K=32, V=64, seed=13, h0=True),
    dict(B=1, T=128, H=2, K=64, V=128, seed=7),
    dict(B=2, T=32, H=4, K=16, V=128, seed=20),
    dict(B=2, T=32, H=4, K=128, V=16, seed=21),
    dict(B=1, T=1, H=2, K=32, V=64, seed=30),
    dict(B=1, T=3, H=2, K=32, V=64, seed=31),
    dict(B=2, T=37, H=4, K=16, V=32, seed=40),
    dict(B=1, T=100, H=2, K=32, V=64, seed=42, h0=True),
    dict(B=2, T=32, H=2, K=8, V=16, seed=71, h0=True),
    dict(B=2, T=32, H=4, K=32, V=64, seed=200, scale=0.1),
    dict(B=1, T=96, H=4, K=32, V=64, seed=10, cu=[0, 32, 64, 96]),
    dict(B=1, T=48, H=4, K=32, V=64, seed=18, cu=[0, 16, 48], h0=True),
    dict(B=1, T=50, H=2, K=16, V=32, seed=402, cu=[0, 13, 37, 50]),
    dict(B=1, T=300, H=2, K=64, V=64, seed=404, cu=[0, 20, 21, 200, 300], h0=True),
    dict(B=1, T=512, H=2, K=128, V=64, seed=352, h0=True),
    dict(B=2, T=512, H=4, K=64, V=64, seed=1001),            # BASELINE config 1 (fp32)
    dict(B=1, T=1024, H=2, K=128, V=128, seed=1003, h0=True),
    dict(B=2, T=200, H=3, K=128, V=192, seed=77, h0=True),   # V > 128 (3 V tiles)
]


def _id(c):
    return "-".join(f"{k}{v}" for k, v in c.items() if k not in ("seed",))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("cfg", CASES, ids=[_id(c) for c in CASES])
def test_chunk_gla_fwd(cfg, dtype, cuda_device):
    from tops.ops.gla import chunk_gla
    B, T, H, K, V = (cfg[x] for x in "BTHKV")
    cu = cfg.get("cu")
    n = len(cu) - 1 if cu else B
    d = gla_inputs(B, T, H, K, V, cfg["seed"], gate_div=1.0, h0=cfg.get("h0", False), N=n)
    scale = cfg.get("scale")
    q, k, v = (to_dev(d[x], dtype, cuda_device) for x in "qkv")
    g = to_dev(d["g"], torch.float32, cuda_device)
    h0 = to_dev(d["h0"], torch.float32, cuda_device)
    o, ht = chunk_gla(q, k, v, g, scale=scale, initial_state=h0, output_final_state=True,
                      cu_seqlens=cu)
    torch.cuda.synchronize()
    ro, rht = O.chunk_gla(seen(d["q"], dtype), seen(d["k"], dtype), seen(d["v"], dtype), d["g"],
                          scale=scale, initial_state=d["h0"], output_final_state=True,
                          cu_seqlens=cu, chunk_size=64)
    assert o.dtype == dtype and ht.dtype == torch.float32
    eo, eh = rel(host(o), ro), rel(host(ht), rht)
    print(f"rel o={eo:.2e} ht={eh:.2e}")
    assert eo < tol(dtype), eo
    assert eh < tol(dtype), eh


def test_no_final_state(cuda_device):
    from tops.ops.gla import chunk_gla
    d = gla_inputs(2, 32, 4, 32, 64, 210)
    q, k, v, g = (to_dev(d[x], torch.float32, cuda_device) for x in "qkvg")
    o, ht = chunk_gla(q, k, v, g, output_final_state=False)
    assert ht is None
    ro, _ = O.chunk_gla(d["q"], d["k"], d["v"], d["g"])
    assert rel(host(o), ro) < 1e-4


def test_state_split(cuda_device):
    from tops.ops.gla import chunk_gla
    d = gla_inputs(1, 40, 2, 16, 32, 77, gate_div=1.0)
    t = {x: to_dev(d[x], torch.float32, cuda_device) for x in "qkvg"}
    _, full = chunk_gla(t["q"], t["k"], t["v"], t["g"], output_final_state=True)
    _, s1 = chunk_gla(*(t[x][:, :20] for x in "qkvg"), output_final_state=True)
    _, s2 = chunk_gla(*(t[x][:, 20:] for x in "qkvg"), initial_state=s1, output_final_state=True)
    assert rel(host(s2), host(full)) < 1e-5


def test_large_gates_finite(cuda_device):
    """Gate cumsum reaching ~ -80 inside a chunk stays finite (midpoint stabilisation),
    as tests/ops/gla/test_exp_overflow_stabilization.py:62-217 requires."""
    from tops.ops.gla import chunk_gla
    rng = np.random.default_rng(5)
    B, T, H, K, V = 1, 256, 2, 32, 32
    d = gla_inputs(B, T, H, K, V, 5)
    d["g"] = -rng.uniform(0.0, 2.5, (B, T, H, K)).astype(np.float32)
    t = {x: to_dev(d[x], torch.float32, cuda_device) for x in "qkvg"}
    o, ht = chunk_gla(t["q"], t["k"], t["v"], t["g"], output_final_state=True)
    assert torch.isfinite(o).all() and torch.isfinite(ht).all()
    ro, rht = O.chunk_gla(d["q"], d["k"], d["v"], d["g"], output_final_state=True, chunk_size=64)
    assert rel(host(o), ro) < 1e-4


def _padded_oracle(d, C, cu, scale):
    """g_cumsum, A (full square) and h of the reference's padded layout, from the oracle's
    stage functions: per sequence padded to a multiple of C (chunk.py:1140-1148)."""
    from oracle.common import chunk_local_cumsum, chunk_fwd_h, pad_time
    T = d["q"].shape[1]
    bounds = [(0, T)] if cu is None else list(zip(cu[:-1], cu[1:]))
    gcs, As, hs = [], [], []
    for n, (a, b) in enumerate(bounds):
        q, k, v, g = (pad_time(d[x][:, a:b].astype(np.float64), C) for x in ("q", "k", "v", "g"))
        h0 = None if d["h0"] is None else (d["h0"] if cu is None else d["h0"][n:n + 1])
        gc = chunk_local_cumsum(g, C)
        gcs.append(gc)
        As.append(O.chunk_gla_fwd_intra_gk(q, k, gc, scale, C))
        hs.append(chunk_fwd_h(k, v, gk=gc, h0=h0, C=C)[0])
    return np.concatenate(gcs, 1), np.concatenate(As, 1), np.concatenate(hs, 1)


FWD_ORCH = [
    dict(B=2, T=100, H=2, K=32, V=64, C=64, h0=True, seed=41),
    dict(B=1, T=300, H=2, K=64, V=64, C=64, h0=True, seed=42, cu=[0, 13, 140, 141, 300]),
    dict(B=2, T=96, H=2, K=32, V=32, C=16, h0=False, seed=43),
    dict(B=1, T=200, H=2, K=64, V=64, C=32, h0=True, seed=44, cu=[0, 50, 200]),
]


@pytest.mark.parametrize("c", FWD_ORCH, ids=lambda c: "B{B}-T{T}-C{C}".format(**c) + ("-varlen" if "cu" in c else ""))
def test_chunk_gla_fwd_intermediates(c, cuda_device):
    """chunk_gla_fwd returns (g_cumsum, A, h, ht, o) as the reference (chunk.py:1103-1199);
    g_cumsum fed back instead of g (g = None) reproduces o, ht and the gradients."""
    from tops.ops.gla import chunk_gla_fwd, chunk_gla_bwd
    B, T, H, K, V, C = (c[x] for x in "BTHKVC")
    cu = c.get("cu")
    n = len(cu) - 1 if cu else B
    d = gla_inputs(B, T, H, K, V, c["seed"], gate_div=4.0, h0=c["h0"], N=n, grads=True)
    t = {x: to_dev(d[x], torch.float32, cuda_device) for x in ("q", "k", "v", "g", "h0", "do", "dht")}
    scale = K ** -0.5
    gc, A, h, ht, o = chunk_gla_fwd(t["q"], t["k"], t["v"], t["g"], None, None, scale, t["h0"],
                                    True, cu_seqlens=cu, chunk_size=C)
    torch.cuda.synchronize()
    rgc, rA, rh = _padded_oracle(d, C, cu, scale)
    ro, rht = O.chunk_gla(d["q"], d["k"], d["v"], d["g"], initial_state=d["h0"],
                          output_final_state=True, cu_seqlens=cu)
    assert gc.shape == rgc.shape and A.shape == rA.shape, (gc.shape, A.shape)
    assert h.shape == (1 if cu else B,) + rh.shape[1:], (h.shape, rh.shape)
    for name, a, b in (("g_cumsum", gc, rgc), ("A", A, rA), ("h", h, rh), ("ht", ht, rht), ("o", o, ro)):
        e = rel(host(a), b)
        assert e < 1e-4, (name, e)
    # the cumsum given back in place of g
    _, _, _, ht2, o2 = chunk_gla_fwd(t["q"], t["k"], t["v"], None, None, gc, scale, t["h0"], True,
                                     cu_seqlens=cu, chunk_size=C)
    assert rel(host(o2), ro) < 1e-4 and rel(host(ht2), rht) < 1e-4
    grads = chunk_gla_bwd(t["q"], t["k"], t["v"], None, None, gc, scale, t["h0"], h, A, t["do"],
                          t["dht"], cu_seqlens=cu, chunk_size=C)
    ref = O.chunk_gla_bwd(d["q"], d["k"], d["v"], d["g"], scale, d["h0"], d["do"], d["dht"],
                          cu_seqlens=cu)
    for name, a, b in zip(("dq", "dk", "dv", "dg", "dh0"), grads, ref):
        if a is None or b is None:
            continue
        e = rel(host(a), b)
        assert e < 1e-4, (name, e)


@pytest.mark.parametrize("form", ["none", "scalar", "head", "head_channel"])
def test_chunk_gla_constant_gates(form, cuda_device):
    """g = None with no g_gamma or with the reference's three g_gamma forms runs the constant
    [H, K] gate mode: forward, and the g_gamma gradient (the broadcast gate's gradient summed
    to g_gamma's shape, chunk.py:987-995), against the oracle on the broadcast gate."""
    from tops.ops.gla import chunk_gla
    B, T, H, K, V = 2, 150, 3, 64, 32
    d = gla_inputs(B, T, H, K, V, 45, h0=True, grads=True)
    rng = np.random.default_rng(46)
    shape = {"none": None, "scalar": (), "head": (1, 1, H, 1), "head_channel": (1, 1, H, K)}[form]
    gam = None if shape is None else (-np.abs(rng.standard_normal(shape)) * 0.2).astype(np.float32)
    q, k, v = (to_dev(d[x], torch.float32, cuda_device).requires_grad_() for x in "qkv")
    h0 = to_dev(d["h0"], torch.float32, cuda_device).requires_grad_()
    gg = None if gam is None else torch.tensor(gam, device=cuda_device, requires_grad=True)
    o, ht = chunk_gla(q, k, v, g_gamma=gg, initial_state=h0, output_final_state=True)
    torch.autograd.backward((o, ht), (to_dev(d["do"], torch.float32, cuda_device),
                                      to_dev(d["dht"], torch.float32, cuda_device)))
    gfull = np.zeros((B, T, H, K), np.float32) if gam is None else \
        np.broadcast_to(gam, (B, T, H, K)).astype(np.float32)
    ro, rht = O.chunk_gla(d["q"], d["k"], d["v"], gfull, initial_state=d["h0"], output_final_state=True)
    rq, rk, rv, rg, rh0 = O.chunk_gla_bwd(d["q"], d["k"], d["v"], gfull, K ** -0.5, d["h0"],
                                          d["do"], d["dht"])
    for name, a, b in (("o", o, ro), ("ht", ht, rht), ("dq", q.grad, rq), ("dk", k.grad, rk),
                       ("dv", v.grad, rv), ("dh0", h0.grad, rh0)):
        assert rel(host(a), b) < 1e-4, name
    if gg is not None:
        want = rg.sum(axis=(0, 1), keepdims=True)
        want = want.sum() if gam.ndim == 0 else want.sum(axis=tuple(i for i in range(4) if gam.shape[i] == 1 and want.shape[i] != 1), keepdims=True)
        assert gg.grad.shape == gg.shape
        assert rel(host(gg.grad).reshape(-1), np.asarray(want).reshape(-1)) < 1e-4


@pytest.mark.parametrize("form", ["none", "scalar", "head"])
def test_chunk_gla_constant_gate_per_head_bf16(form, cuda_device, monkeypatch):
    """bf16 chunk_gla with no gate, or a g_gamma shared by the K channels that needs no
    gradient, runs the one-decay-per-head mode (the value-side gate kernels: q and k stay
    exact): o, ht and dq, dk, dv, dh0 against the oracle on the broadcast gate."""
    from tops import _native as N
    from tops.ops.gla import chunk_gla
    names = []
    real = N.call
    monkeypatch.setattr(N, "call", lambda name, *a: (names.append(name), real(name, *a))[1])
    B, T, H, K, V = 1, 300, 2, 64, 64
    cu = [0, 13, 140, 141, 300]
    d = gla_inputs(B, T, H, K, V, 47, h0=True, N=len(cu) - 1, grads=True)
    rng = np.random.default_rng(48)
    shape = {"none": None, "scalar": (), "head": (1, 1, H, 1)}[form]
    gam = None if shape is None else (-np.abs(rng.standard_normal(shape)) * 0.3).astype(np.float32)
    bf = torch.bfloat16
    q, k, v = (to_dev(d[x], bf, cuda_device).requires_grad_() for x in "qkv")
    h0 = to_dev(d["h0"], torch.float32, cuda_device).requires_grad_()
    gg = None if gam is None else torch.tensor(gam, device=cuda_device)
    o, ht = chunk_gla(q, k, v, g_gamma=gg, initial_state=h0, output_final_state=True, cu_seqlens=cu)
    torch.autograd.backward((o, ht), (to_dev(d["do"], bf, cuda_device),
                                      to_dev(d["dht"], torch.float32, cuda_device)))
    torch.cuda.synchronize()
    # (training keeps fp16 checkpoints: the _c16 variant of the same entry point)
    assert any(n.startswith("tops_simple_gla_chunk_fwd") for n in names)
    assert not any(n.startswith("tops_gla_chunk_fwd_gamma") for n in names)
    gfull = np.zeros((B, T, H, K), np.float32) if gam is None else \
        np.broadcast_to(gam, (B, T, H, K)).astype(np.float32)
    sq, sk, sv, sdo = (seen(d[x], bf) for x in ("q", "k", "v", "do"))
    ro, rht = O.chunk_gla(sq, sk, sv, gfull, initial_state=d["h0"], output_final_state=True,
                          cu_seqlens=cu)
    rq, rk, rv, _, rh0 = O.chunk_gla_bwd(sq, sk, sv, gfull, K ** -0.5, d["h0"], sdo, d["dht"],
                                         cu_seqlens=cu)
    for name, a, b in (("o", o, ro), ("ht", ht, rht), ("dq", q.grad, rq), ("dk", k.grad, rk),
                       ("dv", v.grad, rv), ("dh0", h0.grad, rh0)):
        assert rel(host(a), b) < 2e-3, name
