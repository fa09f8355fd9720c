"""chunk_gla backward on MI355X vs the float64 oracle (tops/cpu/ops/gla/chunk.py:469-640).

Gradients of L = sum(o * do) + sum(ht * dht) taken through torch autograd of
tops.ops.gla.chunk_gla (the HIP forward + fused HIP backward), compared with the
oracle's chunk_gla_bwd on the same (bf16-rounded) inputs.  Cases mirror the
reference's backward suites (tests/ops/gla/test_pallas_chunk_bwd.py:20-80: ragged T,
varlen with non-chunk-aligned segments, h0) plus BASELINE config 3 at reduced T.
Tolerance: fp32 1e-4, bf16 2e-3 (relative L2) on every gradient.
"""
import numpy as np
import pytest
import torch

from oracle import gla as O
from _inputs import gla_inputs
from _gpu import to_dev, seen, host, rel, tol

pytestmark = pytest.mark.gpu

CASES = [
    dict(B=2, T=64, H=2, K=32, V=32, seed=1),
    dict(B=1, T=37, H=2, K=16, V=32, seed=2, h0=True),
    dict(B=2, T=130, H=3, K=64, V=64, seed=3, h0=True),
    dict(B=1, T=1, H=2, K=32, V=64, seed=4, h0=True),
    dict(B=2, T=100, H=2, K=128, V=128, seed=5, h0=True),
    dict(B=1, T=256, H=2, K=128, V=64, seed=6),
    dict(B=1, T=200, H=2, K=64, V=128, seed=7, h0=True, scale=0.1),
    dict(B=2, T=96, H=2, K=8, V=16, seed=8, h0=True),
    dict(B=1, T=160, H=2, K=32, V=64, seed=9, cu=[0, 10, 64, 65, 160], h0=True),
    dict(B=1, T=300, H=2, K=128, V=128, seed=10, cu=[0, 100, 300]),
    dict(B=2, T=512, H=4, K=128, V=128, seed=1003, h0=True),   # config-3 shape, short T
]


def _id(c):
    return "-".join(f"{k}{v}" for k, v in c.items() if k != "seed")


def _run(cfg, dtype, device, dht=True):
    from tops.ops.gla import chunk_gla
    B, T, H, K, V = (cfg[x] for x in "BTHKV")
    cu = cfg.get("cu")
    n = len(cu) - 1 if cu else B
    d = gla_inputs(B, T, H, K, V, cfg["seed"], gate_div=1.0, h0=cfg.get("h0", False), N=n,
                   grads=True)
    scale = cfg.get("scale")
    q, k, v = (to_dev(d[x], dtype, device).requires_grad_() for x in "qkv")
    g = to_dev(d["g"], torch.float32, device).requires_grad_()
    h0 = to_dev(d["h0"], torch.float32, device)
    if h0 is not None:
        h0.requires_grad_()
    o, ht = chunk_gla(q, k, v, g, scale=scale, initial_state=h0, output_final_state=True,
                      cu_seqlens=cu)
    do = to_dev(d["do"], dtype, device)
    dht_t = to_dev(d["dht"], torch.float32, device) if dht else None
    loss = (o.float() * do.float()).sum()
    if dht:
        loss = loss + (ht * dht_t).sum()
    loss.backward()
    torch.cuda.synchronize()
    K_ = K
    ref = O.chunk_gla_bwd(seen(d["q"], dtype), seen(d["k"], dtype), seen(d["v"], dtype), d["g"],
                          K_ ** -0.5 if scale is None else scale, d["h0"], seen(d["do"], dtype),
                          d["dht"] if dht else None, chunk_size=64, cu_seqlens=cu)
    got = dict(dq=q.grad, dk=k.grad, dv=v.grad, dg=g.grad,
               dh0=None if h0 is None else h0.grad)
    return got, dict(zip(("dq", "dk", "dv", "dg", "dh0"), ref))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("cfg", CASES, ids=[_id(c) for c in CASES])
def test_chunk_gla_bwd(cfg, dtype, cuda_device):
    got, ref = _run(cfg, dtype, cuda_device)
    assert got["dq"].dtype == dtype and got["dk"].dtype == dtype and got["dv"].dtype == dtype
    assert got["dg"].dtype == torch.float32
    errs = {}
    for name in ("dq", "dk", "dv", "dg", "dh0"):
        if got[name] is None:
            continue
        errs[name] = rel(host(got[name]), ref[name])
    print(" ".join(f"{k}={v:.2e}" for k, v in errs.items()))
    for name, e in errs.items():
        assert e < tol(dtype), (name, e)


def test_chunk_gla_bwd_no_dht(cuda_device):
    got, ref = _run(dict(B=1, T=128, H=2, K=64, V=64, seed=11, h0=True), torch.float32,
                    cuda_device, dht=False)
    for name in ("dq", "dk", "dv", "dg", "dh0"):
        assert rel(host(got[name]), ref[name]) < 1e-4, name


def test_chunk_gla_bwd_orchestrator(cuda_device):
    """tops.ops.gla.chunk_gla_bwd (explicit orchestrator API) with recomputed states."""
    from tops.ops.gla import chunk_gla_bwd
    B, T, H, K, V = 1, 150, 2, 32, 32
    d = gla_inputs(B, T, H, K, V, 12, gate_div=1.0, h0=True, grads=True)
    t = {x: to_dev(d[x], torch.float32, cuda_device) for x in ("q", "k", "v", "g", "h0", "do", "dht")}
    dq, dk, dv, dg, dh0 = chunk_gla_bwd(t["q"], t["k"], t["v"], t["g"], None, None, K ** -0.5,
                                        t["h0"], None, None, t["do"], t["dht"])
    ref = O.chunk_gla_bwd(d["q"], d["k"], d["v"], d["g"], K ** -0.5, d["h0"], d["do"], d["dht"])
    for x, r in zip((dq, dk, dv, dg, dh0), ref):
        assert rel(host(x), r) < 1e-4


def test_g_gamma_gradient_reduces(cuda_device):
    """chunk_gla with g_gamma: dg is the broadcast-sum of the per-channel dg
    (tops/ops/gla/chunk.py:987-995)."""
    from tops.ops.gla import chunk_gla
    B, T, H, K, V = 1, 70, 2, 16, 16
    d = gla_inputs(B, T, H, K, V, 13, grads=True)
    gam = -np.abs(np.random.default_rng(0).standard_normal((H, K))).astype(np.float32) * 0.1
    q, k, v = (to_dev(d[x], torch.float32, cuda_device).requires_grad_() for x in "qkv")
    gg = torch.tensor(gam, device=cuda_device, requires_grad=True)
    o, _ = chunk_gla(q, k, v, g_gamma=gg)
    (o * to_dev(d["do"], torch.float32, cuda_device)).sum().backward()
    gfull = np.broadcast_to(gam, (B, T, H, K))
    ro, _ = O.chunk_gla(d["q"], d["k"], d["v"], gfull, chunk_size=64)
    assert rel(host(o), ro) < 1e-4
    ref = O.chunk_gla_bwd(d["q"], d["k"], d["v"], gfull, K ** -0.5, None, d["do"], None)
    assert rel(host(gg.grad), ref[3].sum(axis=(0, 1))) < 1e-4


def test_many_sequences(cuda_device):
    """300 varlen sequences of 1..40 tokens (more than the sweeps' in-kernel longest-first
    ranking covers): forward and backward against the oracle."""
    from tops.ops.gla import chunk_gla
    rng = np.random.default_rng(300)
    lens = rng.integers(1, 41, size=300)
    cu = [0] + [int(x) for x in np.cumsum(lens)]
    B, T, H, K, V = 1, cu[-1], 1, 32, 32
    d = gla_inputs(B, T, H, K, V, 300, gate_div=4.0, h0=True, N=300, grads=True)
    q, k, v = (to_dev(d[x], torch.float32, cuda_device).requires_grad_() for x in "qkv")
    g = to_dev(d["g"], torch.float32, cuda_device).requires_grad_()
    h0 = to_dev(d["h0"], torch.float32, cuda_device).requires_grad_()
    o, ht = chunk_gla(q, k, v, g, initial_state=h0, output_final_state=True, cu_seqlens=cu)
    torch.autograd.backward((o, ht), (to_dev(d["do"], torch.float32, cuda_device),
                                      to_dev(d["dht"], torch.float32, cuda_device)))
    ro, rht = O.chunk_gla(d["q"], d["k"], d["v"], d["g"], initial_state=d["h0"],
                          output_final_state=True, cu_seqlens=cu)
    ref = O.chunk_gla_bwd(d["q"], d["k"], d["v"], d["g"], K ** -0.5, d["h0"], d["do"], d["dht"],
                          chunk_size=64, cu_seqlens=cu)
    got = [o, ht, q.grad, k.grad, v.grad, g.grad, h0.grad]
    want = [ro, rht] + list(ref)
    for name, a, b in zip(("o", "ht", "dq", "dk", "dv", "dg", "dh0"), got, want):
        assert rel(host(a), b) < 1e-4, name


@pytest.mark.parametrize("cu", [[0, 0, 64, 64], [0, 50, 50, 130, 130], [0, 0, 0, 37]],
                         ids=["empty-first-last", "empty-middle-last", "two-empty-first"])
def test_empty_sequences(cu, cuda_device):
    """Zero-length sequences (0 chunks, tops/utils.py:71-90): their final state is h0 and their
    dh0 is dht; the other sequences match the oracle run on them alone."""
    from tops.ops.gla import chunk_gla
    lens = np.diff(cu)
    n, T, H, K, V = len(lens), cu[-1], 2, 64, 64
    d = gla_inputs(1, T, H, K, V, 77, gate_div=4.0, h0=True, N=n, grads=True)
    q, k, v = (to_dev(d[x], torch.float32, cuda_device).requires_grad_() for x in "qkv")
    g = to_dev(d["g"], torch.float32, cuda_device).requires_grad_()
    h0 = to_dev(d["h0"], torch.float32, cuda_device).requires_grad_()
    print(f"empty-sequence case cu={cu}", flush=True)
    o, ht = chunk_gla(q, k, v, g, initial_state=h0, output_final_state=True, cu_seqlens=cu)
    torch.autograd.backward((o, ht), (to_dev(d["do"], torch.float32, cuda_device),
                                      to_dev(d["dht"], torch.float32, cuda_device)))
    torch.cuda.synchronize()
    keep = [i for i in range(n) if lens[i] > 0]
    cu_ne = [0] + [int(x) for x in np.cumsum(lens[keep])]
    ro, rht = O.chunk_gla(d["q"], d["k"], d["v"], d["g"], initial_state=d["h0"][keep],
                          output_final_state=True, cu_seqlens=cu_ne)
    rq, rk, rv, rg, rh0 = O.chunk_gla_bwd(d["q"], d["k"], d["v"], d["g"], K ** -0.5,
                                          d["h0"][keep], d["do"], d["dht"][keep], cu_seqlens=cu_ne)
    for name, a, b in (("o", o, ro), ("dq", q.grad, rq), ("dk", k.grad, rk), ("dv", v.grad, rv),
                       ("dg", g.grad, rg)):
        assert rel(host(a), b) < 1e-4, name
    want_ht, want_dh0 = d["h0"].astype(np.float64).copy(), d["dht"].astype(np.float64).copy()
    want_ht[keep], want_dh0[keep] = rht, rh0
    assert rel(host(ht), want_ht) < 1e-4
    assert rel(host(h0.grad), want_dh0) < 1e-4
