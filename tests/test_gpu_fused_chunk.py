"""fused_chunk_gla and fused_chunk_simple_gla on MI355X against the float64 oracle.

fused_chunk_gla (tops/ops/gla/fused_chunk.py:4-30) is the reference's alias of chunk_gla;
fused_chunk_simple_gla (tops/ops/simple_gla/fused_chunk.py:503-555) is a custom_vjp op over a
per-head g_gamma with o / final state in q.dtype and dq / dk / dv / dh0 in dO's dtype.  Both
are compared with the oracle (oracle/gla.py, oracle/simple_gla.py) forward and backward,
never with the chunk ops they share kernels with.  Shapes: the reference's
tests/ops/simple_gla/test_fused_chunk_simple_gla_tpu.py FWD / BWD cases (bf16,
g_gamma = -|N(0,1)| / 2 per head, T = chunk multiples and chunk_size 128) at full or reduced
size, and chunk_gla-shaped cases for the GLA alias (ragged T, varlen, h0).
Tolerance: relative L2, fp32 1e-4, bf16 2e-3; an output the op returns in bf16 (o, the
final state and dh0 of fused_chunk_simple_gla) is compared with the oracle rounded to bf16.
"""
import numpy as np
import pytest
import torch

from oracle import gla as O
from oracle import simple_gla as S
from _inputs import gla_inputs
from _gpu import to_dev, seen, host, rel, tol, out_bound

pytestmark = pytest.mark.gpu

GLA = [
    dict(B=2, T=64, H=2, K=32, V=64, seed=21),
    dict(B=1, T=100, H=3, K=64, V=64, seed=22, h0=True),
    dict(B=2, T=130, H=2, K=128, V=128, seed=23, h0=True),
    dict(B=1, T=160, H=2, K=32, V=64, seed=24, h0=True, cu=[0, 10, 64, 65, 160]),
]


def _gid(c):
    return "B{B}-T{T}-H{H}-K{K}-V{V}".format(**c) + ("-h0" if c.get("h0") else "") + \
        ("-varlen" if "cu" in c else "")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("c", GLA, ids=_gid)
def test_fused_chunk_gla(c, dtype, cuda_device):
    from tops.ops.gla import fused_chunk_gla
    B, T, H, K, V = (c[x] for x in "BTHKV")
    cu = c.get("cu")
    n = len(cu) - 1 if cu else B
    d = gla_inputs(B, T, H, K, V, c["seed"], gate_div=4.0, h0=c.get("h0", False), N=n, grads=True)
    print(f"fused_chunk_gla {_gid(c)} {dtype}", flush=True)
    q, k, v = (to_dev(d[x], dtype, cuda_device).requires_grad_() for x in "qkv")
    g = to_dev(d["g"], torch.float32, cuda_device).requires_grad_()
    h0 = to_dev(d["h0"], torch.float32, cuda_device)
    if h0 is not None:
        h0.requires_grad_()
    o, ht = fused_chunk_gla(q, k, v, g, initial_state=h0, output_final_state=True, cu_seqlens=cu)
    assert o.dtype == dtype and ht.dtype == torch.float32
    torch.autograd.backward((o, ht), (to_dev(d["do"], dtype, cuda_device),
                                      to_dev(d["dht"], torch.float32, cuda_device)))
    torch.cuda.synchronize()
    sq, sk, sv, sdo = (seen(d[x], dtype) for x in ("q", "k", "v", "do"))
    ro, rht = O.fused_chunk_gla(sq, sk, sv, d["g"], initial_state=d["h0"], output_final_state=True,
                                cu_seqlens=cu)
    ref = O.chunk_gla_bwd(sq, sk, sv, d["g"], K ** -0.5, d["h0"], sdo, d["dht"], cu_seqlens=cu)
    got = [o, ht, q.grad, k.grad, v.grad, g.grad] + ([h0.grad] if h0 is not None else [])
    want = [ro, rht] + list(ref[:4]) + ([ref[4]] if h0 is not None else [])
    for name, a, b in zip(("o", "ht", "dq", "dk", "dv", "dg", "dh0"), got, want):
        e = rel(host(a), b)
        assert e < tol(dtype), (name, e)


SIMPLE = [   # reference FWD / BWD cases (test_fused_chunk_simple_gla_tpu.py:40-75, 199-)
    dict(B=2, T=64, H=4, K=128, V=128, seed=150),
    dict(B=2, T=128, H=4, K=128, V=128, seed=151),
    dict(B=2, T=64, H=4, K=128, V=128, seed=152, h0=True),
    dict(B=1, T=256, H=2, K=128, V=128, seed=161, h0=True),
    dict(B=2, T=64, H=1, K=128, V=128, seed=162),
    dict(B=1, T=64, H=2, K=128, V=256, seed=154),
    dict(B=2, T=64, H=4, K=256, V=128, seed=163),
    dict(B=8, T=64, H=4, K=128, V=128, seed=165),
    dict(B=2, T=64, H=4, K=128, V=128, seed=201, scale=0.1, h0=True),
    dict(B=2, T=512, H=16, K=128, V=128, seed=304, h0=True),      # T 4096 in the reference
    dict(B=1, T=256, H=2, K=128, V=128, seed=800, chunk_size=128),
    dict(B=2, T=100, H=2, K=64, V=32, seed=900, h0=True),          # ragged T (padded there)
]


def _sid(c):
    s = "B{B}-T{T}-H{H}-K{K}-V{V}".format(**c)
    for key in ("h0", "scale", "chunk_size"):
        if key in c:
            s += f"-{key}{c[key] if key != 'h0' else ''}"
    return s


def _simple_inputs(c):
    B, T, H, K, V = (c[x] for x in "BTHKV")
    rng = np.random.Generator(np.random.PCG64(c["seed"]))
    d = dict(q=rng.standard_normal((B, T, H, K)).astype(np.float32),
             k=rng.standard_normal((B, T, H, K)).astype(np.float32),
             v=rng.standard_normal((B, T, H, V)).astype(np.float32),
             g_gamma=(-np.abs(rng.standard_normal(H)) * 0.5).astype(np.float32),
             do=rng.standard_normal((B, T, H, V)).astype(np.float32),
             dht=(0.1 * rng.standard_normal((B, H, K, V))).astype(np.float32))
    d["h0"] = rng.standard_normal((B, H, K, V)).astype(np.float32) if c.get("h0") else None
    return d


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("c", SIMPLE, ids=_sid)
def test_fused_chunk_simple_gla(c, dtype, cuda_device):
    from tops.ops.simple_gla import fused_chunk_simple_gla
    K = c["K"]
    d = _simple_inputs(c)
    print(f"fused_chunk_simple_gla {_sid(c)} {dtype}", flush=True)
    q, k, v = (to_dev(d[x], dtype, cuda_device).requires_grad_() for x in "qkv")
    gg = torch.tensor(d["g_gamma"], device=cuda_device, requires_grad=True)
    h0 = to_dev(d["h0"], dtype, cuda_device)
    if h0 is not None:
        h0.requires_grad_()
    scale = c.get("scale")
    o, ht = fused_chunk_simple_gla(q, k, v, gg, initial_state=h0, scale=scale,
                                   output_final_state=True, chunk_size=c.get("chunk_size", 64))
    assert o.dtype == dtype and ht.dtype == dtype
    do, dht = to_dev(d["do"], dtype, cuda_device), to_dev(d["dht"], dtype, cuda_device)
    torch.autograd.backward((o, ht), (do, dht))
    torch.cuda.synchronize()
    assert q.grad.dtype == dtype and (h0 is None or h0.grad.dtype == dtype)
    assert torch.count_nonzero(gg.grad) == 0          # g_gamma is a fixed decay (zero cotangent)
    sq, sk, sv, sdo, sdht = (seen(d[x], dtype) for x in ("q", "k", "v", "do", "dht"))
    sh0 = seen(d["h0"], dtype)
    sc = K ** -0.5 if scale is None else scale
    ro, rht = S.chunk_simple_gla(sq, sk, sv, g_gamma=d["g_gamma"], scale=sc, initial_state=sh0,
                                 output_final_state=True)
    rq, rk, rv, _, rh0 = S.chunk_simple_gla_bwd(sq, sk, sv, None, d["g_gamma"], sh0, sdo, sdht, sc)

    # every output (stored in the op's dtype) against the unrounded oracle
    checks = [("o", o, ro), ("ht", ht, rht), ("dq", q.grad, rq), ("dk", k.grad, rk),
              ("dv", v.grad, rv)]
    if h0 is not None:
        checks.append(("dh0", h0.grad, rh0))
    for name, a, b in checks:
        e = rel(host(a), b)
        print(f"{name} {e:.2e}")
        assert e < out_bound(b, dtype, dtype), (name, e)


def test_fused_chunk_simple_gla_no_grad_path(cuda_device):
    """Inference (no input needs a gradient): no checkpoints are kept; the output matches the
    oracle."""
    from tops.ops.simple_gla import fused_chunk_simple_gla
    c = dict(B=1, T=192, H=2, K=64, V=64, seed=31, h0=True)
    d = _simple_inputs(c)
    q, k, v = (to_dev(d[x], torch.float32, cuda_device) for x in "qkv")
    with torch.no_grad():
        o, ht = fused_chunk_simple_gla(q, k, v, torch.tensor(d["g_gamma"], device=cuda_device),
                                       initial_state=to_dev(d["h0"], torch.float32, cuda_device),
                                       output_final_state=True)
    ro, rht = S.chunk_simple_gla(d["q"], d["k"], d["v"], g_gamma=d["g_gamma"], initial_state=d["h0"],
                                 output_final_state=True)
    assert rel(host(o), ro) < 1e-4 and rel(host(ht), rht) < 1e-4
