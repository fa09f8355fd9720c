"""GLA and simple GLA beyond one kernel tile, and fp16 inputs, on MI355X against the float64
oracle.  K > 128 (and V > 128 in the dq / dk / dg stage) runs as equal slices of at most 128
on the strided entry points (tops_chunk_*_slice: pointers into the full tensors, no copies),
whose outputs add up in fp32 (the recurrence is separate per state entry).  fp16 inputs are
read by the kernels as fp16 (TOPS_F16) and split into exact bf16 hi / lo halves.
Shapes include the reference's simple-GLA K = 256 cases
(tests/ops/simple_gla/test_chunk_simple_gla_tpu.py:54, test_fused_chunk_simple_gla_tpu.py:53)
and its V = 256 state tests.  Tolerances (relative L2): fp32 1e-4; bf16 / fp16 2e-3.
"""
import numpy as np
import pytest
import torch

from oracle import gla as O
from oracle import simple_gla as S
from _gpu import to_dev, host, rel
from _inputs import gla_inputs, simple_gla_inputs, bf16_round

pytestmark = pytest.mark.gpu


def _seen(x, dt):
    if x is None:
        return None
    x = np.asarray(x, np.float32)
    if dt == torch.bfloat16:
        x = bf16_round(x)
    elif dt == torch.float16:
        x = x.astype(np.float16).astype(np.float32)
    return x.astype(np.float64)


def _lim(dt):
    return 1e-4 if dt == torch.float32 else 2e-3


DTS = [torch.float32, torch.bfloat16, torch.float16]
IDS = ["f32", "bf16", "f16"]

GLA = [
    dict(B=2, T=128, H=2, K=256, V=128, h0=True),
    dict(B=1, T=192, H=2, K=128, V=256),
    dict(B=1, T=130, H=1, K=192, V=192, h0=True),
    dict(B=1, T=300, H=2, K=256, V=64, cu=[0, 100, 101, 300], h0=True),
    dict(B=2, T=64, H=2, K=64, V=64),
]


def _gid(c):
    return f"B{c['B']}-T{c['T']}-H{c['H']}-K{c['K']}-V{c['V']}" + ("-varlen" if "cu" in c else "")


@pytest.mark.parametrize("dt", DTS, ids=IDS)
@pytest.mark.parametrize("c", GLA, ids=_gid)
def test_chunk_gla_sliced_and_fp16(c, dt, cuda_device):
    from tops.ops.gla import chunk_gla
    B, T, H, K, V = (c[x] for x in "BTHKV")
    cu = c.get("cu")
    n = B if cu is None else len(cu) - 1
    print(f"chunk_gla {_gid(c)} {dt}", flush=True)
    d = gla_inputs(B, T, H, K, V, seed=T + K + V, h0=c.get("h0", False), N=n, grads=True)
    q, k, v = (to_dev(d[x], dt, cuda_device).requires_grad_() for x in "qkv")
    g = to_dev(d["g"], torch.float32, cuda_device).requires_grad_()
    h0 = to_dev(d["h0"], torch.float32, cuda_device)
    if h0 is not None:
        h0.requires_grad_()
    o, ht = chunk_gla(q, k, v, g, initial_state=h0, output_final_state=True, cu_seqlens=cu)
    assert o.dtype == dt
    do = to_dev(d["do"], dt, cuda_device)
    torch.autograd.backward((o, ht), (do, to_dev(d["dht"], torch.float32, cuda_device)))
    sq, sk, sv, sdo = (_seen(d[x], dt) for x in ("q", "k", "v", "do"))
    ro, rht = O.chunk_gla(sq, sk, sv, d["g"], K ** -0.5, d["h0"], True, cu_seqlens=cu)
    rq, rk, rv, rg, rh0 = O.chunk_gla_bwd(sq, sk, sv, d["g"], K ** -0.5, d["h0"], sdo, d["dht"],
                                          cu_seqlens=cu)
    assert q.grad.dtype == dt and v.grad.dtype == dt
    errs = dict(o=rel(host(o), ro), ht=rel(host(ht), rht), dq=rel(host(q.grad), rq),
                dk=rel(host(k.grad), rk), dv=rel(host(v.grad), rv), dg=rel(host(g.grad), rg))
    if h0 is not None:
        errs["dh0"] = rel(host(h0.grad), rh0)
    print(" ".join(f"{n_}={e:.2e}" for n_, e in errs.items()))
    for n_, e in errs.items():
        assert e < _lim(dt), (n_, e)


def test_chunk_gla_fwd_bwd_states_roundtrip_sliced(cuda_device):
    """chunk_gla_fwd's h (assembled from K / V slices) fed back to chunk_gla_bwd gives the
    same gradients as recomputing it."""
    from tops.ops.gla import chunk_gla_bwd, chunk_gla_fwd
    B, T, H, K, V = 1, 128, 2, 256, 256
    d = gla_inputs(B, T, H, K, V, seed=9, h0=True, grads=True)
    f = lambda x: to_dev(x, torch.float32, cuda_device)
    q, k, v, g, h0, do, dht = (f(d[x]) for x in ("q", "k", "v", "g", "h0", "do", "dht"))
    _, _, h, ht, o = chunk_gla_fwd(q, k, v, g, None, None, K ** -0.5, h0, True)
    assert h.shape == (B, T // 64, H, K, V)
    rh, _ = O.chunk_fwd_h(d["k"], d["v"], gk=O.chunk_local_cumsum(d["g"], 64), h0=d["h0"], C=64)
    assert rel(host(h), rh) < 1e-4
    a = chunk_gla_bwd(q, k, v, g, None, None, K ** -0.5, h0, h, None, do, dht)
    b = chunk_gla_bwd(q, k, v, g, None, None, K ** -0.5, h0, None, None, do, dht)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


SIMPLE = [
    dict(B=2, T=64, H=4, K=256, V=128, gate="gamma"),
    dict(B=1, T=128, H=2, K=256, V=128, gate="g", h0=True),
    dict(B=1, T=128, H=2, K=128, V=256, gate="gamma", h0=True),
]


@pytest.mark.parametrize("dt", DTS, ids=IDS)
@pytest.mark.parametrize("c", SIMPLE, ids=lambda c: "{gate}-B{B}-T{T}-K{K}-V{V}".format(**c))
def test_chunk_simple_gla_sliced_and_fp16(c, dt, cuda_device):
    from tops.ops.simple_gla import chunk_simple_gla
    B, T, H, K, V = (c[x] for x in "BTHKV")
    print(f"simple {c} {dt}", flush=True)
    d = simple_gla_inputs(B, T, H, K, V, seed=T + K, h0=c.get("h0", False), grads=True)
    q, k, v = (to_dev(d[x], dt, cuda_device).requires_grad_() for x in "qkv")
    g = to_dev(d["g"], torch.float32, cuda_device).requires_grad_() if c["gate"] == "g" else None
    gg = to_dev(d["g_gamma"], torch.float32, cuda_device) if c["gate"] == "gamma" else None
    h0 = to_dev(d["h0"], torch.float32, cuda_device)
    if h0 is not None:
        h0.requires_grad_()
    o, ht = chunk_simple_gla(q, k, v, gg, initial_state=h0, output_final_state=True, g=g)
    assert o.dtype == dt
    do = to_dev(d["do"], dt, cuda_device)
    torch.autograd.backward((o, ht), (do, to_dev(d["dht"], torch.float32, cuda_device)))
    gs = d["g"] if c["gate"] == "g" else None
    gam = d["g_gamma"] if c["gate"] == "gamma" else None
    sq, sk, sv, sdo = (_seen(d[x], dt) for x in ("q", "k", "v", "do"))
    ro, rht = S.chunk_simple_gla(sq, sk, sv, g=gs, g_gamma=gam, initial_state=d["h0"],
                                 output_final_state=True)
    rq, rk, rv, rg, rh0 = S.chunk_simple_gla_bwd(sq, sk, sv, gs, gam, d["h0"], sdo, d["dht"],
                                                 K ** -0.5)
    errs = dict(o=rel(host(o), ro), ht=rel(host(ht), rht), dq=rel(host(q.grad), rq),
                dk=rel(host(k.grad), rk), dv=rel(host(v.grad), rv))
    if g is not None:
        errs["dg"] = rel(host(g.grad), rg)
    if h0 is not None:
        errs["dh0"] = rel(host(h0.grad), rh0)
    print(" ".join(f"{n_}={e:.2e}" for n_, e in errs.items()))
    for n_, e in errs.items():
        assert e < _lim(dt), (n_, e)


FR = [
    dict(B=1, T=40, H=2, K=256, V=64, gv=True, reverse=False),
    dict(B=2, T=33, H=1, K=192, V=32, gv=False, reverse=True),
    dict(B=1, T=50, H=2, K=256, V=64, gv=False, reverse=False),
]


@pytest.mark.parametrize("dt", DTS, ids=IDS)
@pytest.mark.parametrize("c", FR, ids=lambda c: "B{B}-T{T}-K{K}-V{V}-gv{gv}-rev{reverse}".format(**c))
def test_fused_recurrent_gla_wide_and_fp16(c, dt, cuda_device):
    from tops.ops.gla import fused_recurrent_gla
    B, T, H, K, V = (c[x] for x in "BTHKV")
    print(f"fused_recurrent {c} {dt}", flush=True)
    d = gla_inputs(B, T, H, K, V, seed=T * K, h0=True, grads=True)
    rng = np.random.default_rng(T)
    gvn = (np.log(1 / (1 + np.exp(-rng.standard_normal((B, T, H, V))))) / 16).astype(np.float32) \
        if c["gv"] else None
    q, k, v = (to_dev(d[x], dt, cuda_device).requires_grad_() for x in "qkv")
    gk = to_dev(d["g"], torch.float32, cuda_device).requires_grad_()
    gv = None if gvn is None else to_dev(gvn, torch.float32, cuda_device).requires_grad_()
    h0 = to_dev(d["h0"], torch.float32, cuda_device).requires_grad_()
    o, ht = fused_recurrent_gla(q, k, v, gk, gv, initial_state=h0, output_final_state=True,
                                reverse=c["reverse"])
    assert o.dtype == dt and ht.shape == (B, H, K, V)
    do = to_dev(d["do"], dt, cuda_device)
    torch.autograd.backward((o, ht), (do, to_dev(d["dht"], torch.float32, cuda_device)))
    sq, sk, sv, sdo = (_seen(d[x], dt) for x in ("q", "k", "v", "do"))
    ro, rht = O.fused_recurrent_gla(sq, sk, sv, d["g"], gvn, K ** -0.5, d["h0"], True,
                                    reverse=c["reverse"])
    r = O.fused_recurrent_bwd(sq, sk, sv, d["g"], gvn, ro, sdo, d["dht"], K ** -0.5, d["h0"],
                              reverse=c["reverse"])
    errs = dict(o=rel(host(o), ro), ht=rel(host(ht), rht), dq=rel(host(q.grad), r[0]),
                dk=rel(host(k.grad), r[1]), dv=rel(host(v.grad), r[2]), dgk=rel(host(gk.grad), r[3]),
                dh0=rel(host(h0.grad), r[5]))
    if gv is not None:
        errs["dgv"] = rel(host(gv.grad), r[4])
    print(" ".join(f"{n_}={e:.2e}" for n_, e in errs.items()))
    for n_, e in errs.items():
        assert e < _lim(dt), (n_, e)


def test_simple_gla_naive_mode_returns_float32(cuda_device):
    """simple_gla(mode='naive') goes through simple_gla_naive, whose output is float32 as the
    reference's (tops/ops/simple_gla/__init__.py:144-155, naive.py:69-100)."""
    from tops.ops.simple_gla import simple_gla
    d = simple_gla_inputs(1, 33, 2, 32, 16, seed=3, h0=True)
    q, k, v = (to_dev(d[x], torch.bfloat16, cuda_device) for x in "qkv")
    g = to_dev(d["g"], torch.float32, cuda_device)
    o, ht = simple_gla(q, k, v, g=g, initial_state=to_dev(d["h0"], torch.float32, cuda_device),
                       output_final_state=True, mode="naive")
    assert o.dtype == torch.float32 and ht.dtype == torch.float32
    sq, sk, sv = (_seen(d[x], torch.bfloat16) for x in "qkv")
    ro, rht = S.naive_simple_gla(sq, sk, sv, g=d["g"], initial_state=d["h0"],
                                 output_final_state=True)
    assert rel(host(o), ro) < 1e-4 and rel(host(ht), rht) < 1e-4


@pytest.mark.parametrize("K,V", [(128, 128), (64, 96), (256, 128)])
def test_fp16_entry_points_read_fp16(K, V, cuda_device):
    """The chunk entry points take fp16 tensors themselves (TOPS_F16): forward and both
    backward stages through the C ABI on fp16 inputs match the fp32 entry points run on the
    same (fp16-representable) values, up to the fp16 rounding of the stored outputs.  K = 256
    goes through the channel-slice entry points."""
    import tops._native as N
    from tops.ops._chunk_core import chunk_bwd, chunk_fwd
    from tops.utils import ChunkPlan
    B, T, H = 2, 150, 2
    d = gla_inputs(B, T, H, K, V, seed=K + V, h0=True, grads=True)
    f16 = lambda x: to_dev(x, torch.float16, cuda_device)
    q, k, v, do = (f16(d[x]) for x in ("q", "k", "v", "do"))
    q32, k32, v32, do32 = (x.float() for x in (q, k, v, do))
    g = to_dev(d["g"], torch.float32, cuda_device)
    h0 = to_dev(d["h0"], torch.float32, cuda_device)
    dht = to_dev(d["dht"], torch.float32, cuda_device)
    plan = ChunkPlan.get(B, T, None, cuda_device)
    gate = ("k", g)
    o, ht, hs = chunk_fwd(q, k, v, gate, h0, K ** -0.5, True, plan, True)
    o32, ht32, hs32 = chunk_fwd(q32, k32, v32, gate, h0, K ** -0.5, True, plan, True)
    assert o.dtype == torch.float16 and N.chunk_dtype_code(q.dtype) == N.TOPS_F16
    assert rel(host(o), host(o32)) < 1e-3
    assert rel(host(ht), host(ht32)) < 1e-5 and rel(host(hs), host(hs32)) < 1e-5
    a = chunk_bwd(q, k, v, gate, do, dht, hs, K ** -0.5, plan, True)
    b = chunk_bwd(q32, k32, v32, gate, do32, dht, hs32, K ** -0.5, plan, True)
    for name, x, y in zip(("dq", "dk", "dv", "dg", "dh0"), a, b):
        lim = 1e-3 if x.dtype == torch.float16 else 1e-5
        assert rel(host(x), host(y)) < lim, name
    assert a[0].dtype == a[1].dtype == a[2].dtype == torch.float16
