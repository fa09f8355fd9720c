"""The reference's own chunk_gla test shapes (tests/ops/gla/test_pallas_chunk_gla.py:26-86
and test_pallas_chunk_gla_g_gamma.py:60-74), run through tops.ops.gla.chunk_gla (forward
and autograd backward) on MI355X against the float64 oracle: tiny and ragged T, T = 1,
K / V from 8 to 128, custom scale, h0, chunk-aligned and chunk-crossing varlen, and the
three g_gamma forms (scalar, per head (1,1,H,1), per head and channel (1,1,H,K)) whose
gradient is the broadcast gate's gradient summed to g_gamma's shape.
Tolerances (relative L2 against the unrounded float64 oracle): fp32 1e-4, bf16 2e-3; a bf16
output of a few dozen elements, whose correctly rounded value alone can miss 2e-3, gets that
rounding floor plus 2.5e-4 (_gpu.out_bound).
"""
import numpy as np
import pytest
import torch

from oracle import gla as O
from _gpu import to_dev, seen, host, rel, out_bound
from _inputs import gla_inputs

pytestmark = pytest.mark.gpu

REF = [
    dict(B=2, T=32, H=4, K=32, V=64), dict(B=2, T=32, H=4, K=32, V=64, h0=True),
    dict(B=1, T=128, H=2, K=64, V=128), dict(B=2, T=32, H=1, K=32, V=64),
    dict(B=2, T=32, H=4, K=16, V=128), dict(B=2, T=32, H=4, K=128, V=16),
    dict(B=1, T=1, H=2, K=32, V=64), dict(B=1, T=3, H=2, K=32, V=64),
    dict(B=2, T=37, H=4, K=16, V=32), dict(B=1, T=50, H=2, K=32, V=64),
    dict(B=1, T=100, H=2, K=32, V=64, h0=True), dict(B=8, T=32, H=4, K=32, V=64),
    dict(B=1, T=64, H=16, K=32, V=64), dict(B=2, T=32, H=2, K=8, V=16),
    dict(B=2, T=32, H=2, K=8, V=16, h0=True), dict(B=1, T=16, H=1, K=16, V=16),
    dict(B=4, T=64, H=8, K=32, V=64), dict(B=2, T=48, H=4, K=32, V=32),
    dict(B=2, T=32, H=4, K=32, V=64, scale=0.1),
    dict(B=1, T=32, H=4, K=32, V=64, cu=[0, 16, 32]),
    dict(B=1, T=96, H=4, K=32, V=64, cu=[0, 32, 64, 96]),
    dict(B=1, T=48, H=4, K=32, V=64, cu=[0, 16, 48]),
    dict(B=1, T=64, H=2, K=16, V=32, cu=[0, 16, 48, 64]),
    dict(B=1, T=32, H=4, K=32, V=64, cu=[0, 16, 32], h0=True),
    dict(B=1, T=48, H=4, K=32, V=64, cu=[0, 16, 48], h0=True),
    dict(B=1, T=64, H=2, K=16, V=32, cu=[0, 16, 32, 48, 64]),
    dict(B=1, T=80, H=2, K=32, V=64, cu=[0, 16, 80]),
    dict(B=1, T=64, H=2, K=32, V=64, cu=[0, 48, 64]),
    dict(B=1, T=96, H=2, K=16, V=32, cu=[0, 16, 32, 48, 64, 80, 96]),
    dict(B=1, T=64, H=4, K=32, V=64, cu=[0, 64]),
    dict(B=2, T=32, H=4, K=32, V=64, scale=0.1, h0=True),
    dict(B=1, T=32, H=4, K=32, V=64, scale=0.1, cu=[0, 16, 32]),
    dict(B=1, T=256, H=2, K=32, V=64), dict(B=1, T=512, H=2, K=32, V=64),
    dict(B=1, T=1024, H=2, K=32, V=64), dict(B=1, T=256, H=2, K=32, V=64, h0=True),
    dict(B=1, T=512, H=2, K=32, V=64, h0=True), dict(B=1, T=256, H=2, K=32, V=64, scale=0.1),
    dict(B=1, T=512, H=2, K=32, V=64, scale=0.01),
    dict(B=1, T=256, H=2, K=32, V=64, cu=[0, 128, 256]),
]


def _rid(c):
    s = "B{B}-T{T}-H{H}-K{K}-V{V}".format(**c)
    for key in ("h0", "scale", "cu"):
        if key in c:
            s += f"-{key}" + (str(c[key]) if key == "scale" else "")
    return s


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("c", REF, ids=_rid)
def test_reference_chunk_gla_shapes(c, dt, cuda_device):
    from tops.ops.gla import chunk_gla
    B, T, H, K, V = (c[x] for x in "BTHKV")
    cu = c.get("cu")
    n = B if cu is None else len(cu) - 1
    scale = c.get("scale", K ** -0.5)
    print(f"ref shape {_rid(c)} {dt}", flush=True)
    d = gla_inputs(B, T, H, K, V, seed=B * 1000 + T + K + V, gate_div=4.0, h0=c.get("h0", False),
                   N=n, grads=True)
    q, k, v = (to_dev(d[x], dt, cuda_device).requires_grad_() for x in "qkv")
    g = to_dev(d["g"], torch.float32, cuda_device).requires_grad_()
    h0 = to_dev(d["h0"], torch.float32, cuda_device)
    if h0 is not None:
        h0.requires_grad_()
    o, ht = chunk_gla(q, k, v, g, scale=scale, initial_state=h0, output_final_state=True,
                      cu_seqlens=cu)
    torch.autograd.backward((o, ht), (to_dev(d["do"], dt, cuda_device),
                                      to_dev(d["dht"], torch.float32, cuda_device)))
    sq, sk, sv, sdo = (seen(d[x], dt) for x in ("q", "k", "v", "do"))
    ro, rht = O.chunk_gla(sq, sk, sv, d["g"], scale, d["h0"], True, cu_seqlens=cu)
    rq, rk, rv, rg, rh0 = O.chunk_gla_bwd(sq, sk, sv, d["g"], scale, d["h0"], sdo, d["dht"],
                                          cu_seqlens=cu)
    # every output against the unrounded oracle (out_bound: 2e-3 for bf16, or the rounding
    # floor of a tensor too small for 2e-3 plus 2.5e-4)
    errs = dict(o=rel(host(o), ro), ht=rel(host(ht), rht), dq=rel(host(q.grad), rq),
                dk=rel(host(k.grad), rk), dv=rel(host(v.grad), rv))
    lims = dict(o=out_bound(ro, dt, dt), dq=out_bound(rq, dt, dt), dk=out_bound(rk, dt, dt),
                dv=out_bound(rv, dt, dt))
    # dg is a difference of k * dk-sized terms (q dq - k dk + ...); with no initial state
    # the first token's gate multiplies a zero state, so at T = 1 the exact dg is 0 and only
    # the cancellation residue remains: measure it against the scale of those terms
    den = max(float(np.linalg.norm(rg)), float(np.linalg.norm(sk * rk)))
    errs["dg"] = float(np.linalg.norm(host(g.grad) - rg)) / den
    if h0 is not None:
        errs["dh0"] = rel(host(h0.grad), rh0)
    print(" ".join(f"{n_}={e:.2e}" for n_, e in errs.items()))
    lim = 1e-4 if dt == torch.float32 else 2e-3
    for n_, e in errs.items():
        assert e < lims.get(n_, lim), (n_, e, lims.get(n_, lim))


GAMMA = [
    dict(B=2, T=32, H=4, K=32, V=64, shape="scalar"),
    dict(B=2, T=32, H=4, K=32, V=64, shape="per_head"),
    dict(B=2, T=32, H=4, K=32, V=64, shape="per_head_K"),
    dict(B=1, T=64, H=2, K=16, V=32, shape="per_head_K", h0=True),
    dict(B=4, T=48, H=2, K=32, V=64, shape="per_head"),
    dict(B=2, T=32, H=4, K=32, V=64, shape="per_head", scale=0.1),
    dict(B=1, T=256, H=2, K=32, V=64, shape="per_head"),
]


@pytest.mark.parametrize("c", GAMMA, ids=lambda c: "{shape}-B{B}-T{T}-H{H}-K{K}".format(**c))
def test_reference_chunk_gla_g_gamma(c, cuda_device):
    from tops.ops.gla import chunk_gla
    B, T, H, K, V = (c[x] for x in "BTHKV")
    scale = c.get("scale", K ** -0.5)
    rng = np.random.default_rng(T + H)
    gshape = {"scalar": (), "per_head": (1, 1, H, 1), "per_head_K": (1, 1, H, K)}[c["shape"]]
    gam = (-np.abs(rng.standard_normal(gshape)) * 0.1).astype(np.float32)
    d = gla_inputs(B, T, H, K, V, seed=T * 3 + K, h0=c.get("h0", False), grads=True)
    f = lambda x: to_dev(x, torch.float32, cuda_device)
    q, k, v = (f(d[x]).requires_grad_() for x in "qkv")
    gg = torch.tensor(gam, device=cuda_device, requires_grad=True)
    h0 = None if d["h0"] is None else f(d["h0"])
    o, ht = chunk_gla(q, k, v, None, g_gamma=gg, scale=scale, initial_state=h0,
                      output_final_state=True)
    torch.autograd.backward((o, ht), (f(d["do"]), f(d["dht"])))
    gfull = np.broadcast_to(gam, (B, T, H, K)).astype(np.float64)
    ro, rht = O.chunk_gla(d["q"], d["k"], d["v"], gfull, scale, d["h0"], True)
    rq, rk, rv, rg, _ = O.chunk_gla_bwd(d["q"], d["k"], d["v"], gfull, scale, d["h0"], d["do"],
                                        d["dht"])
    lead = 4 - len(gshape)               # g_gamma's gradient: sum over its broadcast axes
    rgam = rg.sum(axis=tuple(i for i in range(4) if i < lead or gshape[i - lead] == 1))
    errs = dict(o=rel(host(o), ro), ht=rel(host(ht), rht), dq=rel(host(q.grad), rq),
                dk=rel(host(k.grad), rk), dv=rel(host(v.grad), rv),
                dgamma=rel(host(gg.grad).reshape(-1), np.asarray(rgam).reshape(-1)))
    print(" ".join(f"{n_}={e:.2e}" for n_, e in errs.items()))
    for n_, e in errs.items():
        assert e < 1e-4, (n_, e)


# tests/ops/simple_gla/test_chunk_simple_gla_tpu.py:43-74 (the T = 4096 / 8192 cases, beyond
# what the float64 oracle checks in seconds, are left to the long-sequence tests)
SIMPLE = [
    dict(B=2, T=64, H=4, K=128, V=128), dict(B=2, T=128, H=4, K=128, V=128),
    dict(B=1, T=256, H=2, K=128, V=128), dict(B=2, T=64, H=4, K=128, V=128, h0=True),
    dict(B=2, T=128, H=4, K=128, V=128, h0=True), dict(B=1, T=256, H=2, K=128, V=128, h0=True),
    dict(B=2, T=64, H=1, K=128, V=128), dict(B=1, T=64, H=2, K=128, V=256),
    dict(B=2, T=64, H=4, K=256, V=128), dict(B=2, T=64, H=2, K=128, V=128),
    dict(B=8, T=64, H=4, K=128, V=128), dict(B=1, T=128, H=16, K=128, V=128),
    dict(B=2, T=64, H=4, K=128, V=128, scale=0.1),
    dict(B=2, T=64, H=4, K=128, V=128, scale=0.1, h0=True),
    dict(B=1, T=512, H=2, K=128, V=128), dict(B=1, T=512, H=2, K=128, V=128, h0=True),
    dict(B=4, T=256, H=2, K=128, V=128), dict(B=2, T=256, H=4, K=128, V=128),
    dict(B=1, T=256, H=2, K=128, V=128, chunk_size=128),
    dict(B=2, T=256, H=4, K=128, V=128, chunk_size=128),
]


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("c", SIMPLE, ids=_rid)
def test_reference_simple_gla_shapes(c, dt, cuda_device):
    from tops.ops.simple_gla import chunk_simple_gla
    from oracle import simple_gla as S
    from _inputs import simple_gla_inputs
    B, T, H, K, V = (c[x] for x in "BTHKV")
    scale = c.get("scale", K ** -0.5)
    print(f"simple ref shape {_rid(c)} {dt}", flush=True)
    d = simple_gla_inputs(B, T, H, K, V, seed=B * 100 + T + K + V, h0=c.get("h0", False),
                          grads=True)
    q, k, v = (to_dev(d[x], dt, cuda_device).requires_grad_() for x in "qkv")
    gg = to_dev(d["g_gamma"], torch.float32, cuda_device)
    h0 = to_dev(d["h0"], torch.float32, cuda_device)
    if h0 is not None:
        h0.requires_grad_()
    o, ht = chunk_simple_gla(q, k, v, gg, initial_state=h0, scale=scale, output_final_state=True,
                             chunk_size=c.get("chunk_size", 64))
    torch.autograd.backward((o, ht), (to_dev(d["do"], dt, cuda_device),
                                      to_dev(d["dht"], torch.float32, cuda_device)))
    sq, sk, sv, sdo = (seen(d[x], dt) for x in ("q", "k", "v", "do"))
    ro, rht = S.chunk_simple_gla(sq, sk, sv, g_gamma=d["g_gamma"], scale=scale,
                                 initial_state=d["h0"], output_final_state=True)
    rq, rk, rv, _, rh0 = S.chunk_simple_gla_bwd(sq, sk, sv, None, d["g_gamma"], d["h0"], sdo,
                                                d["dht"], scale)
    errs = dict(o=rel(host(o), ro), ht=rel(host(ht), rht), dq=rel(host(q.grad), rq),
                dk=rel(host(k.grad), rk), dv=rel(host(v.grad), rv))
    lims = dict(o=out_bound(ro, dt, dt), dq=out_bound(rq, dt, dt), dk=out_bound(rk, dt, dt),
                dv=out_bound(rv, dt, dt))
    if h0 is not None:
        errs["dh0"] = rel(host(h0.grad), rh0)
    print(" ".join(f"{n_}={e:.2e}" for n_, e in errs.items()))
    lim = 1e-4 if dt == torch.float32 else 2e-3
    for n_, e in errs.items():
        assert e < lims.get(n_, lim), (n_, e, lims.get(n_, lim))


# tests/ops/kda/test_chunk_kda_bwd_tpu.py:21-25
KDA = [
    dict(B=1, T=64, H=2, K=64, V=64), dict(B=2, T=128, H=4, K=64, V=64),
    dict(B=1, T=256, H=2, K=128, V=128), dict(B=2, T=128, H=4, K=64, V=128, h0=True),
    dict(B=1, T=128, H=2, K=64, V=64, h0=True),
]


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("c", KDA, ids=_rid)
def test_reference_kda_shapes(c, dt, cuda_device):
    """chunk_kda forward + autograd and the functional chunk_kda_bwd on the reference's KDA
    backward shapes, against the float64 oracle."""
    from tops.ops.kda import chunk_kda
    from tops.ops.kda.chunk_bwd import chunk_kda_bwd
    from tops.ops.common.cumsum import chunk_local_cumsum_vector
    from oracle import kda as KO
    from _inputs import kda_inputs
    B, T, H, K, V = (c[x] for x in "BTHKV")
    print(f"kda ref shape {_rid(c)} {dt}", flush=True)
    d = kda_inputs(B, T, H, K, V, seed=T + K + V + B, h0=c.get("h0", False), grads=True)
    q, k, v = (to_dev(d[x], dt, cuda_device).requires_grad_() for x in "qkv")
    f = lambda x: None if x is None else to_dev(x, torch.float32, cuda_device)
    g, beta = f(d["g"]).requires_grad_(), f(d["beta"]).requires_grad_()
    h0 = f(d["h0"])
    if h0 is not None:
        h0.requires_grad_()
    o, ht = chunk_kda(q, k, v, g, beta, initial_state=h0, output_final_state=True)
    do, dht = to_dev(d["do"], dt, cuda_device), f(d["dht"])
    torch.autograd.backward((o, ht), (do, dht))
    scale = K ** -0.5
    sq, sk, sv, sdo = (seen(d[x], dt) for x in ("q", "k", "v", "do"))
    ro, rht = KO.chunk_kda(sq, sk, sv, d["g"], d["beta"], scale, d["h0"], True)
    rq, rk, rv, rb, rg, rh0 = KO.chunk_kda_bwd(sq, sk, sv, d["g"], d["beta"], scale, d["h0"], sdo,
                                               d["dht"])
    errs = dict(o=rel(host(o), ro), ht=rel(host(ht), rht), dq=rel(host(q.grad), rq),
                dk=rel(host(k.grad), rk), dv=rel(host(v.grad), rv),
                db=rel(host(beta.grad), rb), dg=rel(host(g.grad), rg))
    lims = dict(o=out_bound(ro, dt, dt), dq=out_bound(rq, dt, dt), dk=out_bound(rk, dt, dt),
                dv=out_bound(rv, dt, dt), fn_dq=out_bound(rq, dt, dt))
    if h0 is not None:
        errs["dh0"] = rel(host(h0.grad), rh0)
    # the functional backward on the log2 gate cumsum (dg in log2 units)
    g2 = chunk_local_cumsum_vector(g.detach(), 64, scale=1 / np.log(2.0))
    fq, fk, fv, fb, fg, fh0, _, _ = chunk_kda_bwd(q.detach(), k.detach(), v.detach(),
                                                  beta.detach(), None, None, scale,
                                                  None if h0 is None else h0.detach(), do, dht,
                                                  g=g2)
    errs["fn_dq"] = rel(host(fq), rq)
    errs["fn_dg"] = rel(host(fg) / np.log(2.0), rg)
    print(" ".join(f"{n_}={e:.2e}" for n_, e in errs.items()))
    lim = 1e-4 if dt == torch.float32 else 2e-3
    for n_, e in errs.items():
        assert e < lims.get(n_, lim), (n_, e, lims.get(n_, lim))


# tests/ops/gla/test_pallas_fused_recurrent.py:26-119 (gates, reverse, varlen, scale, h0)
FR = [
    dict(B=2, T=32, H=4, K=32, V=64), dict(B=2, T=32, H=4, K=32, V=64, h0=True),
    dict(B=1, T=128, H=2, K=64, V=128), dict(B=2, T=32, H=4, K=16, V=128),
    dict(B=2, T=32, H=4, K=128, V=16), dict(B=1, T=1, H=2, K=32, V=64),
    dict(B=1, T=3, H=2, K=32, V=64), dict(B=2, T=37, H=4, K=16, V=32),
    dict(B=1, T=100, H=2, K=32, V=64, h0=True), dict(B=2, T=32, H=2, K=8, V=16, h0=True),
    dict(B=2, T=32, H=4, K=32, V=64, gate="gv"), dict(B=2, T=32, H=4, K=32, V=64, gate="gk+gv"),
    dict(B=2, T=32, H=4, K=32, V=64, gate="none"),
    dict(B=2, T=32, H=4, K=32, V=64, reverse=True),
    dict(B=2, T=32, H=4, K=32, V=64, reverse=True, h0=True),
    dict(B=1, T=1, H=2, K=16, V=32, reverse=True), dict(B=2, T=32, H=4, K=32, V=64, scale=0.1),
    dict(B=1, T=48, H=4, K=32, V=64, cu=[0, 10, 24, 48]),
    dict(B=1, T=23, H=2, K=16, V=32, cu=[0, 7, 20, 23]),
    dict(B=1, T=48, H=4, K=32, V=64, cu=[0, 10, 24, 48], h0=True),
    dict(B=1, T=4, H=2, K=16, V=32, cu=[0, 1, 2, 3, 4]),
    dict(B=1, T=67, H=2, K=32, V=64, cu=[0, 3, 67]),
    dict(B=1, T=23, H=2, K=16, V=32, cu=[0, 7, 20, 23], reverse=True),
    dict(B=1, T=32, H=4, K=32, V=64, gate="gk+gv", cu=[0, 16, 32]),
    dict(B=2, T=32, H=4, K=32, V=64, gate="gv", h0=True),
    dict(B=2, T=32, H=4, K=32, V=64, gate="gk+gv", reverse=True),
    dict(B=1, T=32, H=4, K=32, V=64, scale=0.1, cu=[0, 16, 32]),
    dict(B=1, T=512, H=2, K=32, V=64),
]


def _fid(c):
    s = _rid(c) + "-" + c.get("gate", "gk")
    return s + ("-rev" if c.get("reverse") else "")


@pytest.mark.parametrize("c", FR, ids=_fid)
def test_reference_fused_recurrent_shapes(c, cuda_device):
    from tops.ops.gla import fused_recurrent_gla
    B, T, H, K, V = (c[x] for x in "BTHKV")
    cu = c.get("cu")
    n = B if cu is None else len(cu) - 1
    gate = c.get("gate", "gk")
    rev = c.get("reverse", False)
    scale = c.get("scale", K ** -0.5)
    print(f"fused_recurrent ref shape {_fid(c)}", flush=True)
    d = gla_inputs(B, T, H, K, V, seed=T * 7 + K + V, gate_div=4.0, h0=c.get("h0", False), N=n,
                   grads=True)
    rng = np.random.default_rng(T + K)
    gvn = (np.log(1 / (1 + np.exp(-rng.standard_normal((B, T, H, V))))) / 4).astype(np.float32)
    gkn = d["g"] if "gk" in gate else None
    gvn = gvn if "gv" in gate else None
    f = lambda x: None if x is None else to_dev(x, torch.float32, cuda_device)
    q, k, v = (f(d[x]).requires_grad_() for x in "qkv")
    gk = None if gkn is None else f(gkn).requires_grad_()
    gv = None if gvn is None else f(gvn).requires_grad_()
    h0 = f(d["h0"])
    if h0 is not None:
        h0.requires_grad_()
    o, ht = fused_recurrent_gla(q, k, v, gk, gv, scale=scale, initial_state=h0,
                                output_final_state=True, reverse=rev, cu_seqlens=cu)
    torch.autograd.backward((o, ht), (f(d["do"]), f(d["dht"])))
    ro, rht = O.fused_recurrent_gla(d["q"], d["k"], d["v"], gkn, gvn, scale, d["h0"], True,
                                    reverse=rev, cu_seqlens=cu)
    r = O.fused_recurrent_bwd(d["q"], d["k"], d["v"], gkn, gvn, ro, d["do"], d["dht"], scale,
                              d["h0"], reverse=rev, cu_seqlens=cu)
    errs = dict(o=rel(host(o), ro), ht=rel(host(ht), rht), dq=rel(host(q.grad), r[0]),
                dk=rel(host(k.grad), r[1]), dv=rel(host(v.grad), r[2]))
    # gate gradients are differences of k * dk (v * dv)-sized terms that cancel exactly for a
    # sequence's first token without an initial state (T = 1, one-token sequences): measure
    # them against the scale of those terms
    def gerr(got, ref, x, dx):
        den = max(float(np.linalg.norm(ref)), float(np.linalg.norm(np.asarray(x) * dx)))
        return float(np.linalg.norm(host(got) - ref)) / den
    if gk is not None:
        errs["dgk"] = gerr(gk.grad, r[3], d["k"], r[1])
    if gv is not None:
        errs["dgv"] = gerr(gv.grad, r[4], d["v"], r[2])
    if h0 is not None:
        errs["dh0"] = rel(host(h0.grad), r[5])
    print(" ".join(f"{n_}={e:.2e}" for n_, e in errs.items()))
    for n_, e in errs.items():
        assert e < 1e-4, (n_, e)
