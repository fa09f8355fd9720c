"""fused_recurrent_gla on MI355X vs the float64 oracle (tops/cpu/ops/gla/fused_recurrent.py
restated).

Forward (o, ht) and backward through torch autograd (dq, dk, dv, dgk, dgv, dh0) for gk and
gv gates, h0 / dht, reverse and varlen, plus the explicit fused_recurrent_gla_bwd API and a
one-token decode step chained from a prefix state.  Cases follow the reference's
tests/ref/gla/test_fused_recurrent_gla.py (gk / gv / reverse / varlen) and BASELINE config 2
(B16 T2048 H8 K=V=128, here at reduced T).  Error metric: relative L2 against the fp64
oracle on the inputs the kernel saw.  Tolerance: fp32 1e-4, bf16 2e-3.
"""
import numpy as np
import pytest
import torch

from oracle import gla as O
from _inputs import gla_inputs
from _gpu import to_dev, seen, host, rel, tol

pytestmark = pytest.mark.gpu

CASES = [
    dict(B=2, T=64, H=2, K=32, V=32, gk=True),
    dict(B=2, T=50, H=2, K=64, V=64, gk=True, h0=True),
    dict(B=1, T=37, H=3, K=16, V=40, gk=True, gv=True, h0=True),
    dict(B=2, T=33, H=2, K=32, V=64, gk=True, h0=True, reverse=True),
    dict(B=1, T=30, H=2, K=8, V=16, gv=True, reverse=True, h0=True),
    dict(B=1, T=1, H=2, K=32, V=64, gk=True, h0=True),
    dict(B=1, T=120, H=2, K=32, V=32, gk=True, h0=True, cu=[0, 13, 64, 65, 120]),
    dict(B=1, T=90, H=2, K=16, V=16, gk=True, gv=True, reverse=True, cu=[0, 30, 31, 90]),
    dict(B=2, T=256, H=2, K=128, V=128, gk=True, h0=True),          # config-2 shape, short T
    dict(B=1, T=70, H=1, K=128, V=200, gk=True, h0=True),           # V > 128, ragged tiles
    dict(B=1, T=40, H=2, K=24, V=32, h0=True),                      # no gates
]


def _id(c):
    return "-".join(f"{k}{v}" for k, v in c.items() if k != "cu") + ("-varlen" if "cu" in c else "")


def _inputs(cfg):
    B, T, H, K, V = (cfg[x] for x in "BTHKV")
    cu = cfg.get("cu")
    n = len(cu) - 1 if cu else B
    d = gla_inputs(B, T, H, K, V, seed=T * 5 + K + V, gate_div=4.0, h0=cfg.get("h0", False), N=n,
                   grads=True)
    rng = np.random.default_rng(T + V)
    d["gv"] = (-np.abs(rng.standard_normal((B, T, H, V))) * 0.2).astype(np.float32) \
        if cfg.get("gv") else None
    if not cfg.get("gk"):
        d["g"] = None
    return d, cu


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("cfg", CASES, ids=[_id(c) for c in CASES])
def test_fused_recurrent_fwd_bwd(cfg, dtype, cuda_device):
    from tops.ops.gla import fused_recurrent_gla
    d, cu = _inputs(cfg)
    rev = cfg.get("reverse", False)
    q, k, v = (to_dev(d[x], dtype, cuda_device).requires_grad_() for x in "qkv")
    gk = None if d["g"] is None else to_dev(d["g"], torch.float32, cuda_device).requires_grad_()
    gv = None if d["gv"] is None else to_dev(d["gv"], torch.float32, cuda_device).requires_grad_()
    h0 = to_dev(d["h0"], torch.float32, cuda_device)
    if h0 is not None:
        h0.requires_grad_()
    o, ht = fused_recurrent_gla(q, k, v, gk, gv, initial_state=h0, output_final_state=True,
                                reverse=rev, cu_seqlens=cu)
    do, dht = to_dev(d["do"], dtype, cuda_device), to_dev(d["dht"], torch.float32, cuda_device)
    torch.autograd.backward((o, ht), (do, dht))
    torch.cuda.synchronize()
    sq, sk, sv, sdo = (seen(d[x], dtype) for x in ("q", "k", "v", "do"))
    ro, rht = O.fused_recurrent_fwd(sq, sk, sv, d["g"], d["gv"], initial_state=d["h0"],
                                    output_final_state=True, reverse=rev, cu_seqlens=cu)
    rq, rk, rv, rgk, rgv, rh0 = O.fused_recurrent_bwd(sq, sk, sv, d["g"], d["gv"], ro, sdo, d["dht"],
                                                      initial_state=d["h0"], reverse=rev,
                                                      cu_seqlens=cu)
    assert o.dtype == dtype and ht.dtype == torch.float32
    got = dict(o=o, ht=ht, dq=q.grad, dk=k.grad, dv=v.grad)
    ref = dict(o=ro, ht=rht, dq=rq, dk=rk, dv=rv)
    if gk is not None:
        got["dgk"], ref["dgk"] = gk.grad, rgk
    if gv is not None:
        got["dgv"], ref["dgv"] = gv.grad, rgv
    if h0 is not None:
        got["dh0"], ref["dh0"] = h0.grad, rh0
    errs = {n: rel(host(got[n]), ref[n]) for n in got}
    print(" ".join(f"{k}={v:.2e}" for k, v in errs.items()))
    for n, e in errs.items():
        assert e < tol(dtype), (n, e)


def test_bwd_api(cuda_device):
    """tops.ops.gla.fused_recurrent_gla_bwd (tops/ops/gla/fused_recurrent.py:881-958)."""
    from tops.ops.gla import fused_recurrent_gla_bwd, fused_recurrent_gla_fwd
    d, _ = _inputs(dict(B=1, T=45, H=2, K=32, V=32, gk=True, gv=True, h0=True))
    t = {x: to_dev(d[x], torch.float32, cuda_device) for x in ("q", "k", "v", "g", "gv", "h0", "do", "dht")}
    o, _ = fused_recurrent_gla_fwd(t["q"], t["k"], t["v"], t["g"], t["gv"], initial_state=t["h0"])
    dq, dk, dv, dgk, dgv, dh0 = fused_recurrent_gla_bwd(t["q"], t["k"], t["v"], t["g"], t["gv"], o,
                                                        t["do"], t["dht"], initial_state=t["h0"])
    ro, _ = O.fused_recurrent_fwd(d["q"], d["k"], d["v"], d["g"], d["gv"], initial_state=d["h0"])
    ref = O.fused_recurrent_bwd(d["q"], d["k"], d["v"], d["g"], d["gv"], ro, d["do"], d["dht"],
                                initial_state=d["h0"])
    for x, r in zip((dq, dk, dv, dgk, dgv, dh0), ref):
        assert rel(host(x), r) < 1e-4


def test_decode_step_continues_chunk_prefix(cuda_device):
    """Decode: a chunk_gla prefix state fed to fused_recurrent_gla for the next token equals
    one fused_recurrent run over the whole sequence (tops/layers/gla.py:288-297 routes
    q_len <= 64 to fused_recurrent)."""
    from tops.ops.gla import chunk_gla, fused_recurrent_gla
    d = gla_inputs(1, 129, 2, 64, 64, seed=55, gate_div=8.0)
    t = {x: to_dev(d[x], torch.float32, cuda_device) for x in "qkvg"}
    _, s = chunk_gla(*(t[x][:, :128] for x in "qkvg"), output_final_state=True)
    o1, s1 = fused_recurrent_gla(*(t[x][:, 128:] for x in "qkvg"), initial_state=s,
                                 output_final_state=True)
    of, sf = fused_recurrent_gla(t["q"], t["k"], t["v"], t["g"], output_final_state=True)
    assert rel(host(o1), host(of[:, 128:])) < 1e-4
    assert rel(host(s1), host(sf)) < 1e-4
