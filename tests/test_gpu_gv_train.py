"""fused_recurrent_gla with a value-side gate gv (no gk) and gradients, bf16: forward and
backward on the chunk kernels (the value-gate forward with fp32 and bf16 output, the
key-gated chunk forward on the transposed state for dq, the key-gated state-gradient sweep
on the transposed problem for dk, the value-gated state-gradient sweep for dv and dh0,
suffix sums for dgv) against the float64 oracle (tops/cpu/ops/gla/fused_recurrent.py
restated), and a check that no per-token kernel ran.  Cases: fixed length with and without
h0, varlen with a one-token sequence, K != V both ways, BASELINE config 2's K = V = 128 at
reduced T, one long sequence, a loss on o alone and on ht alone.  Tolerance: bf16 2e-3
(relative L2) on o, ht and every gradient; the forward's two outputs bitwise.
"""
import numpy as np
import pytest
import torch

from oracle import gla as O
from _inputs import gla_inputs
from _gpu import to_dev, seen, host, rel, tol

pytestmark = pytest.mark.gpu

CASES = [
    dict(B=2, T=100, H=2, K=32, V=64, h0=True),
    dict(B=1, T=64, H=1, K=16, V=24, h0=False),
    dict(B=1, T=150, H=2, K=64, V=32, h0=True, cu=[0, 1, 70, 150]),
    dict(B=2, T=256, H=2, K=128, V=128, h0=True),
    dict(B=1, T=333, H=3, K=48, V=96, h0=True, cu=[0, 129, 130, 333]),
    # one long sequence on few heads (the chunk kernels' plan would split it; the gv sweeps
    # take it whole)
    dict(B=1, T=4096, H=1, K=64, V=64, h0=True),
]


def _id(c):
    return "-".join(f"{k}{v}" for k, v in c.items() if k != "cu") + ("-varlen" if "cu" in c else "")


@pytest.mark.parametrize("cfg", CASES, ids=[_id(c) for c in CASES])
def test_gv_training_on_chunk_kernels(cfg, cuda_device, monkeypatch):
    from tops import _native as N
    from tops.ops.gla import fused_recurrent_gla
    names = []
    real = N.call
    monkeypatch.setattr(N, "call", lambda name, *a: (names.append(name), real(name, *a))[1])
    B, T, H, K, V = (cfg[x] for x in "BTHKV")
    cu = cfg.get("cu")
    n = len(cu) - 1 if cu else B
    d = gla_inputs(B, T, H, K, V, seed=T + 7 * V, gate_div=4.0, h0=cfg["h0"], N=n, grads=True)
    rng = np.random.default_rng(T + K)
    gvn = (-np.abs(rng.standard_normal((B, T, H, V))) * 0.2).astype(np.float32)
    bf = torch.bfloat16
    q, k, v = (to_dev(d[x], bf, cuda_device).requires_grad_() for x in "qkv")
    gv = to_dev(gvn, torch.float32, cuda_device).requires_grad_()
    h0 = to_dev(d["h0"], torch.float32, cuda_device)
    if h0 is not None:
        h0.requires_grad_()
    o, ht = fused_recurrent_gla(q, k, v, None, gv, initial_state=h0, output_final_state=True,
                                cu_seqlens=cu)
    torch.autograd.backward((o, ht), (to_dev(d["do"], bf, cuda_device),
                                      to_dev(d["dht"], torch.float32, cuda_device)))
    torch.cuda.synchronize()
    assert "tops_gla_chunk_fwd_gv32" in names
    assert not any(x.startswith("tops_gla_fused_recurrent") for x in names), names
    sq, sk, sv, sdo = (seen(d[x], bf) for x in ("q", "k", "v", "do"))
    ro, rht = O.fused_recurrent_fwd(sq, sk, sv, None, gvn, initial_state=d["h0"],
                                    output_final_state=True, cu_seqlens=cu)
    rq, rk, rv, _, rgv, rh0 = O.fused_recurrent_bwd(sq, sk, sv, None, gvn, ro, sdo, d["dht"],
                                                    initial_state=d["h0"], cu_seqlens=cu)
    got = dict(o=o, ht=ht, dq=q.grad, dk=k.grad, dv=v.grad, dgv=gv.grad)
    ref = dict(o=ro, ht=rht, dq=rq, dk=rk, dv=rv, dgv=rgv)
    if h0 is not None:
        got["dh0"], ref["dh0"] = h0.grad, rh0
    errs = {x: rel(host(got[x]), ref[x]) for x in got}
    print(" ".join(f"{x}={e:.2e}" for x, e in errs.items()))
    for x, e in errs.items():
        assert e < tol(bf), (x, e)


@pytest.mark.parametrize("used", ["o", "ht"])
def test_gv_training_with_one_output_unused(used, cuda_device):
    """A loss on o alone (backward gets no dht: no final-state term) or on ht alone (no dO):
    the same gradients as the oracle's with the missing one zero."""
    from tops.ops.gla import fused_recurrent_gla
    B, T, H, K, V = 2, 200, 2, 64, 64
    d = gla_inputs(B, T, H, K, V, seed=11, gate_div=4.0, h0=True, N=B, grads=True)
    rng = np.random.default_rng(5)
    gvn = (-np.abs(rng.standard_normal((B, T, H, V))) * 0.2).astype(np.float32)
    bf = torch.bfloat16
    q, k, v = (to_dev(d[x], bf, cuda_device).requires_grad_() for x in "qkv")
    gv = to_dev(gvn, torch.float32, cuda_device).requires_grad_()
    h0 = to_dev(d["h0"], torch.float32, cuda_device).requires_grad_()
    o, ht = fused_recurrent_gla(q, k, v, None, gv, initial_state=h0, output_final_state=True)
    if used == "o":
        o.backward(to_dev(d["do"], bf, cuda_device))
        do, dht = d["do"], np.zeros_like(d["dht"])
    else:
        ht.backward(to_dev(d["dht"], torch.float32, cuda_device))
        do, dht = np.zeros_like(d["do"]), d["dht"]
    torch.cuda.synchronize()
    sq, sk, sv, sdo = (seen(x, bf) for x in (d["q"], d["k"], d["v"], do))
    ro, _ = O.fused_recurrent_fwd(sq, sk, sv, None, gvn, initial_state=d["h0"],
                                  output_final_state=True)
    rq, rk, rv, _, rgv, rh0 = O.fused_recurrent_bwd(sq, sk, sv, None, gvn, ro, sdo, dht,
                                                    initial_state=d["h0"])
    got = dict(dq=q.grad, dk=k.grad, dv=v.grad, dgv=gv.grad, dh0=h0.grad)
    ref = dict(dq=rq, dk=rk, dv=rv, dgv=rgv, dh0=rh0)
    errs = {x: rel(host(got[x]), ref[x]) for x in got}
    print(" ".join(f"{x}={e:.2e}" for x, e in errs.items()))
    for x, e in errs.items():
        assert e < tol(bf), (x, e)


def test_gv32_forward_writes_the_bf16_output_from_the_same_sum(cuda_device):
    """tops_gla_chunk_fwd_gv32 with the optional bf16 o: o32 is bitwise the same as without
    it, and o is o32 rounded to bf16 (torch's round-to-nearest-even), on a varlen call whose
    V is not a multiple of 64."""
    from tops import _native as N
    B, T, H, K, V = 1, 300, 2, 64, 72
    cu = [0, 1, 130, 300]
    d = gla_inputs(B, T, H, K, V, seed=23, gate_div=4.0, h0=True, N=3)
    rng = np.random.default_rng(9)
    gv = to_dev((-np.abs(rng.standard_normal((B, T, H, V))) * 0.2).astype(np.float32),
                torch.float32, cuda_device)
    q, k, v = (to_dev(d[x], torch.bfloat16, cuda_device) for x in "qkv")
    h0 = to_dev(d["h0"], torch.float32, cuda_device)
    cut = torch.tensor(cu, dtype=torch.int32, device=cuda_device)
    outs = []
    for with_o in (False, True):
        o32 = torch.full((B, T, H, V), float("nan"), device=cuda_device)
        o = torch.zeros(B, T, H, V, device=cuda_device, dtype=torch.bfloat16) if with_o else None
        ht = torch.empty(3, H, K, V, device=cuda_device)
        N.call("tops_gla_chunk_fwd_gv32", N.ptr(q), N.ptr(k), N.ptr(v), N.ptr(gv), N.ptr(h0),
               N.ptr(o32), N.ptr(o), N.ptr(ht), N.ptr(cut), B, T, H, K, V, 3,
               N.dtype_code(torch.bfloat16), K ** -0.5, N.stream())
        torch.cuda.synchronize()
        outs.append((o32, o))
    assert not outs[0][0].isnan().any()
    assert torch.equal(outs[0][0], outs[1][0])
    assert torch.equal(outs[1][1].view(torch.int16), outs[1][0].to(torch.bfloat16).view(torch.int16))
