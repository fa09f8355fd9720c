"""fused_recurrent_gla with a value-side gate (gv, no gk) on the chunk sweep
(tops_gla_chunk_fwd_gv) vs the float64 oracle.

Without gradients and for bf16 inputs, fused_recurrent_gla / fused_recurrent_gla_fwd with gv
run S_t = S_(t-1) diag(exp gv_t) + k_t v_t^T, o_t = scale S_t^T q_t
(tops/cpu/ops/gla/fused_recurrent.py:51-167) in 64-token chunks on MFMA.  Checked against the
oracle's per-token recurrence (oracle.gla.fused_recurrent_fwd) for h0, ragged T, T = 1, varlen
with empty and one-token sequences, K or V not 64-aligned, V > 128 and gates up to a few
units per token; every case checks that the chunk entry point ran.  With gradients wanted
(bf16) the chunked training path runs instead (tests/test_gpu_gv_train.py checks its
gradients); fp32 inputs keep the per-token kernel, also checked.
Tolerance: bf16 2e-3 (relative L2).
"""
import numpy as np
import pytest
import torch

from oracle import gla as O
from _inputs import gla_inputs
from _gpu import to_dev, seen, host, rel, tol

pytestmark = pytest.mark.gpu


@pytest.fixture
def calls(monkeypatch):
    """Names of the C entry points called during the test."""
    from tops import _native as N
    seen_calls = []
    real = N.call

    def spy(name, *args):
        seen_calls.append(name)
        return real(name, *args)
    monkeypatch.setattr(N, "call", spy)
    return seen_calls


CASES = [
    dict(B=2, T=64, H=2, K=32, V=32),
    dict(B=2, T=50, H=2, K=64, V=64, h0=True),
    dict(B=1, T=1, H=2, K=32, V=64, h0=True),
    dict(B=2, T=200, H=3, K=16, V=40, h0=True),
    dict(B=1, T=150, H=2, K=32, V=32, h0=True, cu=[0, 13, 13, 64, 65, 150]),
    dict(B=2, T=256, H=2, K=128, V=128, h0=True),                   # config-2 head shape
    dict(B=1, T=70, H=1, K=128, V=200, h0=True),                    # V > 128
    dict(B=1, T=100, H=2, K=24, V=72, h0=True, scale=0.3),
    dict(B=1, T=130, H=2, K=64, V=64, h0=True, strong=True),        # gates down to -3 per token
]


def _id(c):
    return "-".join(f"{k}{v}" for k, v in c.items() if k != "cu") + ("-varlen" if "cu" in c else "")


def _gv(B, T, H, V, seed, strong=False):
    rng = np.random.default_rng(seed)
    x = -np.abs(rng.standard_normal((B, T, H, V)))
    return (x * (1.5 if strong else 0.2)).astype(np.float32)


@pytest.mark.parametrize("cfg", CASES, ids=[_id(c) for c in CASES])
def test_gv_native(cfg, cuda_device, calls):
    from tops.ops.gla import fused_recurrent_gla
    B, T, H, K, V = (cfg[x] for x in "BTHKV")
    cu = cfg.get("cu")
    n = len(cu) - 1 if cu else B
    d = gla_inputs(B, T, H, K, V, seed=T * 7 + K + V, h0=cfg.get("h0", False), N=n)
    gv = _gv(B, T, H, V, T + V, cfg.get("strong", False))
    sc = cfg.get("scale")
    bf = torch.bfloat16
    q, k, v = (to_dev(d[x], bf, cuda_device) for x in "qkv")
    with torch.no_grad():
        o, ht = fused_recurrent_gla(q, k, v, None, to_dev(gv, torch.float32, cuda_device),
                                    scale=sc, initial_state=to_dev(d["h0"], torch.float32, cuda_device),
                                    output_final_state=True, cu_seqlens=cu)
    torch.cuda.synchronize()
    # sequences of at most 4 tokens take the decode kernel, longer ones the gv sweep
    longest = T if cu is None else max(b - a for a, b in zip(cu[:-1], cu[1:]))
    assert ("tops_gla_fused_recurrent_fwd_decode" if longest <= 4 else "tops_gla_chunk_fwd_gv") in calls
    ro, rht = O.fused_recurrent_fwd(seen(d["q"], bf), seen(d["k"], bf), seen(d["v"], bf), None, gv,
                                    scale=sc, initial_state=d["h0"], output_final_state=True,
                                    cu_seqlens=cu)
    assert o.dtype == bf and ht.dtype == torch.float32 and tuple(ht.shape) == rht.shape
    assert rel(host(o), ro) < tol(bf), f"o rel {rel(host(o), ro):.2e}"
    assert rel(host(ht), rht) < tol(bf), f"ht rel {rel(host(ht), rht):.2e}"


def test_gv_fwd_api(cuda_device, calls):
    """fused_recurrent_gla_fwd with gv takes the same path, without a final state too."""
    from tops.ops.gla import fused_recurrent_gla_fwd
    B, T, H, K, V = 2, 130, 2, 64, 32
    d = gla_inputs(B, T, H, K, V, seed=3, h0=True)
    gv = _gv(B, T, H, V, 4)
    bf = torch.bfloat16
    q, k, v = (to_dev(d[x], bf, cuda_device) for x in "qkv")
    o, ht = fused_recurrent_gla_fwd(q, k, v, None, to_dev(gv, torch.float32, cuda_device),
                                    initial_state=to_dev(d["h0"], torch.float32, cuda_device))
    torch.cuda.synchronize()
    assert calls.count("tops_gla_chunk_fwd_gv") == 1 and ht is None
    ro, _ = O.fused_recurrent_fwd(seen(d["q"], bf), seen(d["k"], bf), seen(d["v"], bf), None, gv,
                                  initial_state=d["h0"])
    assert rel(host(o), ro) < 2e-3


@pytest.mark.parametrize("case", ["grad", "fp32"])
def test_gv_routing_with_gradients_and_fp32(case, cuda_device, calls):
    """With gradients wanted (bf16) the chunked training path runs (its forward writes o in
    fp32: tops_gla_chunk_fwd_gv32); fp32 inputs keep the per-token kernel.  Both match."""
    from tops.ops.gla import fused_recurrent_gla
    B, T, H, K, V = 1, 90, 2, 32, 32
    d = gla_inputs(B, T, H, K, V, seed=8, h0=True)
    gv = _gv(B, T, H, V, 9)
    dt = torch.float32 if case == "fp32" else torch.bfloat16
    q, k, v = (to_dev(d[x], dt, cuda_device) for x in "qkv")
    if case == "grad":
        q.requires_grad_()
        o, ht = fused_recurrent_gla(q, k, v, None, to_dev(gv, torch.float32, cuda_device),
                                    initial_state=to_dev(d["h0"], torch.float32, cuda_device),
                                    output_final_state=True)
    else:
        with torch.no_grad():
            o, ht = fused_recurrent_gla(q, k, v, None, to_dev(gv, torch.float32, cuda_device),
                                        initial_state=to_dev(d["h0"], torch.float32, cuda_device),
                                        output_final_state=True)
    torch.cuda.synchronize()
    assert "tops_gla_chunk_fwd_gv" not in calls
    if case == "grad":
        assert "tops_gla_chunk_fwd_gv32" in calls and "tops_gla_fused_recurrent_fwd" not in calls
    else:
        assert "tops_gla_fused_recurrent_fwd" in calls
    ro, rht = O.fused_recurrent_fwd(seen(d["q"], dt), seen(d["k"], dt), seen(d["v"], dt), None, gv,
                                    initial_state=d["h0"], output_final_state=True)
    assert rel(host(o), ro) < tol(dt) and rel(host(ht), rht) < tol(dt)
