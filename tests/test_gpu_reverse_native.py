"""fused_recurrent with reverse=True on the reverse chunk sweep (tops_chunk_reverse_fwd) vs
the float64 oracle.

Without gradients, fused_recurrent_gla / fused_recurrent_gla_fwd / fused_recurrent_simple_gla
with reverse=True run the reverse-time recurrence S_t = diag(exp g_t) S_(t+1) + k_t v_t^T,
o_t = scale S_t^T q_t (tops/cpu/ops/gla/fused_recurrent.py:116-160) on the backward's reverse
sweep with q and k exchanged and the gate read one token later.  Checked against the oracle's
per-token reverse recurrence (oracle.gla.fused_recurrent_fwd, oracle.simple_gla.naive_simple_gla
on the flipped sequence) for per-channel, per-token, constant and absent gates, h0, ragged T,
varlen with empty and one-token sequences, K or V not 64-aligned and V > 128; every case also
checks that the native entry point ran (and, for a call that the chunk kernels would split into
sequence-parallel segments, that the time-reversal route ran instead).
Tolerance: fp32 1e-4, bf16 2e-3 (relative L2).
"""
import numpy as np
import pytest
import torch

from oracle import gla as O
from oracle import simple_gla as S
from _inputs import gla_inputs, simple_gla_inputs
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
    dict(B=1, T=4, H=2, K=8, V=16, h0=True, cu=[0, 1, 2, 3, 4]),
    dict(B=2, T=256, H=2, K=128, V=128, h0=True),                   # config-2 head shape
    dict(B=1, T=70, H=1, K=128, V=200, h0=True),                    # V > 128
    dict(B=1, T=90, H=2, K=24, V=32, h0=True, nogate=True),
    dict(B=1, T=100, H=2, K=32, V=32, scale=0.3, h0=True),
]


def _id(c):
    return "-".join(f"{k}{v}" for k, v in c.items() if k != "cu") + ("-varlen" if "cu" in c else "")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("cfg", CASES, ids=[_id(c) for c in CASES])
def test_reverse_gla_native(cfg, dtype, cuda_device, calls):
    from tops.ops.gla import fused_recurrent_gla
    B, T, H, K, V = (cfg[x] for x in "BTHKV")
    cu = cfg.get("cu")
    n = len(cu) - 1 if cu else B
    d = gla_inputs(B, T, H, K, V, seed=T * 3 + K + V, gate_div=4.0, h0=cfg.get("h0", False), N=n)
    g = None if cfg.get("nogate") else d["g"]
    sc = cfg.get("scale")
    q, k, v = (to_dev(d[x], dtype, cuda_device) for x in "qkv")
    with torch.no_grad():
        o, ht = fused_recurrent_gla(q, k, v, to_dev(g, torch.float32, cuda_device),
                                    scale=sc, initial_state=to_dev(d["h0"], torch.float32, cuda_device),
                                    output_final_state=True, reverse=True, cu_seqlens=cu)
    torch.cuda.synchronize()
    # sequences of at most 4 tokens take the decode kernel, longer ones the reverse sweep
    longest = T if cu is None else max(b - a for a, b in zip(cu[:-1], cu[1:]))
    assert ("tops_gla_fused_recurrent_fwd_decode" if longest <= 4 else "tops_chunk_reverse_fwd") in calls
    ro, rht = O.fused_recurrent_fwd(seen(d["q"], dtype), seen(d["k"], dtype), seen(d["v"], dtype),
                                    g, None, scale=sc, initial_state=d["h0"],
                                    output_final_state=True, reverse=True, cu_seqlens=cu)
    assert o.dtype == dtype and ht.dtype == torch.float32 and tuple(ht.shape) == rht.shape
    assert rel(host(o), ro) < tol(dtype), f"o rel {rel(host(o), ro):.2e}"
    assert rel(host(ht), rht) < tol(dtype), f"ht rel {rel(host(ht), rht):.2e}"


def test_reverse_fwd_api_and_no_final_state(cuda_device, calls):
    """fused_recurrent_gla_fwd(reverse=True) takes the same path; without output_final_state
    no final state comes back."""
    from tops.ops.gla import fused_recurrent_gla, fused_recurrent_gla_fwd
    B, T, H, K, V = 2, 130, 2, 64, 32
    d = gla_inputs(B, T, H, K, V, seed=5, gate_div=4.0, h0=True)
    q, k, v = (to_dev(d[x], torch.float32, cuda_device) for x in "qkv")
    g, h0 = to_dev(d["g"], torch.float32, cuda_device), to_dev(d["h0"], torch.float32, cuda_device)
    o1, ht1 = fused_recurrent_gla_fwd(q, k, v, g, initial_state=h0, output_final_state=True,
                                      reverse=True)
    with torch.no_grad():
        o2, ht2 = fused_recurrent_gla(q, k, v, g, initial_state=h0, reverse=True)
    torch.cuda.synchronize()
    assert calls.count("tops_chunk_reverse_fwd") == 2 and ht2 is None
    assert torch.equal(o1, o2)
    ro, rht = O.fused_recurrent_fwd(d["q"], d["k"], d["v"], d["g"], initial_state=d["h0"],
                                    output_final_state=True, reverse=True)
    assert rel(host(o1), ro) < 1e-4 and rel(host(ht1), rht) < 1e-4


def test_reverse_with_grad_keeps_time_reversal(cuda_device, calls):
    """With gradients wanted the time-reversal route runs (autograd through chunk_gla), and
    its forward equals the native path's."""
    from tops.ops.gla import fused_recurrent_gla
    B, T, H, K, V = 1, 100, 2, 32, 32
    d = gla_inputs(B, T, H, K, V, seed=9, gate_div=4.0, h0=True)
    q, k, v = (to_dev(d[x], torch.float32, cuda_device) for x in "qkv")
    g, h0 = to_dev(d["g"], torch.float32, cuda_device), to_dev(d["h0"], torch.float32, cuda_device)
    with torch.no_grad():
        o1, ht1 = fused_recurrent_gla(q, k, v, g, initial_state=h0, output_final_state=True,
                                      reverse=True)
    n_native = calls.count("tops_chunk_reverse_fwd")
    q.requires_grad_()
    o2, ht2 = fused_recurrent_gla(q, k, v, g, initial_state=h0, output_final_state=True,
                                  reverse=True)
    torch.cuda.synchronize()
    assert n_native == 1 and calls.count("tops_chunk_reverse_fwd") == 1
    assert rel(host(o1), host(o2)) < 1e-5 and rel(host(ht1), host(ht2)) < 1e-5


def test_reverse_segmented_call_uses_time_reversal(cuda_device, calls):
    """A long single sequence (which the chunk kernels split into sequence-parallel segments)
    keeps the time-reversal route, and matches the oracle."""
    from tops.ops.gla import fused_recurrent_gla
    B, T, H, K, V = 1, 64 * 40, 1, 32, 32
    d = gla_inputs(B, T, H, K, V, seed=11, gate_div=4.0, h0=True)
    q, k, v = (to_dev(d[x], torch.float32, cuda_device) for x in "qkv")
    with torch.no_grad():
        o, ht = fused_recurrent_gla(q, k, v, to_dev(d["g"], torch.float32, cuda_device),
                                    initial_state=to_dev(d["h0"], torch.float32, cuda_device),
                                    output_final_state=True, reverse=True)
    torch.cuda.synchronize()
    assert "tops_chunk_reverse_fwd" not in calls
    ro, rht = O.fused_recurrent_fwd(d["q"], d["k"], d["v"], d["g"], initial_state=d["h0"],
                                    output_final_state=True, reverse=True)
    assert rel(host(o), ro) < 1e-4 and rel(host(ht), rht) < 1e-4


@pytest.mark.parametrize("gates", ["g", "gamma", "both"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_reverse_simple_gla_native(gates, dtype, cuda_device, calls):
    """fused_recurrent_simple_gla(reverse=True) without gradients: per-token g (mode s), g_gamma
    (constant gate) and both, vs the naive oracle on the time-flipped sequences (varlen with
    an empty sequence)."""
    from tops.ops.simple_gla import fused_recurrent_simple_gla
    B, T, H, K, V = 1, 150, 2, 32, 48
    cu = [0, 40, 40, 99, 150]
    d = simple_gla_inputs(B, T, H, K, V, seed=23, h0=True, N=len(cu) - 1)
    g = d["g"] if gates != "gamma" else None
    gg = d["g_gamma"] if gates != "g" else None
    q, k, v = (to_dev(d[x], dtype, cuda_device) for x in "qkv")
    with torch.no_grad():
        o, ht = fused_recurrent_simple_gla(q, k, v, g=to_dev(g, torch.float32, cuda_device),
                                           g_gamma=to_dev(gg, torch.float32, cuda_device),
                                           initial_state=to_dev(d["h0"], torch.float32, cuda_device),
                                           output_final_state=True, reverse=True, cu_seqlens=cu)
    torch.cuda.synchronize()
    assert "tops_chunk_reverse_fwd" in calls
    sq, sk, sv = (seen(d[x], dtype) for x in "qkv")
    ro = np.zeros((B, T, H, V))
    rhts = []
    for n in range(len(cu) - 1):
        a, b = cu[n], cu[n + 1]
        fl = lambda x: None if x is None else np.ascontiguousarray(x[:, a:b][:, ::-1])  # noqa: E731
        if b == a:
            rhts.append(np.float64(d["h0"][n]))
            continue
        on, htn = S.naive_simple_gla(fl(sq), fl(sk), fl(sv), g=fl(g), g_gamma=gg,
                                     initial_state=d["h0"][n:n + 1], output_final_state=True)
        ro[:, a:b] = on[:, ::-1]
        rhts.append(htn[0])
    rht = np.stack(rhts)
    assert rel(host(o), ro) < tol(dtype), f"o rel {rel(host(o), ro):.2e}"
    assert rel(host(ht), rht) < tol(dtype), f"ht rel {rel(host(ht), rht):.2e}"
