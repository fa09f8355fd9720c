"""fused_recurrent_gla on sequences of a few tokens (decode steps) vs the float64 oracle.

Without gradients, calls whose longest sequence has at most 4 tokens run on the register-state
kernel (tops_gla_fused_recurrent_fwd_decode): the per-token recurrence
h <- h*exp(gk_t)[:,None]*exp(gv_t)[None,:] + k_t v_t^T, o_t = scale h^T q_t
(tops/cpu/ops/gla/fused_recurrent.py:51-167).  Checked against the oracle's per-token recurrence
(oracle.gla.fused_recurrent_fwd) for gk, gv, both and no gate, reverse, h0 present or absent,
K and V off the 8-column tile (K = 4, 36; V = 7, 20, 100), fixed length and varlen (empty and
one-token sequences, many one-token sequences packed), fp32 and bf16; every case checks that the
decode entry point ran (and that a 5-token call does not).  The fixed-length per-token entry takes
the same kernel for T <= 4, and a call with gradients keeps the autograd path (checked against the
oracle's backward).
Tolerance: fp32 1e-4, bf16 2e-3 (relative L2).
"""
import numpy as np
import pytest
import torch

from oracle import gla as O
from _inputs import gla_inputs, bf16_round
from _gpu import to_dev, seen, host, rel, tol, out_bound

pytestmark = pytest.mark.gpu

DECODE = "tops_gla_fused_recurrent_fwd_decode"


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
    dict(B=4, T=1, H=4, K=128, V=128, gate="gk", h0=True),          # one decode step
    dict(B=2, T=3, H=2, K=64, V=64, gate="gv", h0=True),
    dict(B=2, T=4, H=2, K=128, V=128, gate="both", h0=True),
    dict(B=1, T=4, H=2, K=36, V=20, gate="gk", h0=True, reverse=True),
    dict(B=1, T=8, H=3, K=32, V=100, gate="none", cu=[0, 1, 1, 4, 8]),
    dict(B=1, T=64, H=2, K=128, V=64, gate="gk", h0=True, cu=list(range(65))),   # 64 x 1 token
    dict(B=3, T=2, H=1, K=4, V=7, gate="gk", h0=True),
    dict(B=2, T=3, H=2, K=128, V=128, gate="both", h0=True, reverse=True, scale=0.3),
    dict(B=2, T=3, H=2, K=64, V=160, gate="both", h0=True),        # two tile groups, 3 idle waves
]


def _id(c):
    return "-".join(f"{k}{v}" for k, v in c.items() if k != "cu") + ("-varlen" if "cu" in c else "")


def _gates(cfg, d, B, T, H, V, seed):
    rng = np.random.Generator(np.random.PCG64(seed))
    gv = (np.log(1 / (1 + np.exp(-rng.standard_normal((B, T, H, V))))) / 8).astype(np.float32)
    gk = d["g"] if cfg["gate"] in ("gk", "both") else None
    return gk, (gv if cfg["gate"] in ("gv", "both") else None)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("cfg", CASES, ids=[_id(c) for c in CASES])
def test_decode_matches_oracle(cfg, dtype, cuda_device, calls):
    from tops.ops.gla import fused_recurrent_gla
    B, T, H, K, V = (cfg[x] for x in "BTHKV")
    cu = cfg.get("cu")
    n = len(cu) - 1 if cu else B
    print(f"decode case {_id(cfg)} {dtype}", flush=True)
    d = gla_inputs(B, T, H, K, V, seed=T * 5 + K + V, gate_div=4.0, h0=cfg.get("h0", False), N=n)
    gk, gv = _gates(cfg, d, B, T, H, V, T + K)
    sc, rev = cfg.get("scale"), cfg.get("reverse", False)
    dv = lambda x: to_dev(x, torch.float32, cuda_device)
    q, k, v = (to_dev(d[x], dtype, cuda_device) for x in "qkv")
    with torch.no_grad():
        o, ht = fused_recurrent_gla(q, k, v, dv(gk), dv(gv), scale=sc, initial_state=dv(d["h0"]),
                                    output_final_state=True, reverse=rev, cu_seqlens=cu)
    torch.cuda.synchronize()
    assert DECODE in calls
    ro, rht = O.fused_recurrent_fwd(seen(d["q"], dtype), seen(d["k"], dtype), seen(d["v"], dtype),
                                    gk, gv, scale=sc, initial_state=d["h0"], output_final_state=True,
                                    reverse=rev, cu_seqlens=cu)
    assert o.dtype == dtype and ht.dtype == torch.float32 and tuple(ht.shape) == rht.shape
    eo, eh = rel(host(o), ro), rel(host(ht), rht)
    print(f"o {eo:.2e} ht {eh:.2e}")
    assert eo < tol(dtype) and eh < tol(dtype)


def test_decode_fwd_api_without_final_state(cuda_device, calls):
    """fused_recurrent_gla_fwd takes the decode kernel too; without output_final_state no state
    comes back, and o is the same as with it."""
    from tops.ops.gla import fused_recurrent_gla_fwd
    B, T, H, K, V = 8, 1, 4, 128, 128
    d = gla_inputs(B, T, H, K, V, seed=11, h0=True)
    bf = torch.bfloat16
    q, k, v = (to_dev(d[x], bf, cuda_device) for x in "qkv")
    g, h0 = to_dev(d["g"], torch.float32, cuda_device), to_dev(d["h0"], torch.float32, cuda_device)
    o1, ht1 = fused_recurrent_gla_fwd(q, k, v, g, initial_state=h0, output_final_state=True)
    o2, ht2 = fused_recurrent_gla_fwd(q, k, v, g, initial_state=h0)
    torch.cuda.synchronize()
    assert calls.count(DECODE) == 2 and ht2 is None
    assert torch.equal(o1, o2)
    ro, rht = O.fused_recurrent_fwd(seen(d["q"], bf), seen(d["k"], bf), seen(d["v"], bf), d["g"],
                                    initial_state=d["h0"], output_final_state=True)
    assert rel(host(o1), ro) < 2e-3 and rel(host(ht1), rht) < 2e-3


def test_decode_steps_chain(cuda_device, calls):
    """Eight one-token steps, each starting from the previous step's state, give the outputs
    and final state of one 8-token call (the state cache of a decode loop; the 8-token call
    itself runs on the chunk kernels)."""
    from tops.ops.gla import fused_recurrent_gla
    B, T, H, K, V = 2, 8, 2, 64, 128
    d = gla_inputs(B, T, H, K, V, seed=21, h0=True)
    q, k, v = (to_dev(d[x], torch.float32, cuda_device) for x in "qkv")
    g, h = to_dev(d["g"], torch.float32, cuda_device), to_dev(d["h0"], torch.float32, cuda_device)
    outs = []
    with torch.no_grad():
        for t in range(T):
            s = slice(t, t + 1)
            o_t, h = fused_recurrent_gla(q[:, s], k[:, s], v[:, s], g[:, s], initial_state=h,
                                         output_final_state=True)
            outs.append(o_t)
        o_all, h_all = fused_recurrent_gla(q, k, v, g, initial_state=to_dev(d["h0"], torch.float32,
                                                                              cuda_device),
                                           output_final_state=True)
    torch.cuda.synchronize()
    assert calls.count(DECODE) == T
    assert rel(host(torch.cat(outs, 1)), host(o_all)) < 1e-5 and rel(host(h), host(h_all)) < 1e-5


def test_longer_call_skips_decode(cuda_device, calls):
    """A 5-token call goes to the chunk kernels."""
    from tops.ops.gla import fused_recurrent_gla
    B, T, H, K, V = 2, 5, 2, 64, 64
    d = gla_inputs(B, T, H, K, V, seed=41, h0=True)
    q, k, v = (to_dev(d[x], torch.bfloat16, cuda_device) for x in "qkv")
    with torch.no_grad():
        o, ht = fused_recurrent_gla(q, k, v, to_dev(d["g"], torch.float32, cuda_device),
                                    initial_state=to_dev(d["h0"], torch.float32, cuda_device),
                                    output_final_state=True)
    torch.cuda.synchronize()
    assert DECODE not in calls and "tops_gla_chunk_fwd" in calls
    ro, rht = O.fused_recurrent_fwd(seen(d["q"], torch.bfloat16), seen(d["k"], torch.bfloat16),
                                    seen(d["v"], torch.bfloat16), d["g"], initial_state=d["h0"],
                                    output_final_state=True)
    assert rel(host(o), ro) < 2e-3 and rel(host(ht), rht) < 2e-3


def test_short_call_with_grad_keeps_autograd(cuda_device, calls):
    """With gradients wanted the autograd path runs.  With gk and gv that is the per-token
    entry, whose forward takes the decode kernel itself for T <= 4 (o also in fp32 for the gv
    gradient); its gradients match the oracle's backward."""
    from tops.ops.gla import fused_recurrent_gla
    B, T, H, K, V = 2, 4, 2, 32, 48
    d = gla_inputs(B, T, H, K, V, seed=31, h0=True, grads=True)
    gk, gv = _gates(dict(gate="both"), d, B, T, H, V, 32)
    q, k, v = (to_dev(d[x], torch.float32, cuda_device).requires_grad_() for x in "qkv")
    g = to_dev(gk, torch.float32, cuda_device).requires_grad_()
    gvt = to_dev(gv, torch.float32, cuda_device).requires_grad_()
    h0 = to_dev(d["h0"], torch.float32, cuda_device).requires_grad_()
    o, ht = fused_recurrent_gla(q, k, v, g, gvt, initial_state=h0, output_final_state=True)
    torch.autograd.backward((o, ht), (to_dev(d["do"], torch.float32, cuda_device),
                                      to_dev(d["dht"], torch.float32, cuda_device)))
    torch.cuda.synchronize()
    assert DECODE not in calls and "tops_gla_fused_recurrent_fwd" in calls
    ro, rht = O.fused_recurrent_fwd(d["q"], d["k"], d["v"], gk, gv, initial_state=d["h0"],
                                    output_final_state=True)
    rdq, rdk, rdv, rdg, rdgv, rdh0 = O.fused_recurrent_bwd(d["q"], d["k"], d["v"], gk, gv, ro,
                                                           d["do"], d["dht"], initial_state=d["h0"])
    errs = dict(o=rel(host(o), ro), ht=rel(host(ht), rht), dq=rel(host(q.grad), rdq),
                dk=rel(host(k.grad), rdk), dv=rel(host(v.grad), rdv), dgk=rel(host(g.grad), rdg),
                dgv=rel(host(gvt.grad), rdgv), dh0=rel(host(h0.grad), rdh0))
    print({x: f"{e:.2e}" for x, e in errs.items()})
    assert all(e < 1e-4 for e in errs.values()), errs


@pytest.mark.parametrize("gates", ["g", "gamma", "both", "none"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_simple_gla_decode(gates, dtype, cuda_device, calls):
    """fused_recurrent_simple_gla without gradients on sequences of at most 4 tokens: per-token
    g [B,T,H], g_gamma [H], both or none, on the decode kernel (the gate broadcast over K), vs
    the naive simple-GLA oracle; varlen with an empty and a one-token sequence."""
    from tops.ops.simple_gla import fused_recurrent_simple_gla
    from oracle import simple_gla as S
    from _inputs import simple_gla_inputs
    B, T, H, K, V = 1, 8, 3, 64, 96
    cu = [0, 3, 3, 4, 8]
    d = simple_gla_inputs(B, T, H, K, V, seed=51, h0=True, N=len(cu) - 1)
    g = d["g"] if gates in ("g", "both") else None
    gg = d["g_gamma"] if gates in ("gamma", "both") else None
    q, k, v = (to_dev(d[x], dtype, cuda_device) for x in "qkv")
    with torch.no_grad():
        o, ht = fused_recurrent_simple_gla(q, k, v, g=to_dev(g, torch.float32, cuda_device),
                                           g_gamma=to_dev(gg, torch.float32, cuda_device),
                                           initial_state=to_dev(d["h0"], torch.float32, cuda_device),
                                           output_final_state=True, cu_seqlens=cu)
    torch.cuda.synchronize()
    assert DECODE in calls
    ro, rht = S.naive_simple_gla(seen(d["q"], dtype), seen(d["k"], dtype), seen(d["v"], dtype),
                                 g=g, g_gamma=gg, initial_state=d["h0"], output_final_state=True,
                                 cu_seqlens=cu)
    eo, eh = rel(host(o), ro), rel(host(ht), rht)
    print(f"simple gla decode {gates} {dtype}: o {eo:.2e} ht {eh:.2e}")
    assert eo < tol(dtype) and eh < tol(dtype)


LONG_CASES = [
    dict(B=2, T=9, H=2, K=128, V=128, gate="gk", h0=True),
    dict(B=1, T=20, H=2, K=64, V=96, gate="both", h0=True, reverse=True),
    dict(B=1, T=40, H=2, K=128, V=64, gate="gv", h0=True, cu=[0, 9, 9, 25, 26, 40]),
    dict(B=1, T=33, H=3, K=32, V=128, gate="none", cu=[0, 16, 17, 33]),
    dict(B=3, T=17, H=1, K=36, V=20, gate="gk", h0=True, reverse=True),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("cfg", LONG_CASES, ids=[_id(c) for c in LONG_CASES])
def test_decode_entry_longer_sequences(cfg, dtype, cuda_device):
    """tops_gla_fused_recurrent_fwd_decode called directly through the C ABI on sequences of
    9-20 tokens (the route sends it at most 4): the kernel stages 8 tokens at a time in LDS,
    so these walk two or three token blocks, restaging between them; varlen with empty and
    one-token sequences, reverse, every gate form."""
    from tops import _native as N
    B, T, H, K, V = (cfg[x] for x in "BTHKV")
    cu = cfg.get("cu")
    n = len(cu) - 1 if cu else B
    print(f"decode entry {_id(cfg)} {dtype}", flush=True)
    d = gla_inputs(B, T, H, K, V, seed=T * 3 + K, gate_div=4.0, h0=cfg.get("h0", False), N=n)
    gk, gv = _gates(cfg, d, B, T, H, V, T + V)
    rev = cfg.get("reverse", False)
    f = lambda x: to_dev(x, torch.float32, cuda_device)  # noqa: E731
    q, k, v = (to_dev(d[x], dtype, cuda_device) for x in "qkv")
    gkt, gvt, h0 = f(gk), f(gv), f(d["h0"])
    o = torch.empty_like(v)
    ht = torch.empty(n, H, K, V, device=cuda_device, dtype=torch.float32)
    cut = None if cu is None else torch.tensor(cu, dtype=torch.int32, device=cuda_device)
    scale = K ** -0.5
    N.call("tops_gla_fused_recurrent_fwd_decode", N.ptr(q), N.ptr(k), N.ptr(v), N.ptr(gkt),
           N.ptr(gvt), N.ptr(h0), N.ptr(o), None, N.ptr(ht), N.ptr(cut), B, T, H, K, V, n,
           N.dtype_code(dtype), float(scale), int(rev), N.stream())
    torch.cuda.synchronize()
    ro, rht = O.fused_recurrent_fwd(seen(d["q"], dtype), seen(d["k"], dtype), seen(d["v"], dtype),
                                    gk, gv, scale=scale, initial_state=d["h0"],
                                    output_final_state=True, reverse=rev, cu_seqlens=cu)
    eo, eh = rel(host(o), ro), rel(host(ht), rht)
    print(f"o {eo:.2e} ht {eh:.2e}")
    assert eo < tol(dtype) and eh < tol(dtype)


def test_device_cu_seqlens_routes_without_readback(cuda_device, calls):
    """Boundaries given as a device tensor are not read back on the decode route: a batch of
    one-token sequences (mean length 1) takes the decode kernel, a batch whose mean length is
    above 4 takes the chunk kernels; both against the oracle."""
    from tops.ops.gla import fused_recurrent_gla
    H, K, V = 2, 64, 64
    for cu, want in (([0, 1, 2, 3, 4, 5, 6], True), ([0, 3, 20], False)):
        T = cu[-1]
        d = gla_inputs(1, T, H, K, V, seed=T, h0=True, N=len(cu) - 1)
        q, k, v = (to_dev(d[x], torch.bfloat16, cuda_device) for x in "qkv")
        cut = torch.tensor(cu, dtype=torch.int32, device=cuda_device)
        calls.clear()
        with torch.no_grad():
            o, ht = fused_recurrent_gla(q, k, v, to_dev(d["g"], torch.float32, cuda_device),
                                        initial_state=to_dev(d["h0"], torch.float32, cuda_device),
                                        output_final_state=True, cu_seqlens=cut)
        torch.cuda.synchronize()
        assert (DECODE in calls) == want
        bf = torch.bfloat16
        ro, rht = O.fused_recurrent_fwd(seen(d["q"], bf), seen(d["k"], bf), seen(d["v"], bf),
                                        d["g"], initial_state=d["h0"], output_final_state=True,
                                        cu_seqlens=cu)
        assert rel(host(o), ro) < 2e-3 and rel(host(ht), rht) < 2e-3


NORM_CASES = [
    dict(B=8, T=1, H=4, K=128, V=128, gate="gk", h0=True, og=True, w=True),
    dict(B=2, T=3, H=2, K=64, V=100, gate="both", h0=True, og=True, w=False),
    dict(B=1, T=8, H=3, K=32, V=64, gate="gv", og=False, w=True, cu=[0, 1, 1, 4, 8]),
    dict(B=2, T=4, H=2, K=36, V=20, gate="none", h0=True, og=True, w=True, reverse=True),
    dict(B=1, T=12, H=2, K=128, V=128, gate="gk", h0=True, og=True, w=True, direct=True),
    dict(B=1, T=40, H=2, K=64, V=96, gate="both", h0=True, og=True, w=True, direct=True,
         cu=[0, 9, 9, 25, 26, 40]),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("cfg", NORM_CASES, ids=[_id(c) for c in NORM_CASES])
def test_decode_norm_gate(cfg, dtype, cuda_device, calls):
    """The GLA layer's decode route with its output norm fused into the decode kernel:
    y = RMSNorm(o) * weight * silu(g) over V (tops/layers/gla.py:288-297, 330-336), against
    the oracle's recurrence composed with the norm oracle (oracle.modules.rmsnorm_gated), for
    gk / gv / both / no gate, output gate and weight on and off, reverse, varlen with empty
    sequences, V off the 32-column tile; the `direct` cases call the C entry with sequences of
    up to 20 tokens (several 8-token blocks, the epilogue between their barriers)."""
    from oracle import modules as M
    from tops import _native as N
    from tops.ops.gla import fused_recurrent_gla_norm_gate
    B, T, H, K, V = (cfg[x] for x in "BTHKV")
    cu = cfg.get("cu")
    n = len(cu) - 1 if cu else B
    print(f"decode norm case {_id(cfg)} {dtype}", flush=True)
    d = gla_inputs(B, T, H, K, V, seed=T * 7 + V, gate_div=4.0, h0=cfg.get("h0", False), N=n)
    gk, gv = _gates(cfg, d, B, T, H, V, T + K + 1)
    rng = np.random.Generator(np.random.PCG64(V + T))
    og = rng.standard_normal((B, T, H, V)).astype(np.float32) * 2 if cfg["og"] else None
    w = (1 + 0.3 * rng.standard_normal(V)).astype(np.float32) if cfg["w"] else None
    rev, eps = cfg.get("reverse", False), 1e-5
    f = lambda x: to_dev(x, torch.float32, cuda_device)  # noqa: E731
    q, k, v = (to_dev(d[x], dtype, cuda_device) for x in "qkv")
    ogt = to_dev(og, dtype, cuda_device)
    if cfg.get("direct"):
        y = torch.empty_like(v)
        ht = torch.empty(n, H, K, V, device=cuda_device, dtype=torch.float32)
        cut = None if cu is None else torch.tensor(cu, dtype=torch.int32, device=cuda_device)
        N.call("tops_gla_fused_recurrent_fwd_decode_norm_gate", N.ptr(q), N.ptr(k), N.ptr(v),
               N.ptr(f(gk)), N.ptr(f(gv)), N.ptr(f(d["h0"])), N.ptr(ogt), N.ptr(f(w)), eps,
               N.ptr(y), N.ptr(ht), N.ptr(cut), B, T, H, K, V, n, N.dtype_code(dtype),
               float(K ** -0.5), int(rev), N.stream())
    else:
        with torch.no_grad():
            y, ht = fused_recurrent_gla_norm_gate(q, k, v, f(gk), f(gv), ogt, f(w), eps,
                                                  initial_state=f(d["h0"]), output_final_state=True,
                                                  reverse=rev, cu_seqlens=cu)
        assert "tops_gla_fused_recurrent_fwd_decode_norm_gate" in calls
        assert "tops_rmsnorm_gated_fwd" not in calls
    torch.cuda.synchronize()
    ro, rht = O.fused_recurrent_fwd(seen(d["q"], dtype), seen(d["k"], dtype), seen(d["v"], dtype),
                                    gk, gv, scale=K ** -0.5, initial_state=d["h0"],
                                    output_final_state=True, reverse=rev, cu_seqlens=cu)
    ry = M.rmsnorm_gated(ro, seen(og, dtype), w, eps)
    assert y.dtype == dtype
    ey, eh = rel(host(y), ry), rel(host(ht), rht)
    print(f"y {ey:.2e} ht {eh:.2e}")
    assert ey < out_bound(ry, dtype, dtype) and eh < tol(dtype)


def test_decode_norm_gate_unfused_routes(cuda_device, calls):
    """Calls the fused kernel does not take compose fused_recurrent_gla with the standalone norm
    kernel: a 6-token sequence (chunk kernels), and a decode step with gradients (autograd
    through both ops), each against the oracle; the gradient of y w.r.t. the output gate too."""
    from oracle import modules as M
    from tops.ops.gla import fused_recurrent_gla_norm_gate
    B, H, K, V = 2, 2, 64, 64
    rng = np.random.Generator(np.random.PCG64(3))
    for T, grad in ((6, False), (1, True)):
        calls.clear()
        d = gla_inputs(B, T, H, K, V, seed=60 + T, h0=True)
        og = rng.standard_normal((B, T, H, V)).astype(np.float32)
        w = (1 + 0.3 * rng.standard_normal(V)).astype(np.float32)
        q, k, v = (to_dev(d[x], torch.float32, cuda_device) for x in "qkv")
        g, h0 = to_dev(d["g"], torch.float32, cuda_device), to_dev(d["h0"], torch.float32, cuda_device)
        ogt = to_dev(og, torch.float32, cuda_device).requires_grad_(grad)
        y, ht = fused_recurrent_gla_norm_gate(q, k, v, g, None, ogt, to_dev(w, torch.float32, cuda_device),
                                              initial_state=h0, output_final_state=True)
        if grad:
            dy = rng.standard_normal((B, T, H, V)).astype(np.float32)
            y.backward(to_dev(dy, torch.float32, cuda_device))
        torch.cuda.synchronize()
        assert "tops_gla_fused_recurrent_fwd_decode_norm_gate" not in calls
        assert "tops_rmsnorm_gated_fwd" in calls
        ro, rht = O.fused_recurrent_fwd(d["q"], d["k"], d["v"], d["g"], initial_state=d["h0"],
                                        output_final_state=True)
        assert rel(host(y), M.rmsnorm_gated(ro, og, w, 1e-5)) < 1e-4
        assert rel(host(ht), rht) < 1e-4
        if grad:
            rdg = M.rmsnorm_gated_bwd(ro, og, w, dy, 1e-5)[1]
            assert rel(host(ogt.grad), rdg) < 1e-4


CONV_CASES = [
    dict(B=8, T=1, H=4, K=128, V=128, W=4, bias=True, act="silu", cache=True, og=True, w=True),
    dict(B=1, T=5, H=2, K=64, V=96, W=3, bias=False, act=None, cache=True, og=True, w=False,
         cu=[0, 1, 2, 3, 4, 5]),
    dict(B=2, T=3, H=2, K=32, V=64, W=4, bias=True, act="silu", cache=True, og=False, w=True),
    dict(B=1, T=5, H=2, K=64, V=64, W=4, bias=True, act="silu", cache=False, og=True, w=True,
         cu=[0, 2, 2, 5]),
    dict(B=4, T=1, H=2, K=36, V=20, W=2, bias=True, act="swish", cache=False, og=True, w=True),
    dict(B=2, T=1, H=3, K=128, V=128, W=8, bias=False, act="silu", cache=True, og=True, w=True,
         wdt="bf16"),
]


def _cid(c):
    return "-".join(f"{k}{v}" for k, v in c.items() if k != "cu") + ("-varlen" if "cu" in c else "")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("cfg", CONV_CASES, ids=[_cid(c) for c in CONV_CASES])
def test_decode_conv_norm_gate(cfg, dtype, cuda_device, calls):
    """The GLA layer's decode route from the projections to the normalised output as one kernel
    (ShortConvolution q / k / v -> fused_recurrent_gla -> FusedRMSNormGated), against the
    oracle's conv step (one token per sequence: the caches roll) or prefill (the caches are not
    read; the new ones are the last W inputs, zero-padded), per-token recurrence and norm:
    y, the final state and the three new conv caches; W 2-8, SiLU or none, bias on / off,
    varlen with an empty sequence, no cache, and bf16 conv weights (then y in bf16)."""
    from oracle import modules as M
    from tops.ops.gla import fused_recurrent_gla_conv_norm_gate
    B, T, H, K, V, W = (cfg[x] for x in "BTHKVW")
    cu = cfg.get("cu")
    n = len(cu) - 1 if cu else B
    step = B * T == n
    print(f"decode conv case {_cid(cfg)} {dtype}", flush=True)
    rng = np.random.Generator(np.random.PCG64(B * T + K + V + W))
    d = gla_inputs(B, T, H, K, V, seed=T + K + W, gate_div=4.0, h0=True, N=n)
    xs = [rng.standard_normal((B, T, H, D)).astype(np.float32) for D in (K, K, V)]
    dims = (H * K, H * K, H * V)
    ws = [(rng.standard_normal((D, W)) / np.sqrt(W)).astype(np.float32) for D in dims]
    wdt = torch.bfloat16 if cfg.get("wdt") == "bf16" else torch.float32
    if wdt == torch.bfloat16:
        ws = [bf16_round(w) for w in ws]
    bs = [rng.standard_normal(D).astype(np.float32) * 0.1 for D in dims] if cfg["bias"] else [None] * 3
    cs = [rng.standard_normal((n, D, W)).astype(np.float32) for D in dims] if cfg["cache"] else [None] * 3
    og = (rng.standard_normal((B, T, H, V)) * 2).astype(np.float32) if cfg["og"] else None
    nw = (1 + 0.3 * rng.standard_normal(V)).astype(np.float32) if cfg["w"] else None
    f = lambda x: to_dev(x, torch.float32, cuda_device)  # noqa: E731
    with torch.no_grad():
        y, ht, new = fused_recurrent_gla_conv_norm_gate(
            *(to_dev(x, dtype, cuda_device) for x in xs),
            tuple(to_dev(w, wdt, cuda_device) for w in ws),
            None if not cfg["bias"] else tuple(f(b) for b in bs),
            None if not cfg["cache"] else tuple(f(c) for c in cs),
            cfg["act"], f(d["g"]), to_dev(og, dtype, cuda_device), f(nw), 1e-5,
            initial_state=f(d["h0"]), output_final_state=True, cu_seqlens=cu)
    torch.cuda.synchronize()
    assert "tops_gla_decode_conv_norm_gate" in calls
    ydt = torch.promote_types(dtype, wdt)
    assert y.dtype == ydt
    # oracle: the three convolutions, the recurrence, the norm
    sx = [seen(x, dtype) for x in xs]
    conv_out, conv_new = [], []
    for x, w, b, c, D in zip(sx, ws, bs, cs, dims):
        x3 = x.reshape(B, T, D)
        if step:
            xin = x3[0] if cu else x3[:, 0]
            yv, cn = M.short_conv_step(xin, c if c is not None else np.zeros((n, D, W)), w, b, cfg["act"])
            yv = yv.reshape(B, T, D)
        else:
            yv = M.short_conv(x3, w, b, cfg["act"], cu)
            cn = M.short_conv_final_state(x3, W, cu)
        conv_out.append(yv.reshape(x.shape))
        conv_new.append(cn)
    ro, rht = O.fused_recurrent_fwd(*conv_out, d["g"], None, scale=K ** -0.5,
                                    initial_state=d["h0"], output_final_state=True, cu_seqlens=cu)
    ry = M.rmsnorm_gated(ro, seen(og, dtype), nw, 1e-5)
    ey, eh = rel(host(y), ry), rel(host(ht), rht)
    ec = [rel(host(a), b) for a, b in zip(new, conv_new)]
    print(f"y {ey:.2e} ht {eh:.2e} caches {[f'{e:.1e}' for e in ec]}")
    lim = out_bound(ry, ydt, ydt)
    assert ey < lim and eh < 1e-4 and max(ec) < 1e-6
