"""KDA gate activation, gate cumsum, L2 norm and the FLA options of fused_recurrent_kda /
chunk_kda on MI355X, against the float64 oracle (oracle/kda_gate.py restating
tops/cpu/ops/kda/gate.py and tops/ops/kda/gate.py; oracle/kda.py for the recurrence).

Covers both gate modes, A_log / dt_bias head broadcast (base and expanded bias, fewer
parameter heads than gate heads), fp32 and bf16 gate inputs, the deterministic dA / dbias
reduction over many row blocks, both call forms of kda_gate_chunk_cumsum (fixed and varlen,
chunk sizes 8 / 16 / 64), and fused_recurrent_kda with the gate and q / k L2 norm in the
kernel, grouped heads, varlen and the transposed state layout, forward and backward (the
chained gradients down to A_log and dt_bias).
Tolerances: elementwise fp32 results 2e-6 (relative L2; libm-accurate exp / log1p in fp32),
reductions 1e-5, recurrences fp32 1e-4 / bf16 2e-3.
"""
import math

import numpy as np
import pytest
import torch

from oracle import kda as KO
from oracle import kda_gate as G
from _gpu import to_dev, seen, host, rel, tol

pytestmark = pytest.mark.gpu

EW = 2e-6    # elementwise fp32
RED = 1e-5   # fp32 sums over many elements


def _params(H, K, Ha, bias, seed, a_scale=1.0):
    rng = np.random.Generator(np.random.PCG64(seed))
    A_log = np.log(rng.uniform(1.0, 4.0, Ha) * a_scale).astype(np.float32)
    b = None
    if bias == "base":
        b = rng.standard_normal(Ha * K).astype(np.float32)
    elif bias == "full":
        b = rng.standard_normal(H * K).astype(np.float32)
    return A_log, b


GATE_CASES = [
    dict(H=4, Ha=4, bias=None),
    dict(H=4, Ha=4, bias="base"),
    dict(H=4, Ha=2, bias="base"),
    dict(H=4, Ha=2, bias="full"),
    dict(H=6, Ha=1, bias="full"),
]


def _gid(c):
    return f"H{c['H']}-Ha{c['Ha']}-{c['bias']}"


@pytest.mark.parametrize("lb", [None, -5.0], ids=["softplus", "lb"])
@pytest.mark.parametrize("gdt", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("cfg", GATE_CASES, ids=_gid)
def test_gate_forward_backward(cfg, gdt, lb, cuda_device):
    from tops.ops.kda import fused_kda_gate, kda_gate_bwd
    H, Ha, K = cfg["H"], cfg["Ha"], 64
    rng = np.random.Generator(np.random.PCG64(H + Ha))
    g = (2 * rng.standard_normal((2, 33, H, K))).astype(np.float32)
    dy = rng.standard_normal(g.shape).astype(np.float32)
    A_log, b = _params(H, K, Ha, cfg["bias"], seed=H * Ha)
    print(f"gate {_gid(cfg)} {gdt} lb={lb}", flush=True)
    gt = to_dev(g, gdt, cuda_device).requires_grad_()
    At = to_dev(A_log, torch.float32, cuda_device).requires_grad_()
    bt = to_dev(b, torch.float32, cuda_device)
    if bt is not None:
        bt.requires_grad_()
    y = fused_kda_gate(gt, At, dt_bias=bt, lower_bound=lb)
    assert y.dtype == torch.float32 and y.shape == gt.shape
    y.backward(to_dev(dy, torch.float32, cuda_device))
    sg = seen(g, gdt)
    ry = G.kda_gate(sg, A_log, b, lower_bound=lb)
    rdg, rdA, rdb = G.kda_gate_bwd(sg, A_log, b, dy, lower_bound=lb)
    e = dict(y=rel(host(y), ry), dg=rel(host(gt.grad), rdg), dA=rel(host(At.grad), rdA))
    if b is not None:
        e["db"] = rel(host(bt.grad), rdb)
    print(" ".join(f"{n}={v:.2e}" for n, v in e.items()))
    assert e["y"] < EW
    assert e["dg"] < (EW if gdt == torch.float32 else 2e-3)   # dg is stored in g's dtype
    assert e["dA"] < RED and e.get("db", 0.0) < RED
    assert gt.grad.dtype == gdt
    # the functional backward gives the same numbers
    dg2, dA2, db2 = kda_gate_bwd(gt.detach(), At.detach(), None if bt is None else bt.detach(),
                                 to_dev(dy, torch.float32, cuda_device), lower_bound=lb)
    assert torch.equal(dg2, gt.grad) and torch.equal(dA2, At.grad)
    assert (db2 is None) == (b is None)


def test_gate_backward_many_row_blocks_is_deterministic(cuda_device):
    """Long token axis: the dA / dbias partials of many workgroups, reduced in a fixed order,
    give the oracle's sums and bit-identical results on every call."""
    from tops.ops.kda import kda_gate_bwd
    B, T, H, K = 4, 1000, 4, 128
    rng = np.random.Generator(np.random.PCG64(11))
    g = rng.standard_normal((B, T, H, K)).astype(np.float32)
    dy = rng.standard_normal(g.shape).astype(np.float32)
    A_log, b = _params(H, K, 2, "base", seed=12)
    args = (to_dev(g, torch.float32, cuda_device), to_dev(A_log, torch.float32, cuda_device),
            to_dev(b, torch.float32, cuda_device))
    dyt = to_dev(dy, torch.float32, cuda_device)
    for lb in (None, -3.0):
        r1 = kda_gate_bwd(*args, dyg=dyt, lower_bound=lb)
        r2 = kda_gate_bwd(*args, dyg=dyt, lower_bound=lb)
        for a, c in zip(r1, r2):
            assert torch.equal(a, c)
        rdg, rdA, rdb = G.kda_gate_bwd(g, A_log, b, dy, lower_bound=lb)
        e = (rel(host(r1[0]), rdg), rel(host(r1[1]), rdA), rel(host(r1[2]), rdb))
        print(f"lb={lb} dg={e[0]:.2e} dA={e[1]:.2e} db={e[2]:.2e}")
        assert e[0] < EW and e[1] < RED and e[2] < RED


def test_naive_gates_and_output_dtype(cuda_device):
    from tops.ops.kda import naive_kda_gate, naive_kda_lowerbound_gate, kda_gate_fwd
    rng = np.random.Generator(np.random.PCG64(2))
    g = rng.standard_normal((1, 9, 2, 16)).astype(np.float32)
    A_log, b = _params(2, 16, 2, "full", seed=3)
    gt, At, bt = (to_dev(x, torch.float32, cuda_device) for x in (g, A_log, b))
    y1 = naive_kda_gate(gt, At, bt)
    y2 = naive_kda_lowerbound_gate(gt, At, bt)            # default lower_bound = -5
    y3 = kda_gate_fwd(gt, At, bt, output_dtype=torch.bfloat16)
    assert rel(host(y1), G.kda_gate(g, A_log, b)) < EW
    assert rel(host(y2), G.kda_gate(g, A_log, b, lower_bound=-5.0)) < EW
    assert y3.dtype == torch.bfloat16 and rel(host(y3), G.kda_gate(g, A_log, b)) < 4e-3


CUMSUM_CASES = [
    dict(B=2, T=130, H=2, K=64, C=64),
    dict(B=1, T=19, H=2, K=8, C=8, cu=[0, 7, 19]),
    dict(B=3, T=77, H=3, K=128, C=16),
    dict(B=1, T=300, H=2, K=32, C=64, cu=[0, 1, 65, 200, 300]),
]


@pytest.mark.parametrize("gdt", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("cfg", CUMSUM_CASES,
                         ids=lambda c: f"B{c['B']}-T{c['T']}-H{c['H']}-K{c['K']}-C{c['C']}"
                         + ("-varlen" if "cu" in c else ""))
def test_gate_chunk_cumsum_both_forms(cfg, gdt, cuda_device):
    from tops.ops.kda import kda_gate_chunk_cumsum
    B, T, H, K, C = (cfg[x] for x in ("B", "T", "H", "K", "C"))
    cu = cfg.get("cu")
    rng = np.random.Generator(np.random.PCG64(T + K))
    graw = rng.standard_normal((B, T, H, K)).astype(np.float32)
    A_log, b = _params(H, K, H, "full", seed=T)
    sg = seen(graw, gdt)
    gt = to_dev(graw, gdt, cuda_device)
    # accelerator form: activated natural-log gates in, log2 chunk cumsum out
    out = kda_gate_chunk_cumsum(gt, C, cu)
    assert out.dtype == torch.float32
    e1 = rel(host(out), G.kda_gate_chunk_cumsum(sg, C, cu_seqlens=cu))
    # FLA form: raw gates activated in the kernel, natural-log cumsum times scale
    At, bt = to_dev(A_log, torch.float32, cuda_device), to_dev(b, torch.float32, cuda_device)
    out2 = kda_gate_chunk_cumsum(gt, At, C, scale=1 / math.log(2), dt_bias=bt, cu_seqlens=cu)
    ref2 = G.kda_gate_chunk_cumsum(G.kda_gate(sg, A_log, b), C, cu_seqlens=cu)
    e2 = rel(host(out2), ref2)
    out3 = kda_gate_chunk_cumsum(gt, At, chunk_size=C, dt_bias=bt, cu_seqlens=cu, lower_bound=-1.0)
    ref3 = G.kda_gate_chunk_cumsum(G.kda_gate(sg, A_log, b, lower_bound=-1.0), C,
                                   cu_seqlens=cu) * math.log(2)
    e3 = rel(host(out3), ref3)
    print(f"accel={e1:.2e} fla={e2:.2e} fla_lb={e3:.2e}")
    assert e1 < EW and e2 < EW and e3 < EW


@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("D", [32, 64, 100, 128, 256])
def test_l2norm_forward_backward(D, xdt, cuda_device):
    from tops.ops.kda import l2norm
    rng = np.random.Generator(np.random.PCG64(D))
    x = rng.standard_normal((3, 37, 2, D)).astype(np.float32)
    x[0, 0, 0] = 0.0                                  # an all-zero row: y = 0, dx = dy / 1e-3
    dy = rng.standard_normal(x.shape).astype(np.float32)
    xt = to_dev(x, xdt, cuda_device).requires_grad_()
    y = l2norm(xt)
    y.backward(to_dev(dy, torch.float32, cuda_device))
    sx = seen(x, xdt)
    e_y = rel(host(y), G.l2norm(sx))
    e_dx = rel(host(xt.grad), G.l2norm_bwd(sx, dy))
    print(f"y={e_y:.2e} dx={e_dx:.2e}")
    assert y.dtype == torch.float32 and xt.grad.dtype == xdt
    assert e_y < EW
    assert e_dx < (1e-5 if xdt == torch.float32 else 2e-3)


# ---------------------------------------------------------------- fused_recurrent_kda

FR_CASES = [
    dict(B=2, T=100, H=2, HV=2, K=64, V=64, gate="base", l2=True, h0=True),
    dict(B=1, T=150, H=1, HV=2, K=128, V=64, gate="full", lb=-0.5, l2=True, h0=True),
    dict(B=2, T=70, H=2, HV=2, K=64, V=128, gate=None, l2=False, h0=True),
    dict(B=1, T=200, H=2, HV=4, K=64, V=64, gate="base", l2=True, h0=True,
         cu=[0, 30, 31, 140, 200], transpose=True),
    dict(B=1, T=90, H=2, HV=2, K=32, V=32, gate="base", l2=False, h0=False, cu=[0, 45, 90]),
]


def _fid(c):
    s = f"B{c['B']}-T{c['T']}-H{c['H']}-HV{c['HV']}-K{c['K']}-V{c['V']}-g{c['gate']}"
    s += "-lb" if "lb" in c else ""
    s += "-l2" if c["l2"] else ""
    s += "-varlen" if "cu" in c else ""
    s += "-tr" if c.get("transpose") else ""
    return s


def _fr_inputs(c, seed):
    B, T, H, HV, K, V = (c[x] for x in ("B", "T", "H", "HV", "K", "V"))
    cu = c.get("cu")
    n = len(cu) - 1 if cu else B
    rng = np.random.Generator(np.random.PCG64(seed))
    d = dict(q=rng.standard_normal((B, T, H, K)), k=rng.standard_normal((B, T, H, K)),
             v=rng.standard_normal((B, T, HV, V)),
             beta=1 / (1 + np.exp(-rng.standard_normal((B, T, H)))),
             do=rng.standard_normal((B, T, HV, V)),
             dht=0.1 * rng.standard_normal((n, HV, K, V)),
             h0=0.1 * rng.standard_normal((n, HV, K, V)) if c["h0"] else None)
    if not c["l2"]:   # the recurrence wants normalised keys; give it normalised inputs
        d["q"], d["k"] = G.l2norm(d["q"]), G.l2norm(d["k"])
    if c["gate"]:
        d["g"] = rng.standard_normal((B, T, H, K))
        d["A_log"], d["dt_bias"] = _params(HV, K, HV // 2 if HV % 2 == 0 else HV, c["gate"],
                                           seed + 1, a_scale=1 / 32)
    else:
        d["g"] = np.log(1 / (1 + np.exp(-rng.standard_normal((B, T, H, K))))) / 16
    return {x: (None if y is None else np.asarray(y, np.float32)) for x, y in d.items()}


def _fold(x, H):
    """Sum the repeated heads of [B, T, HV, ...] back to H heads."""
    B, T, HV = x.shape[:3]
    return x.reshape(B, T, H, HV // H, *x.shape[3:]).sum(3)


def _fr_oracle(c, d, dtype, scale):
    H, HV = c["H"], c["HV"]
    rep = HV // H
    cu = c.get("cu")
    sq, sk, sv, sdo = (seen(d[x], dtype) for x in ("q", "k", "v", "do"))
    qh, kh = (np.repeat(x, rep, 2) for x in (sq, sk))
    gh = np.repeat(d["g"].astype(np.float64), rep, 2)
    bh = np.repeat(d["beta"].astype(np.float64), rep, 2)
    qn, kn = (G.l2norm(qh), G.l2norm(kh)) if c["l2"] else (qh, kh)
    lb = c.get("lb")
    ga = G.kda_gate(gh, d["A_log"], d["dt_bias"], lower_bound=lb) if c["gate"] else gh
    segs = [(0, sq.shape[1], None)] if cu is None else [(cu[i], cu[i + 1], i) for i in range(len(cu) - 1)]
    parts = {x: [] for x in ("o", "dq", "dk", "dv", "db", "dg")}
    hts, dh0s = [], []
    h0, dht = d["h0"], d["dht"]
    for s, e, n in segs:
        sl = (slice(None), slice(s, e))
        h0n = None if h0 is None else (h0 if n is None else h0[n:n + 1])
        dhtn = dht if n is None else dht[n:n + 1]
        o, ht = KO.chunk_kda(qn[sl], kn[sl], sv[sl], ga[sl], bh[sl], scale, h0n, True)
        dq, dk, dv, db, dg, dh0 = KO.chunk_kda_bwd(qn[sl], kn[sl], sv[sl], ga[sl], bh[sl], scale,
                                                   h0n, sdo[sl], dhtn)
        for key, val in zip(("o", "dq", "dk", "dv", "db", "dg"), (o, dq, dk, dv, db, dg)):
            parts[key].append(val)
        hts.append(ht)
        dh0s.append(dh0)
    r = {key: np.concatenate(v, axis=1) for key, v in parts.items()}
    r["ht"] = np.concatenate(hts, 0)
    if h0 is not None:
        r["dh0"] = np.concatenate(dh0s, 0)
    if c["l2"]:
        r["dq"], r["dk"] = G.l2norm_bwd(qh, r["dq"]), G.l2norm_bwd(kh, r["dk"])
    if c["gate"]:
        r["dg"], r["dA"], r["dbias"] = G.kda_gate_bwd(gh, d["A_log"], d["dt_bias"], r["dg"],
                                                      lower_bound=lb)
    r["dq"], r["dk"], r["dg"], r["db"] = (_fold(r[x], H) for x in ("dq", "dk", "dg", "db"))
    return r


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("cfg", FR_CASES, ids=_fid)
def test_fused_recurrent_kda_fla_options(cfg, dtype, cuda_device):
    from tops.ops.kda import fused_recurrent_kda
    print(f"case {_fid(cfg)} {dtype}", flush=True)
    d = _fr_inputs(cfg, seed=cfg["T"] + cfg["K"])
    tr = cfg.get("transpose", False)
    dev = cuda_device
    q, k, v = (to_dev(d[x], dtype, dev).requires_grad_() for x in "qkv")
    g = to_dev(d["g"], torch.float32, dev).requires_grad_()
    beta = to_dev(d["beta"], torch.float32, dev).requires_grad_()
    h0 = to_dev(d["h0"], torch.float32, dev)
    if h0 is not None:
        h0 = (h0.transpose(-1, -2).contiguous() if tr else h0).requires_grad_()
    kw = {}
    A = bias = None
    if cfg["gate"]:
        A = to_dev(d["A_log"], torch.float32, dev).requires_grad_()
        bias = to_dev(d["dt_bias"], torch.float32, dev).requires_grad_()
        kw = dict(A_log=A, dt_bias=bias, use_gate_in_kernel=True, lower_bound=cfg.get("lb"))
    scale = cfg["K"] ** -0.5
    o, ht = fused_recurrent_kda(q, k, v, g, beta, scale, h0, True,
                                use_qk_l2norm_in_kernel=cfg["l2"], cu_seqlens=cfg.get("cu"),
                                transpose_state_layout=tr, **kw)
    assert o.dtype == dtype and ht.dtype == torch.float32
    dht = to_dev(d["dht"], torch.float32, dev)
    torch.autograd.backward((o, ht), (to_dev(d["do"], dtype, dev),
                                      dht.transpose(-1, -2).contiguous() if tr else dht))
    torch.cuda.synchronize()
    r = _fr_oracle(cfg, d, dtype, scale)

    def st(x):   # states back to [N, HV, K, V]
        return None if x is None else (np.swapaxes(x, -1, -2) if tr else x)
    got = dict(o=host(o), ht=st(host(ht)), dq=host(q.grad), dk=host(k.grad), dv=host(v.grad),
               db=host(beta.grad), dg=host(g.grad))
    if h0 is not None:
        got["dh0"] = st(host(h0.grad))
    if A is not None:
        got["dA"], got["dbias"] = host(A.grad), host(bias.grad)
    # the l2-normalised path runs the recurrence in fp32 whatever the input dtype
    t = 1e-4 if (dtype == torch.float32 or cfg["l2"]) else 2e-3
    errs = {x: rel(got[x], r[x]) for x in got}
    print(" ".join(f"{x}={e:.2e}" for x, e in errs.items()))
    for x, e in errs.items():
        lim = 2e-3 if (x in ("o", "dq", "dk", "dv") and dtype == torch.bfloat16) else t
        assert e < lim, (x, e)


def test_fused_recurrent_kda_fwd_and_bwd_apis(cuda_device):
    """fused_recurrent_kda_fwd (inplace_final_state / out) matches the public call and leaves
    initial_state untouched; fused_recurrent_kda_bwd returns the gradients of the recurrence's
    own inputs (normalised q, k; activated gate), as tops/cpu/ops/kda/fused_recurrent.py does."""
    from tops.ops.kda import (fused_recurrent_kda, fused_recurrent_kda_bwd,
                              fused_recurrent_kda_fwd)
    cfg = dict(B=2, T=80, H=2, HV=2, K=64, V=64, gate="base", l2=True, h0=True)
    d = _fr_inputs(cfg, seed=5)
    dev = cuda_device
    q, k, v, g, beta = (to_dev(d[x], torch.float32, dev) for x in ("q", "k", "v", "g", "beta"))
    h0 = to_dev(d["h0"], torch.float32, dev)
    A, bias = to_dev(d["A_log"], torch.float32, dev), to_dev(d["dt_bias"], torch.float32, dev)
    kw = dict(A_log=A, dt_bias=bias, use_gate_in_kernel=True, use_qk_l2norm_in_kernel=True)
    h0_before = h0.clone()
    o1, s1 = fused_recurrent_kda(q, k, v, g, beta, None, h0, True, **kw)
    o2, s2 = fused_recurrent_kda_fwd(q, k, v, g, beta, initial_state=h0, **kw)
    out = torch.zeros_like(v, dtype=torch.bfloat16)
    o3, _ = fused_recurrent_kda_fwd(q, k, v, g, beta, initial_state=h0, out=out,
                                    inplace_final_state=False, **kw)
    assert torch.equal(h0, h0_before)
    assert torch.equal(o1, o2) and torch.equal(s1, s2)
    assert o3 is out and o3.dtype == torch.bfloat16
    assert rel(host(o3), host(o1)) < 4e-3
    with pytest.raises(AssertionError):
        fused_recurrent_kda_fwd(q, k, v, g, beta, **kw)          # inplace needs initial_state

    do, dht = to_dev(d["do"], torch.float32, dev), to_dev(d["dht"], torch.float32, dev)
    dq, dk, dv, dg, db, dh0 = fused_recurrent_kda_bwd(q, k, v, g, beta, do, A_log=A, dt_bias=bias,
                                                      initial_state=h0, dht=dht, **{
                                                          x: kw[x] for x in
                                                          ("use_gate_in_kernel",
                                                           "use_qk_l2norm_in_kernel")})
    qn, kn = G.l2norm(d["q"]), G.l2norm(d["k"])
    ga = G.kda_gate(d["g"], d["A_log"], d["dt_bias"])
    scale = cfg["K"] ** -0.5
    ref = KO.chunk_kda_bwd(qn, kn, d["v"], ga, d["beta"], scale, d["h0"], d["do"], d["dht"])
    for name, a, b in zip(("dq", "dk", "dv", "db", "dg", "dh0"), (dq, dk, dv, db, dg, dh0), ref):
        e = rel(host(a), b)
        print(f"{name}={e:.2e}", end=" ")
        assert e < 1e-4, (name, e)


def test_chunk_kda_gate_in_kernel(cuda_device):
    """chunk_kda(use_gate_in_kernel=True): raw gates activated ahead of the chunk kernels,
    gradients reaching A_log and dt_bias (tops/cpu/ops/kda/chunk_bwd.py:617-668)."""
    from tops.ops.kda import chunk_kda
    cfg = dict(B=2, T=130, H=2, HV=2, K=128, V=128, gate="base", lb=-1.0, l2=False, h0=True)
    d = _fr_inputs(cfg, seed=21)
    dev = cuda_device
    dtype = torch.bfloat16
    q, k, v = (to_dev(d[x], dtype, dev).requires_grad_() for x in "qkv")
    g = to_dev(d["g"], torch.bfloat16, dev).requires_grad_()      # raw gate in bf16
    beta = to_dev(d["beta"], torch.float32, dev).requires_grad_()
    h0 = to_dev(d["h0"], torch.float32, dev).requires_grad_()
    A = to_dev(d["A_log"], torch.float32, dev).requires_grad_()
    bias = to_dev(d["dt_bias"], torch.float32, dev).requires_grad_()
    o, ht = chunk_kda(q, k, v, g, beta, initial_state=h0, output_final_state=True, A_log=A,
                      dt_bias=bias, use_gate_in_kernel=True, lower_bound=cfg["lb"])
    torch.autograd.backward((o, ht), (to_dev(d["do"], dtype, dev),
                                      to_dev(d["dht"], torch.float32, dev)))
    torch.cuda.synchronize()
    d2 = dict(d)
    d2["g"] = seen(d["g"], torch.bfloat16).astype(np.float32)
    r = _fr_oracle(cfg, d2, dtype, cfg["K"] ** -0.5)
    got = dict(o=host(o), ht=host(ht), dq=host(q.grad), dk=host(k.grad), dv=host(v.grad),
               db=host(beta.grad), dh0=host(h0.grad), dA=host(A.grad), dbias=host(bias.grad))
    for x, a in got.items():
        e = rel(a, r[x])
        print(f"{x}={e:.2e}", end=" ")
        assert e < 2e-3, (x, e)
    # dg lands in g's dtype (bf16)
    assert g.grad.dtype == torch.bfloat16 and rel(host(g.grad), r["dg"]) < 4e-3


DECODE_CASES = [
    dict(B=4, T=1, H=2, HV=2, K=128, V=128, gate="base", l2=True, h0=True),
    dict(B=2, T=3, H=1, HV=2, K=64, V=96, gate="full", lb=-0.5, l2=True, h0=True),
    dict(B=2, T=4, H=2, HV=2, K=40, V=24, gate=None, l2=False, h0=True),
    dict(B=1, T=6, H=2, HV=4, K=64, V=64, gate="base", l2=True, h0=True, cu=[0, 1, 4, 6],
         transpose=True),
    dict(B=1, T=2, H=2, HV=2, K=32, V=32, gate=None, l2=False, h0=False, cu=[0, 1, 2]),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("cfg", DECODE_CASES, ids=_fid)
def test_fused_recurrent_kda_decode(cfg, dtype, cuda_device, monkeypatch):
    """fused_recurrent_kda without gradients on sequences of at most 4 tokens runs on the KDA
    decode kernel (tops_kda_fused_recurrent_fwd_decode), with the FLA options (gate in kernel,
    lower bound, q / k L2 norm, grouped heads, varlen, transposed state layout); o and the final
    state against the oracle."""
    from tops import _native as N
    from tops.ops.kda import fused_recurrent_kda
    names, real = [], N.call
    monkeypatch.setattr(N, "call", lambda name, *a: (names.append(name), real(name, *a))[1])
    d = _fr_inputs(cfg, seed=cfg["T"] + cfg["K"] + 1)
    tr = cfg.get("transpose", False)
    dev = cuda_device
    q, k, v = (to_dev(d[x], dtype, dev) for x in "qkv")
    g, beta = to_dev(d["g"], torch.float32, dev), to_dev(d["beta"], torch.float32, dev)
    h0 = to_dev(d["h0"], torch.float32, dev)
    if h0 is not None and tr:
        h0 = h0.transpose(-1, -2).contiguous()
    kw = {}
    if cfg["gate"]:
        kw = dict(A_log=to_dev(d["A_log"], torch.float32, dev),
                  dt_bias=to_dev(d["dt_bias"], torch.float32, dev), use_gate_in_kernel=True,
                  lower_bound=cfg.get("lb"))
    scale = cfg["K"] ** -0.5
    with torch.no_grad():
        o, ht = fused_recurrent_kda(q, k, v, g, beta, scale, h0, True,
                                    use_qk_l2norm_in_kernel=cfg["l2"], cu_seqlens=cfg.get("cu"),
                                    transpose_state_layout=tr, **kw)
    torch.cuda.synchronize()
    assert "tops_kda_fused_recurrent_fwd_decode" in names and "tops_kda_chunk_fwd" not in names
    r = _fr_oracle(cfg, d, dtype, scale)
    hto = host(ht)
    eo, eh = rel(host(o), r["o"]), rel(np.swapaxes(hto, -1, -2) if tr else hto, r["ht"])
    print(f"kda decode {_fid(cfg)} {dtype}: o {eo:.2e} ht {eh:.2e}")
    t = 1e-4 if (dtype == torch.float32 or cfg["l2"]) else 2e-3
    assert eo < (2e-3 if dtype == torch.bfloat16 else t) and eh < t


KDA_LONG = [dict(B=2, T=9, H=2, K=128, V=128, h0=True), dict(B=1, T=20, H=2, K=64, V=96, h0=True),
            dict(B=1, T=40, H=2, K=128, V=64, h0=True, cu=[0, 9, 9, 25, 26, 40]),
            dict(B=1, T=33, H=1, K=32, V=128, h0=False, cu=[0, 16, 17, 33])]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("cfg", KDA_LONG,
                         ids=[f"T{c['T']}K{c['K']}V{c['V']}{'-varlen' if 'cu' in c else ''}"
                              for c in KDA_LONG])
def test_kda_decode_entry_longer_sequences(cfg, dtype, cuda_device):
    """tops_kda_fused_recurrent_fwd_decode called directly through the C ABI on sequences of
    9-20 tokens (the route sends it at most 4): two or three 8-token LDS blocks per sequence,
    varlen with empty and one-token sequences; o and the final state against the per-token
    recurrence (tops/cpu/ops/kda/naive.py:10-118)."""
    from tops import _native as N
    from _inputs import kda_inputs
    B, T, H, K, V = (cfg[x] for x in "BTHKV")
    cu = cfg.get("cu")
    n = len(cu) - 1 if cu else B
    print(f"kda decode entry T{T} K{K} V{V} {dtype}", flush=True)
    d = kda_inputs(B, T, H, K, V, seed=T + 2 * K, gate_div=4.0, h0=cfg["h0"], N=n)
    q, k, v = (to_dev(d[x], dtype, cuda_device) for x in "qkv")
    g, beta = (to_dev(d[x], torch.float32, cuda_device) for x in ("g", "beta"))
    h0 = to_dev(d["h0"], torch.float32, cuda_device)
    o = torch.empty_like(v)
    ht = torch.empty(n, H, K, V, device=cuda_device, dtype=torch.float32)
    cut = None if cu is None else torch.tensor(cu, dtype=torch.int32, device=cuda_device)
    scale = K ** -0.5
    N.call("tops_kda_fused_recurrent_fwd_decode", N.ptr(q), N.ptr(k), N.ptr(v), N.ptr(g),
           N.ptr(beta), N.ptr(h0), N.ptr(o), N.ptr(ht), N.ptr(cut), B, T, H, K, V, n,
           N.dtype_code(dtype), float(scale), N.stream())
    torch.cuda.synchronize()
    sq, sk, sv = (seen(d[x], dtype) for x in "qkv")
    spans = [(b, 0, T) for b in range(B)] if cu is None else \
        [(0, cu[i], cu[i + 1]) for i in range(n)]
    ro = np.zeros((B, T, H, V))
    rht = np.zeros((n, H, K, V))
    for i, (b, s, e) in enumerate(spans):
        h0i = None if d["h0"] is None else d["h0"][i:i + 1]
        oo, hh = KO.naive_recurrent_kda(sq[b:b + 1, s:e], sk[b:b + 1, s:e], sv[b:b + 1, s:e],
                                        d["g"][b:b + 1, s:e], d["beta"][b:b + 1, s:e], scale, h0i,
                                        True)
        ro[b, s:e] = oo[0]
        rht[i] = hh[0]
    eo, eh = rel(host(o), ro), rel(host(ht), rht)
    print(f"o {eo:.2e} ht {eh:.2e}")
    assert eo < tol(dtype) and eh < tol(dtype)
