"""GLA stage functions on MI355X against the float64 oracle: the chunk-local cumsum
(tops.ops.gla.chunk_local_cumsum / tops.ops.common.cumsum.chunk_local_cumsum_vector), the
state recurrence (chunk_fwd_h, tops.ops.common.chunk_h forward and backward, all gate
kinds), and the chunk-parallel stages (intra A, o, dA, dv, intra dq/dk, inter dq/dk/dg).
Then the stages composed as the reference's chunk_gla_fwd / chunk_gla_bwd compose them
must reproduce chunk_gla's output and autograd gradients.

Shapes follow the reference's stage tests (tests/ops/gla/test_pallas_chunk_*.py): chunk
sizes 8-128 for the cumsum and 16-128 elsewhere, K up to 256, V up to 256, varlen with
chunk-aligned boundaries.  Tolerances (relative L2): results kept in fp32 1e-5 (fp32
products vs float64), results stored in bf16 4e-3 (one rounding), the composition 1e-4.
"""
import numpy as np
import pytest
import torch

from oracle import common as OC
from oracle import gla as O
from _gpu import to_dev, seen, host, rel

pytestmark = pytest.mark.gpu

F32, BF = 1e-5, 4e-3


def _lim(dt):
    return F32 if dt == torch.float32 else BF


CUMSUM_CASES = [
    dict(B=2, T=32, H=4, K=128, C=16),
    dict(B=2, T=32, H=3, K=128, C=8, reverse=True, scale=0.5),
    dict(B=1, T=33, H=2, K=128, C=16, scale=0.75, cu=[0, 17, 33]),
    dict(B=1, T=33, H=2, K=128, C=16, reverse=True, cu=[0, 17, 33]),
    dict(B=3, T=128, H=6, K=128, C=32, scale=0.125),
    dict(B=2, T=64, H=4, K=128, C=16, hf=True),
    dict(B=2, T=64, H=3, K=128, C=16, reverse=True, scale=0.5, hf=True),
    dict(B=2, T=32, H=4, K=128, C=16, scale=0.125, out=torch.bfloat16),
    dict(B=2, T=32, H=4, K=64, C=16),
    dict(B=2, T=32, H=2, K=256, C=16),
    dict(B=2, T=32, H=2, K=192, C=16),
    dict(B=2, T=16, H=4, K=128, C=16),
    dict(B=1, T=56, H=2, K=128, C=16, cu=[0, 8, 40, 56]),
    dict(B=2, T=64, H=4, K=128, C=32, reverse=True),
    dict(B=8, T=1024, H=64, K=128, C=64, hf=True),
    dict(B=1, T=2048, H=64, K=128, C=128, cu=[0, 512, 888, 2048]),
    dict(B=2, T=100, H=3, K=1, C=16, ind=torch.bfloat16),
    dict(B=1, T=50, H=2, K=64, C=16, hf=True, reverse=True, cu=[0, 20, 50]),
    dict(B=1, T=0, H=2, K=8, C=16),
]


def _cid(c):
    s = f"B{c['B']}-T{c['T']}-H{c['H']}-K{c['K']}-C{c['C']}"
    for k in ("reverse", "hf"):
        if c.get(k):
            s += f"-{k}"
    if c.get("scale") is not None:
        s += f"-s{c['scale']}"
    if "cu" in c:
        s += "-varlen"
    if "out" in c:
        s += "-bf16out"
    if "ind" in c:
        s += "-bf16in"
    return s


@pytest.mark.parametrize("c", CUMSUM_CASES, ids=_cid)
def test_chunk_local_cumsum(c, cuda_device):
    from tops.ops.gla import chunk_local_cumsum
    from tops.ops.common.cumsum import chunk_local_cumsum_vector
    print(f"cumsum {_cid(c)}", flush=True)
    rng = np.random.default_rng(c["T"] * 7 + c["K"])
    hf = c.get("hf", False)
    shape = (c["B"], c["H"], c["T"], c["K"]) if hf else (c["B"], c["T"], c["H"], c["K"])
    g = rng.standard_normal(shape).astype(np.float32)
    ind = c.get("ind", torch.float32)
    gt = to_dev(g, ind, cuda_device)
    out_dt = c.get("out", torch.float32)
    kw = dict(reverse=c.get("reverse", False), scale=c.get("scale"), head_first=hf,
              output_dtype=out_dt, cu_seqlens=c.get("cu"))
    o1 = chunk_local_cumsum(gt, c["C"], **kw)
    o2 = chunk_local_cumsum_vector(gt, c["C"], **kw)
    assert o1.dtype == out_dt and o1.shape == gt.shape
    assert torch.equal(o1, o2)
    ref = OC.chunk_local_cumsum_segments(seen(g, ind), c["C"], kw["reverse"], c.get("cu"), hf,
                                         kw["scale"])
    e = rel(host(o1), ref)
    print(f"rel={e:.2e}")
    assert e < _lim(out_dt)


def _gates(rng, B, T, H, K, C, kinds, cu=None):
    """Raw gates per kind, their chunk-local cumsums and the total per-channel cumsum."""
    out = {}
    total = np.zeros((B, T, H, K))
    if "gk" in kinds:
        gk = np.log(1 / (1 + np.exp(-rng.standard_normal((B, T, H, K))))) / 4
        out["gk"] = OC.chunk_local_cumsum_segments(gk, C, cu_seqlens=cu)
        total += out["gk"]
    if "g" in kinds:
        g = np.log(1 / (1 + np.exp(-rng.standard_normal((B, T, H))))) / 4
        out["g"] = OC.chunk_local_cumsum_segments(g[..., None], C, cu_seqlens=cu)[..., 0]
        total += out["g"][..., None]
    if "g_gamma" in kinds:
        gam = -np.linspace(0.02, 0.2, H)
        out["g_gamma"] = gam
        ramp = np.broadcast_to(gam, (B, T, H))[..., None]
        total += OC.chunk_local_cumsum_segments(ramp, C, cu_seqlens=cu)
    return out, total


STATE_CASES = [
    dict(B=2, T=64, H=4, K=32, V=64, C=16, gates=("gk",)),
    dict(B=1, T=128, H=2, K=32, V=64, C=32, gates=("gk",), h0=True),
    dict(B=2, T=256, H=1, K=256, V=128, C=64, gates=("g", "gk", "g_gamma"), h0=True),
    dict(B=1, T=256, H=2, K=256, V=128, C=128, gates=("g_gamma",)),
    dict(B=2, T=256, H=4, K=128, V=256, C=64, gates=("g", "gk", "g_gamma")),
    dict(B=1, T=128, H=2, K=128, V=256, C=64, gates=("gk",), h0=True),
    dict(B=2, T=128, H=2, K=64, V=48, C=32, gates=("g",), h0=True),
    dict(B=1, T=256, H=2, K=64, V=64, C=32, gates=("gk", "g"), h0=True, cu=[0, 64, 96, 256]),
    dict(B=2, T=256, H=2, K=128, V=128, C=64, gates=("gk",), split=128),
    dict(B=1, T=64, H=1, K=16, V=16, C=16, gates=()),
]


def _sid(c):
    s = f"B{c['B']}-T{c['T']}-H{c['H']}-K{c['K']}-V{c['V']}-C{c['C']}-{'+'.join(c['gates']) or 'nogate'}"
    if c.get("h0"):
        s += "-h0"
    if "cu" in c:
        s += "-varlen"
    if "split" in c:
        s += f"-split{c['split']}"
    return s


def _oracle_states(x, y, total, s0, C, cu, reverse, scale):
    """Oracle state recurrence per sequence, states at absolute chunk positions."""
    B, T, H, K = x.shape
    V = y.shape[-1]
    segs = [(b, 0, T) for b in range(B)] if cu is None else [(0, a, e) for a, e in zip(cu[:-1], cu[1:])]
    states = np.zeros((B, T // C, H, K, V))
    finals = []
    for n, (b, a, e) in enumerate(segs):
        sl = (slice(b, b + 1), slice(a, e))
        init = None if s0 is None else s0[n:n + 1]
        if reverse:
            hs, hf = OC.chunk_bwd_dh(x[sl], y[sl], gk=total[sl], dht=init, scale=scale, C=C)
        else:
            hs, hf = OC.chunk_fwd_h(x[sl], y[sl], gk=total[sl], h0=init, C=C)
        states[b, a // C:e // C] = hs[0]
        finals.append(hf[0])
    return states, np.stack(finals)


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("c", STATE_CASES, ids=_sid)
def test_state_recurrence(c, dt, cuda_device):
    from tops.ops.common.chunk_h import (chunk_bwd_dh_kernel, chunk_bwd_dh_ref, chunk_fwd_h_kernel,
                                         chunk_fwd_h_ref)
    from tops.ops.gla import chunk_fwd_h
    print(f"state {_sid(c)} {dt}", flush=True)
    B, T, H, K, V, C = (c[x] for x in ("B", "T", "H", "K", "V", "C"))
    cu = c.get("cu")
    rng = np.random.default_rng(T + K + V + C)
    q, k = (rng.standard_normal((B, T, H, K)).astype(np.float32) for _ in range(2))
    v, do = (rng.standard_normal((B, T, H, V)).astype(np.float32) for _ in range(2))
    Nseq = B if cu is None else len(cu) - 1
    s0 = rng.standard_normal((Nseq, H, K, V)) * 0.1 if c.get("h0") else None
    gates, total = _gates(rng, B, T, H, K, C, c["gates"], cu)
    d = lambda x: to_dev(x, dt, cuda_device)
    f = lambda x: None if x is None else to_dev(x, torch.float32, cuda_device)
    gk_t, g_t, gg_t = f(gates.get("gk")), f(gates.get("g")), f(gates.get("g_gamma"))
    scale = K ** -0.5
    hs_ref, ht_ref = _oracle_states(seen(k, dt), seen(v, dt), total, s0, C, cu, False, 1.0)
    dh_ref, dh0_ref = _oracle_states(seen(q, dt), seen(do, dt), total, s0, C, cu, True, scale)
    lim = _lim(dt)
    split = c.get("split")
    if split:
        h, ht = chunk_fwd_h_kernel(d(k), d(v), g=g_t, g_gamma=gg_t, gk=gk_t, h0=f(s0),
                                   output_final_state=True, chunk_size=C, split_size=split)
        assert h.shape == (B, T // split, H, K, V) and h.dtype == dt
        e = rel(host(h), hs_ref[:, ::split // C])
        print(f"split h={e:.2e}")
        assert e < lim and rel(host(ht), ht_ref) < F32
        return
    h, ht = chunk_fwd_h_ref(d(k), d(v), g=g_t, g_gamma=gg_t, gk=gk_t, h0=f(s0),
                            output_final_state=True, cu_seqlens_cpu=cu, chunk_size=C)
    assert h.dtype == dt and ht.dtype == torch.float32
    hk, htk = chunk_fwd_h_kernel(d(k), d(v), g=g_t, g_gamma=gg_t, gk=gk_t, h0=f(s0),
                                 output_final_state=False, cu_seqlens_cpu=cu, chunk_size=C,
                                 states_in_fp32=True)
    assert htk is None and hk.dtype == torch.float32
    dh, dh0 = chunk_bwd_dh_ref(d(q), d(k), d(v), g_t, gg_t, gk_t, d(do), h0=None, dht=f(s0),
                               scale=scale, output_dh0=True, cu_seqlens_cpu=cu, chunk_size=C)
    dhk, dh0k = chunk_bwd_dh_kernel(d(q), d(k), d(v), g=g_t, g_gamma=gg_t, gk=gk_t, do=d(do),
                                    dht=f(s0), scale=scale, output_dh0=True, cu_seqlens_dev=cu,
                                    chunk_size=C)
    assert dh.dtype == torch.float32 and dhk.dtype == dt and dh0k.dtype == dt
    e = dict(h=rel(host(h), hs_ref), ht=rel(host(ht), ht_ref), h32=rel(host(hk), hs_ref),
             dh=rel(host(dh), dh_ref), dh0=rel(host(dh0), dh0_ref), dhk=rel(host(dhk), dh_ref))
    print(" ".join(f"{n}={x:.2e}" for n, x in e.items()))
    assert e["h"] < lim and e["dhk"] < lim
    for n in ("ht", "h32", "dh", "dh0"):
        assert e[n] < F32, n
    if "gk" in c["gates"] and len(c["gates"]) == 1:
        h2, ht2 = chunk_fwd_h(d(k), d(v), gk_t, f(s0), False, cu, C)
        assert torch.equal(h2, h) and float(ht2.abs().max()) == 0.0


STAGE_CASES = [
    dict(B=2, T=64, H=4, K=32, V=64, C=16),
    dict(B=1, T=128, H=2, K=32, V=64, C=32),
    dict(B=2, T=256, H=2, K=128, V=128, C=64),
    dict(B=1, T=256, H=1, K=256, V=128, C=128),
    dict(B=1, T=128, H=2, K=80, V=48, C=64),
]


def _tid(c):
    return f"B{c['B']}-T{c['T']}-H{c['H']}-K{c['K']}-V{c['V']}-C{c['C']}"


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("c", STAGE_CASES, ids=_tid)
def test_chunk_parallel_stages(c, dt, cuda_device):
    from tops.ops.gla import (chunk_gla_bwd_dA_ref, chunk_gla_bwd_dqk_intra_ref,
                              chunk_gla_bwd_dqkg_ref, chunk_gla_bwd_dv_ref,
                              chunk_gla_fwd_intra_gk, chunk_gla_fwd_o_gk)
    print(f"stages {_tid(c)} {dt}", flush=True)
    B, T, H, K, V, C = (c[x] for x in ("B", "T", "H", "K", "V", "C"))
    NT = T // C
    rng = np.random.default_rng(B * T + K + V + C)
    q, k = (rng.standard_normal((B, T, H, K)).astype(np.float32) for _ in range(2))
    v, do = (rng.standard_normal((B, T, H, V)).astype(np.float32) for _ in range(2))
    gc = OC.chunk_local_cumsum(np.log(1 / (1 + np.exp(-rng.standard_normal((B, T, H, K))))) / 4, C)
    hs = rng.standard_normal((B, NT, H, K, V)) * 0.3
    dh = rng.standard_normal((B, NT, H, K, V)) * 0.3
    A_full = rng.standard_normal((B, T, H, C)) * 0.2
    dA_in = rng.standard_normal((B, T, H, C)) * 0.2
    dq_in, dk_in = rng.standard_normal((2, B, T, H, K))
    scale = K ** -0.5
    d = lambda x: to_dev(x, dt, cuda_device)
    f = lambda x: to_dev(x, torch.float32, cuda_device)
    sq, sk, sv, sdo = (seen(x, dt) for x in (q, k, v, do))
    lim = _lim(dt)
    errs = {}

    A = chunk_gla_fwd_intra_gk(d(q), d(k), f(gc), scale, C)
    assert A.dtype == torch.float32 and A.shape == (B, T, H, C)
    errs["A"] = (rel(host(A), O.chunk_gla_fwd_intra_gk(sq, sk, gc, scale, C)), F32)

    o = chunk_gla_fwd_o_gk(d(q), d(v), f(gc), f(A_full), f(hs), scale, chunk_size=C)
    assert o.dtype == dt
    ro = O.chunk_gla_fwd_o_gk(sq, sv, gc, O.causal_mask_A(A_full, C), hs, scale, C)
    errs["o"] = (rel(host(o), ro), lim)
    o2 = chunk_gla_fwd_o_gk(d(q), d(v), f(gc), f(A_full), f(hs), scale, chunk_size=C, use_exp2=True)
    ro2 = O.chunk_gla_fwd_o_gk(sq, sv, gc * np.log(2.0), O.causal_mask_A(A_full, C), hs, scale, C)
    errs["o_exp2"] = (rel(host(o2), ro2), lim)

    dA = chunk_gla_bwd_dA_ref(d(v), d(do), scale, chunk_size=C)
    assert dA.dtype == dt
    errs["dA"] = (rel(host(dA), O.chunk_gla_bwd_dA(sv, sdo, scale, C)), lim)

    dv = chunk_gla_bwd_dv_ref(d(k), f(gc), f(A_full), d(do), f(dh), chunk_size=C)
    assert dv.dtype == torch.float32
    errs["dv"] = (rel(host(dv), O.chunk_gla_bwd_dv(sk, gc, O.causal_mask_A(A_full, C), sdo, dh, C)), F32)

    dq, dk = chunk_gla_bwd_dqk_intra_ref(d(q), d(k), f(gc), f(dA_in), chunk_size=C)
    rdq, rdk = O.chunk_gla_bwd_dqk_intra(sq, sk, gc, dA_in, C)
    errs["dq_intra"] = (rel(host(dq), rdq), F32)
    errs["dk_intra"] = (rel(host(dk), rdk), F32)

    dq2, dk2, dg = chunk_gla_bwd_dqkg_ref(d(q), d(k), d(v), f(hs), f(gc), d(do), f(dh), f(dq_in),
                                          f(dk_in), scale, chunk_size=C)
    rq, rk, rg = O.chunk_gla_bwd_dqkg(sq, sk, sv, hs, gc, sdo, dh, dq_in, dk_in, scale, C)
    errs["dq"] = (rel(host(dq2), rq), F32)
    errs["dk"] = (rel(host(dk2), rk), F32)
    errs["dg"] = (rel(host(dg), rg), F32)
    print(" ".join(f"{n}={e:.2e}" for n, (e, _) in errs.items()))
    for n, (e, lim_n) in errs.items():
        assert e < lim_n, (n, e)


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_stages_compose_to_chunk_gla(dt, cuda_device):
    """cumsum -> chunk_fwd_h -> intra A -> o, and chunk_bwd_dh -> dA -> dv -> intra dq/dk ->
    dqkg, as tops/ops/gla/chunk.py:832-997 and :1103-1199 chain them, give chunk_gla's o,
    final state and autograd gradients."""
    from tops.ops.gla import (chunk_fwd_h, chunk_gla, chunk_gla_bwd_dA_ref,
                              chunk_gla_bwd_dqk_intra_ref, chunk_gla_bwd_dqkg_ref,
                              chunk_gla_bwd_dv_ref, chunk_gla_fwd_intra_gk, chunk_gla_fwd_o_gk,
                              chunk_local_cumsum)
    from tops.ops.common.chunk_h import chunk_bwd_dh_ref
    B, T, H, K, V, C = 2, 256, 2, 128, 128, 64
    gen = torch.Generator(device=cuda_device).manual_seed(77)
    r = lambda *s: torch.randn(*s, device=cuda_device, generator=gen)
    q, k, v = (r(B, T, H, D).to(dt) for D in (K, K, V))
    g = torch.nn.functional.logsigmoid(r(B, T, H, K)) / 8
    h0 = r(B, H, K, V) * 0.1
    do = r(B, T, H, V).to(dt)
    dht = r(B, H, K, V) * 0.1
    scale = K ** -0.5
    ins = [x.clone().requires_grad_() for x in (q, k, v, g, h0)]
    o_ref, ht_ref = chunk_gla(*ins[:4], scale=scale, initial_state=ins[4], output_final_state=True)
    grads = torch.autograd.grad((o_ref, ht_ref), ins, (do, dht))

    gc = chunk_local_cumsum(g, C)
    h, ht = chunk_fwd_h(k, v, gc, h0, True, None, C)
    assert h.dtype == dt
    h32 = chunk_fwd_h(k.float(), v.float(), gc, h0, False, None, C)[0]   # fp32 states
    A = chunk_gla_fwd_intra_gk(q, k, gc, scale, C)
    o = chunk_gla_fwd_o_gk(q, v, gc, A, h32, scale, chunk_size=C)
    dh, dh0 = chunk_bwd_dh_ref(q, k, v, None, None, gc, do, h0=h0, dht=dht, scale=scale,
                               output_dh0=True, chunk_size=C)
    dA = chunk_gla_bwd_dA_ref(v, do, scale, chunk_size=C)
    dv = chunk_gla_bwd_dv_ref(k, gc, A, do, dh, chunk_size=C)
    dq, dk = chunk_gla_bwd_dqk_intra_ref(q, k, gc, dA, chunk_size=C)
    dq, dk, dg = chunk_gla_bwd_dqkg_ref(q, k, v, h32, gc, do, dh, dq, dk, scale, chunk_size=C)
    mine = dict(o=o, ht=ht, dq=dq, dk=dk, dv=dv, dg=dg, dh0=dh0)
    # the stages against the float64 oracle of chunk_gla on the same (bf16-rounded) inputs:
    # they compute in fp32 whatever the input dtype
    sq, sk, sv, sdo = (host(x) for x in (q, k, v, do))
    ro, rht = O.chunk_gla(sq, sk, sv, host(g), scale, host(h0), True, chunk_size=C)
    rb = O.chunk_gla_bwd(sq, sk, sv, host(g), scale, host(h0), sdo, host(dht), chunk_size=C)
    ref = dict(o=ro, ht=rht, **dict(zip(("dq", "dk", "dv", "dg", "dh0"), rb)))
    errs = {n: rel(host(mine[n]), ref[n]) for n in mine}
    print("vs oracle: " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()))
    # bf16 inputs: o is stored in bf16, and dA (hence dq, dk, dg) is held in bf16 as the
    # reference's dA = einsum(do, v) of bf16 operands is; states and dv stay fp32
    for n, e in errs.items():
        lim = 2e-3 if dt == torch.bfloat16 and n in ("o", "dq", "dk", "dg") else 1e-4
        assert e < lim, (n, e)
    # and against chunk_gla's own output and autograd gradients (fp32: both fp32-accurate)
    if dt == torch.float32:
        errs = {n: rel(host(mine[n]), host(b)) for n, b in
                zip(("o", "ht", "dq", "dk", "dv", "dg", "dh0"), (o_ref, ht_ref) + tuple(grads))}
        print("vs chunk_gla: " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()))
        for n, e in errs.items():
            assert e < 1e-4, (n, e)


# tests/ops/kda/test_chunk_kda_tpu.py:31-52 (shapes as NT chunks of C)
KDA_INTRA = [
    dict(B=2, H=4, NT=2, C=16, K=32), dict(B=1, H=2, NT=4, C=16, K=16),
    dict(B=2, H=4, NT=1, C=32, K=16), dict(B=1, H=2, NT=2, C=64, K=32),
    dict(B=1, H=2, NT=2, C=16, K=64), dict(B=1, H=2, NT=2, C=16, K=128),
    dict(B=2, H=1, NT=2, C=16, K=32), dict(B=1, H=1, NT=4, C=32, K=64),
    dict(B=1, H=2, NT=3, C=16, K=32), dict(B=2, H=4, NT=5, C=16, K=16),
    dict(B=1, H=2, NT=7, C=32, K=32), dict(B=4, H=4, NT=2, C=16, K=32),
    dict(B=8, H=2, NT=2, C=16, K=16), dict(B=2, H=8, NT=4, C=16, K=16),
    dict(B=1, H=4, NT=8, C=16, K=16), dict(B=1, H=4, NT=16, C=64, K=128),
    dict(B=1, H=2, NT=3, C=64, K=80),
]


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("c", KDA_INTRA, ids=lambda c: "B{B}-H{H}-NT{NT}-C{C}-K{K}".format(**c))
def test_chunk_kda_bwd_intra(c, dt, cuda_device):
    from tops.ops.kda import chunk_kda_bwd_intra
    from oracle import kda as KO
    B, H, NT, C, K = (c[x] for x in ("B", "H", "NT", "C", "K"))
    T = NT * C
    print(f"kda intra bwd B={B} H={H} T={T} C={C} K={K} {dt}", flush=True)
    rng = np.random.default_rng(B * 1000 + H * 100 + NT * 10 + K)
    q, k = (rng.standard_normal((B, T, H, K)).astype(np.float32) * 0.5 for _ in range(2))
    g = (OC.chunk_local_cumsum(-np.abs(rng.standard_normal((B, T, H, K))) * 0.1, C)
         / np.log(2.0)).astype(np.float32)
    beta = (1 / (1 + np.exp(-rng.standard_normal((B, T, H))))).astype(np.float32)
    tri = np.tril(np.ones((C, C)))[None, None, :, None, :]
    stri = np.tril(np.ones((C, C)), -1)[None, None, :, None, :]
    dAqk = (rng.standard_normal((B, NT, C, H, C)) * tri).reshape(B, T, H, C).astype(np.float32)
    dAkk = (rng.standard_normal((B, NT, C, H, C)) * stri).reshape(B, T, H, C).astype(np.float32)
    inc = [rng.standard_normal(s).astype(np.float32) for s in ((B, T, H, K), (B, T, H, K),
                                                                (B, T, H), (B, T, H, K))]
    f = lambda x: to_dev(x, torch.float32, cuda_device)
    sq, sk = seen(q, dt), seen(k, dt)
    rq, rk, rb, rg = KO.chunk_kda_bwd_intra(sq, sk, g, beta, dAqk, dAkk, C)
    # standalone: outputs in q's dtype
    out = chunk_kda_bwd_intra(to_dev(q, dt, cuda_device), to_dev(k, dt, cuda_device), f(g), f(beta),
                              f(dAqk), f(dAkk), chunk_size=C)
    assert all(o.dtype == dt for o in out)
    errs = {n: rel(host(o), r) for n, o, r in zip(("dq", "dk", "db", "dg"), out, (rq, rk, rb, rg))}
    # accumulating into fp32 incoming gradients
    out2 = chunk_kda_bwd_intra(to_dev(q, dt, cuda_device), to_dev(k, dt, cuda_device), f(g), f(beta),
                               f(dAqk), f(dAkk), *(f(x) for x in inc), chunk_size=C)
    for n, o, r, x in zip(("dq", "dk", "db", "dg"), out2, (rq, rk, rb, rg), inc):
        assert o.dtype == torch.float32
        errs[n + "+in"] = rel(host(o), r + x)
    print(" ".join(f"{n}={e:.2e}" for n, e in errs.items()))
    for n, e in errs.items():
        lim = F32 if ("+in" in n or dt == torch.float32) else BF
        assert e < lim, (n, e)


SIMPLE_CASES = [
    dict(B=2, T=128, H=2, K=64, V=64, C=32, gate="g"),
    dict(B=1, T=256, H=4, K=128, V=128, C=64, gate="g_gamma"),
    dict(B=2, T=128, H=2, K=128, V=64, C=64, gate="both"),
    dict(B=1, T=64, H=2, K=32, V=48, C=16, gate="none"),
]


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("c", SIMPLE_CASES, ids=lambda c: "{gate}-B{B}-T{T}-K{K}-V{V}-C{C}".format(**c))
def test_simple_gla_common_stages(c, dt, cuda_device):
    """tops.ops.common.chunk_o / fused_chunk: the scalar-gate stages against the GLA oracle
    stages on the gate broadcast over K (and the raw-dg oracle)."""
    from tops.ops.common import (chunk_bwd_dqkwg, chunk_bwd_dv, chunk_fwd_o,
                                 chunk_simple_gla_bwd_o_pl, fused_chunk_fwd)
    from oracle import simple_gla as SO
    B, T, H, K, V, C = (c[x] for x in ("B", "T", "H", "K", "V", "C"))
    NT = T // C
    print(f"simple stages {c} {dt}", flush=True)
    rng = np.random.default_rng(T + K + V + C + len(c["gate"]))
    q, k = (rng.standard_normal((B, T, H, K)).astype(np.float32) for _ in range(2))
    v, do = (rng.standard_normal((B, T, H, V)).astype(np.float32) for _ in range(2))
    hs, dh = rng.standard_normal((2, B, NT, H, K, V)) * 0.3
    h0 = rng.standard_normal((B, H, K, V)) * 0.3
    g = OC.chunk_local_cumsum(-np.abs(rng.standard_normal((B, T, H))) * 0.1, C) \
        if c["gate"] in ("g", "both") else None
    gam = -np.linspace(0.01, 0.1, H) if c["gate"] in ("g_gamma", "both") else None
    G = np.zeros((B, T, H))
    if g is not None:
        G = G + g
    if gam is not None:
        G = G + ((np.arange(T) % C + 1)[:, None] * gam[None, :])[None]
    Gk = np.repeat(G[..., None], K, axis=-1)
    scale = K ** -0.5
    d = lambda x: to_dev(x, dt, cuda_device)
    f = lambda x: None if x is None else to_dev(x, torch.float32, cuda_device)
    sq, sk, sv, sdo = (seen(x, dt) for x in (q, k, v, do))
    A = O.causal_mask_A(O.chunk_gla_fwd_intra_gk(sq, sk, Gk, scale, C), C)
    errs = {}
    o = chunk_fwd_o(d(q), d(k), d(v), f(hs), g=f(g), g_gamma=f(gam), scale=scale, chunk_size=C)
    assert o.dtype == dt
    errs["o"] = (rel(host(o), O.chunk_gla_fwd_o_gk(sq, sv, Gk, A, hs, scale, C)), _lim(dt))
    dv = chunk_bwd_dv(d(q), d(k), d(do), f(dh), g=f(g), g_gamma=f(gam), scale=scale, chunk_size=C)
    errs["dv"] = (rel(host(dv), O.chunk_gla_bwd_dv(sk, Gk, A, sdo, dh, C)), _lim(dt))
    dq, dk, dw, dg = chunk_bwd_dqkwg(d(q), d(k), d(v), f(hs), d(do), f(dh), g=f(g), g_gamma=f(gam),
                                     scale=scale, chunk_size=C, w=d(k), dv=d(do))
    dA = O.chunk_gla_bwd_dA(sv, sdo, scale, C)
    rqi, rki = O.chunk_gla_bwd_dqk_intra(sq, sk, Gk, dA, C)
    rq, rk, _ = O.chunk_gla_bwd_dqkg(sq, sk, sv, hs, Gk, sdo, dh, rqi, rki, scale, C)
    errs["dq"] = (rel(host(dq), rq), F32)
    errs["dk"] = (rel(host(dk), rk), F32)
    rdw = -np.einsum("bnchv,bnhkv->bnchk", sdo.reshape(B, NT, C, H, V), hs).reshape(B, T, H, K)
    errs["dw"] = (rel(host(dw), rdw), _lim(dt))
    if g is None:
        assert dg is None
    else:
        rdg = SO.chunk_bwd_dqkwg_raw_dg(sq, sk, sv, hs, sdo, dh, G, scale, C)
        errs["dg"] = (rel(host(dg), rdg), 1e-4)
    if gam is not None and g is None:
        pq, pk, pv = chunk_simple_gla_bwd_o_pl(d(q), d(k), d(v), f(gam), f(hs), d(do), f(dh),
                                               scale, C)
        assert pq.dtype == dt and pv.dtype == dt
        errs["pl_dq"] = (rel(host(pq), rq), _lim(dt))
        errs["pl_dv"] = (rel(host(pv), O.chunk_gla_bwd_dv(sk, Gk, A, sdo, dh, C)), _lim(dt))
    o2, ht = fused_chunk_fwd(d(q), d(k), d(v), g=f(g), g_gamma=f(gam), h0=f(h0), scale=scale,
                             use_ht=True, chunk_size=C)
    rh, rht = OC.chunk_fwd_h(sk, sv, gk=Gk, h0=h0, C=C)
    errs["fused_o"] = (rel(host(o2), O.chunk_gla_fwd_o_gk(sq, sv, Gk, A, rh, scale, C)), _lim(dt))
    errs["fused_ht"] = (rel(host(ht), rht), F32)
    print(" ".join(f"{n}={e:.2e}" for n, (e, _) in errs.items()))
    for n, (e, lim) in errs.items():
        assert e < lim, (n, e)


@pytest.mark.parametrize("case", [dict(T=256, cu=None, h0=True), dict(T=300, cu=[0, 100, 300], h0=True),
                                  dict(T=128, cu=None, h0=False, C=32)],
                         ids=["fixed", "varlen", "C32-noh0"])
def test_chunk_kda_bwd_functional(case, cuda_device):
    """tops.ops.kda.chunk_bwd.chunk_kda_bwd (the reference's functional backward on the log2
    gate cumsum) = chunk_kda's autograd, with dg in log2 units (ln 2 times the natural-log
    gradient), as the reference's custom_vjp relates them (tops/ops/kda/chunk.py:230-252)."""
    from tops.ops.kda import chunk_kda
    from tops.ops.kda.chunk_bwd import chunk_kda_bwd
    from tops.ops.common.cumsum import chunk_local_cumsum_vector
    T, cu = case["T"], case["cu"]
    B, H, K, V = 1, 2, 64, 64
    C = case.get("C", 64)
    gen = torch.Generator(device=cuda_device).manual_seed(T)
    r = lambda *s: torch.randn(*s, device=cuda_device, generator=gen)
    l2 = lambda x: x / x.norm(dim=-1, keepdim=True)
    q, k = l2(r(B, T, H, K)), l2(r(B, T, H, K))
    v = r(B, T, H, V)
    g = torch.nn.functional.logsigmoid(r(B, T, H, K)) / 8
    beta = torch.sigmoid(r(B, T, H))
    n = 1 if cu is None else len(cu) - 1
    h0 = r(n, H, K, V) * 0.1 if case["h0"] else None
    do, dht = r(B, T, H, V), r(n, H, K, V) * 0.1
    ins = [x.clone().requires_grad_() for x in (q, k, v, g, beta)]
    hin = None if h0 is None else h0.clone().requires_grad_()
    o, ht = chunk_kda(*ins, initial_state=hin, output_final_state=True, cu_seqlens=cu)
    grads = torch.autograd.grad((o, ht), ins + ([hin] if hin is not None else []), (do, dht))
    g2 = chunk_local_cumsum_vector(g, C, scale=1 / np.log(2.0), cu_seqlens=cu)
    dq, dk, dv, db, dg, dh0, dA, dbias = chunk_kda_bwd(q, k, v, beta, None, None, K ** -0.5, h0, do,
                                                       dht, g=g2, cu_seqlens=cu, chunk_size=C)
    assert dA is None and dbias is None and (dh0 is None) == (h0 is None)
    errs = dict(dq=rel(host(dq), host(grads[0])), dk=rel(host(dk), host(grads[1])),
                dv=rel(host(dv), host(grads[2])), dg=rel(host(dg), host(grads[3]) * np.log(2.0)),
                db=rel(host(db), host(grads[4])))
    if h0 is not None:
        errs["dh0"] = rel(host(dh0), host(grads[5]))
    print(" ".join(f"{n_}={e:.2e}" for n_, e in errs.items()))
    for n_, e in errs.items():
        assert e < 1e-4, (n_, e)


VARLEN_H_CASES = [
    dict(T=512, H=2, K=128, V=128, C=128, cu=[0, 128, 384, 512], gates=("gk",), h0=True),
    dict(T=256, H=2, K=64, V=64, C=64, cu=[0, 64, 256], gates=("gk", "g_gamma"), h0=False),
    dict(T=192, H=1, K=32, V=64, C=64, cu=[0, 192], gates=("g_gamma",), h0=True),
]


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("c", VARLEN_H_CASES, ids=lambda c: "T{T}-H{H}-K{K}-V{V}-C{C}-".format(**c) + "+".join(c["gates"]))
def test_chunk_fwd_h_kernel_varlen(c, dt, cuda_device):
    """chunk_fwd_h_kernel_varlen (tops/ops/common/chunk_h.py:970-1113): the state before every
    chunk of a packed varlen stream [NT, H, K, V] and the final states, against the oracle's
    per-sequence recurrence; the scalar gate g and gv are rejected as in the reference."""
    from tops.ops.common import chunk_fwd_h_kernel_varlen
    T, H, K, V, C, cu = (c[x] for x in ("T", "H", "K", "V", "C", "cu"))
    rng = np.random.default_rng(T + K + C)
    k = rng.standard_normal((1, T, H, K)).astype(np.float32)
    v = rng.standard_normal((1, T, H, V)).astype(np.float32)
    n = len(cu) - 1
    s0 = rng.standard_normal((n, H, K, V)) * 0.1 if c["h0"] else None
    gates, total = _gates(rng, 1, T, H, K, C, c["gates"], cu)
    f = lambda x: None if x is None else to_dev(x, torch.float32, cuda_device)
    print(f"chunk_fwd_h_kernel_varlen {c} {dt}", flush=True)
    h, ht = chunk_fwd_h_kernel_varlen(to_dev(k, dt, cuda_device), to_dev(v, dt, cuda_device),
                                      g_gamma=f(gates.get("g_gamma")), gk=f(gates.get("gk")),
                                      h0=f(s0), output_final_state=True,
                                      cu_seqlens_dev=torch.tensor(cu, dtype=torch.int32, device=cuda_device),
                                      chunk_size=C, states_in_fp32=True)
    hs_ref, ht_ref = _oracle_states(seen(k, dt), seen(v, dt), total, s0, C, cu, False, 1.0)
    assert h.shape == (T // C, H, K, V) and h.dtype == torch.float32
    assert rel(host(h), hs_ref[0]) < _lim(dt) and rel(host(ht), ht_ref) < F32
    with pytest.raises(AssertionError):
        chunk_fwd_h_kernel_varlen(to_dev(k, dt, cuda_device), to_dev(v, dt, cuda_device),
                                  g=torch.zeros(1, T, H, device=cuda_device), cu_seqlens_dev=cu,
                                  chunk_size=C)


@pytest.mark.parametrize("c", [dict(B=2, T=128, H=2, K=128, V=128, h0=False, dht=False),
                               dict(B=1, T=128, H=2, K=128, V=128, h0=True, dht=False),
                               dict(B=1, T=128, H=2, K=128, V=128, h0=False, dht=True),
                               dict(B=1, T=128, H=2, K=128, V=128, h0=True, dht=True),
                               dict(B=1, T=256, H=2, K=64, V=64, h0=True, dht=True, cu=[0, 64, 256])],
                         ids=lambda c: "B{B}-T{T}-h0{h0}-dht{dht}".format(**c) + ("-varlen" if "cu" in c else ""))
def test_chunk_gla_bwd_with_pl(c, cuda_device):
    """chunk_gla_bwd_with_pl (tops/ops/gla/chunk.py:1000-1095) on the reference test's shapes
    (tests/ops/gla/test_pallas_chunk_bwd_with_pl.py:17-22) against the oracle backward; T and
    cu_seqlens off the chunk grid are rejected."""
    from tops.ops.gla import chunk_gla_bwd_with_pl
    from _inputs import gla_inputs
    B, T, H, K, V = (c[x] for x in "BTHKV")
    cu = c.get("cu")
    n = B if cu is None else len(cu) - 1
    d = gla_inputs(B, T, H, K, V, 42 + T + K, gate_div=4.0, h0=c["h0"], N=n, grads=True)
    t = {x: to_dev(d[x], torch.float32, cuda_device) for x in ("q", "k", "v", "g", "h0", "do", "dht")}
    dht = t["dht"] if c["dht"] else None
    got = chunk_gla_bwd_with_pl(t["q"], t["k"], t["v"], t["g"], None, None, K ** -0.5, t["h0"], None,
                                None, t["do"], dht, cu_seqlens=cu, chunk_size=64)
    ref = O.chunk_gla_bwd(d["q"], d["k"], d["v"], d["g"], K ** -0.5, d["h0"], d["do"],
                          d["dht"] if c["dht"] else None, cu_seqlens=cu)
    for name, a, b in zip(("dq", "dk", "dv", "dg", "dh0"), got, ref):
        if a is None or b is None:
            continue
        assert rel(host(a), b) < 1e-4, name
    with pytest.raises(AssertionError):
        chunk_gla_bwd_with_pl(t["q"][:, :100], t["k"][:, :100], t["v"][:, :100], t["g"][:, :100],
                              None, None, K ** -0.5, None, None, None, t["do"][:, :100], None)


def test_stage_inputs_converted_in_one_call_match_fp32(cuda_device):
    """chunk_gla_bwd_dqkg_ref converts five fp32 operands (g_cumsum, h, dh, dq, dk) inside one
    call's argument list.  Given them in bf16, each conversion is a temporary; the result must
    equal, bit for bit, the call given the same (bf16-rounded) values already in fp32 (each
    temporary stays alive until its kernel is queued)."""
    from tops.ops.gla import chunk_gla_bwd_dqkg_ref
    B, T, H, K, V, C = 2, 128, 2, 64, 64, 64
    NT = T // C
    rng = np.random.default_rng(7)
    q, k = (rng.standard_normal((B, T, H, K)).astype(np.float32) for _ in range(2))
    v, do = (rng.standard_normal((B, T, H, V)).astype(np.float32) for _ in range(2))
    gc = OC.chunk_local_cumsum(np.log(1 / (1 + np.exp(-rng.standard_normal((B, T, H, K))))) / 4, C)
    hs = rng.standard_normal((B, NT, H, K, V)) * 0.3
    dh = rng.standard_normal((B, NT, H, K, V)) * 0.3
    dq_in, dk_in = rng.standard_normal((2, B, T, H, K))
    bf = lambda x: to_dev(x, torch.bfloat16, cuda_device)
    fb = lambda x: to_dev(x, torch.bfloat16, cuda_device).to(torch.float32)
    f = lambda x: to_dev(x, torch.float32, cuda_device)
    for _ in range(3):       # repeated, so freed blocks of earlier calls are in the cache too
        a = chunk_gla_bwd_dqkg_ref(f(q), f(k), f(v), bf(hs), bf(gc), f(do), bf(dh), bf(dq_in),
                                   bf(dk_in), K ** -0.5, chunk_size=C)
        b = chunk_gla_bwd_dqkg_ref(f(q), f(k), f(v), fb(hs), fb(gc), f(do), fb(dh), fb(dq_in),
                                   fb(dk_in), K ** -0.5, chunk_size=C)
        torch.cuda.synchronize()
        for x, y in zip(a, b):
            assert x.dtype == y.dtype == torch.float32 and torch.equal(x, y)
