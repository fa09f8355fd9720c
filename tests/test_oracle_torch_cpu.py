"""The torch-CPU float32 restatement (oracle/torch_cpu.py, the CPU baseline bench.py times)
against the float64 NumPy oracle, which the other oracle tests pin: forward and every
gradient within float32 rounding (rel-L2 1e-5).  A planted mistake (the gate total Gamma
left out of the state decay) must fail."""
import numpy as np
import pytest
import torch

from oracle import gla as O
from oracle import torch_cpu as TC
from _inputs import gla_inputs
from _closed_forms import rel


@pytest.mark.parametrize("B,T,H,K,V,h0", [(2, 128, 3, 32, 64, True), (1, 256, 2, 64, 32, False)])
def test_torch_cpu_matches_oracle(B, T, H, K, V, h0):
    d = gla_inputs(B, T, H, K, V, 9, gate_div=4.0, h0=h0, grads=True)
    t = {x: (None if d[x] is None else torch.from_numpy(d[x])) for x in ("q", "k", "v", "g", "h0", "do", "dht")}
    scale = K ** -0.5
    out = TC.chunk_gla_fwd_bwd(t["q"], t["k"], t["v"], t["g"], t["h0"], t["do"], t["dht"], scale)
    ro, rht = O.chunk_gla(d["q"], d["k"], d["v"], d["g"], initial_state=d["h0"],
                          output_final_state=True, chunk_size=64)
    ref = O.chunk_gla_bwd(d["q"], d["k"], d["v"], d["g"], scale, d["h0"], d["do"], d["dht"])
    for name, a, b in zip(("o", "ht", "dq", "dk", "dv", "dg", "dh0"), out, (ro, rht) + tuple(ref)):
        assert rel(a.double().numpy(), b) < 1e-5, name


def test_torch_cpu_planted_decay_mistake_fails():
    d = gla_inputs(1, 128, 2, 32, 32, 10, gate_div=4.0, h0=True, grads=True)
    t = {x: torch.from_numpy(d[x]) for x in ("q", "k", "v", "g", "h0", "do", "dht")}
    orig = torch.exp

    def bad_exp(x):   # every exp(Gamma) of the state decay replaced by 1
        return torch.ones_like(x) if x.dim() == 4 else orig(x)
    torch.exp = bad_exp
    try:
        o, ht = TC.chunk_gla_fwd_bwd(t["q"], t["k"], t["v"], t["g"], t["h0"], t["do"], t["dht"],
                                     32 ** -0.5, backward=False)
    finally:
        torch.exp = orig
    ro, rht = O.chunk_gla(d["q"], d["k"], d["v"], d["g"], initial_state=d["h0"],
                          output_final_state=True, chunk_size=64)
    assert rel(ht.double().numpy(), rht) > 1e-2


def _t(d, *names):
    return [None if d.get(x) is None else torch.from_numpy(np.ascontiguousarray(d[x], np.float32))
            for x in names]


@pytest.mark.parametrize("case", [dict(B=2, T=128, H=2, K=32, V=64, h0=True, cu=None),
                                  dict(B=1, T=300, H=3, K=64, V=32, h0=True,
                                       cu=[0, 13, 140, 141, 300]),
                                  dict(B=1, T=200, H=2, K=32, V=32, h0=False, cu=[0, 77, 200])],
                         ids=["fixed", "varlen", "varlen-noh0"])
def test_torch_cpu_simple_gla_matches_oracle(case):
    """Simple GLA (config 4's gate strength: logsigmoid(N(0,1)), no /16) fwd + bwd, fixed and
    varlen with ragged and one-token sequences, against the float64 oracle (which, as the
    reference, takes no empty sequence)."""
    from oracle import simple_gla as S
    from _inputs import simple_gla_inputs
    B, T, H, K, V, cu = (case[x] for x in ("B", "T", "H", "K", "V", "cu"))
    n = B if cu is None else len(cu) - 1
    d = simple_gla_inputs(B, T, H, K, V, seed=T + K, h0=case["h0"], N=n, grads=True)
    q, k, v, g, h0, do, dht = _t(d, "q", "k", "v", "g", "h0", "do", "dht")
    scale = K ** -0.5
    out = TC.chunk_simple_gla_fwd_bwd(q, k, v, g, scale, h0, do, dht, cu_seqlens=cu)
    ro, rht = S.chunk_simple_gla(d["q"], d["k"], d["v"], g=d["g"], scale=scale,
                                 initial_state=d["h0"], output_final_state=True, cu_seqlens=cu)
    rq, rk, rv, rg, rh0 = S.chunk_simple_gla_bwd(d["q"], d["k"], d["v"], d["g"], None, d["h0"],
                                                 d["do"], d["dht"], scale, cu_seqlens=cu)
    refs = dict(o=ro, ht=rht, dq=rq, dk=rk, dv=rv, dg=rg)
    if case["h0"]:
        refs["dh0"] = rh0
    got = dict(zip(("o", "ht", "dq", "dk", "dv", "dg", "dh0"), out))
    for name, r in refs.items():
        assert rel(got[name].double().numpy(), r) < 1e-5, name


def test_torch_cpu_simple_gla_planted_mistake_fails():
    """The inter-chunk gate term of dg left out must fail the check above."""
    from oracle import simple_gla as S
    from _inputs import simple_gla_inputs
    d = simple_gla_inputs(1, 192, 2, 32, 32, seed=4, h0=True, grads=True)
    q, k, v, g, h0, do, dht = _t(d, "q", "k", "v", "g", "h0", "do", "dht")
    orig = torch.exp

    def no_state_decay(x):   # exp of the per-chunk totals (3-D [B,H,NT]) replaced by 1
        return torch.ones_like(x) if x.dim() == 3 else orig(x)
    torch.exp = no_state_decay
    try:
        o, ht = TC.chunk_simple_gla_fwd_bwd(q, k, v, g, 32 ** -0.5, h0, backward=False)
    finally:
        torch.exp = orig
    ro, rht = S.chunk_simple_gla(d["q"], d["k"], d["v"], g=d["g"], initial_state=d["h0"],
                                 output_final_state=True)
    assert rel(ht.double().numpy(), rht) > 1e-2


@pytest.mark.parametrize("case", [dict(B=2, T=128, H=2, K=32, V=64, h0=True),
                                  dict(B=1, T=150, H=3, K=64, V=32, h0=False)],
                         ids=["aligned-h0", "ragged"])
def test_torch_cpu_kda_matches_oracle(case):
    """KDA fwd + autograd bwd (o, ht, dq, dk, dv, dbeta, dg, dh0) against the float64 oracle
    (itself pinned to torch float64 autograd of the per-token recurrence)."""
    from oracle import kda as KO
    from _inputs import kda_inputs
    B, T, H, K, V = (case[x] for x in "BTHKV")
    d = kda_inputs(B, T, H, K, V, seed=T + V, h0=case["h0"], grads=True)
    q, k, v, g, beta, h0, do, dht = _t(d, "q", "k", "v", "g", "beta", "h0", "do", "dht")
    scale = K ** -0.5
    o, ht, dq, dk, dv, db, dg, dh0 = TC.chunk_kda_fwd_bwd(q, k, v, g, beta, scale, h0, do, dht)
    ro, rht = KO.chunk_kda(d["q"], d["k"], d["v"], d["g"], d["beta"], scale, d["h0"], True)
    rq, rk, rv, rb, rg, rh0 = KO.chunk_kda_bwd(d["q"], d["k"], d["v"], d["g"], d["beta"], scale,
                                               d["h0"], d["do"], d["dht"])
    got = dict(o=o, ht=ht, dq=dq, dk=dk, dv=dv, db=db, dg=dg)
    refs = dict(o=ro, ht=rht, dq=rq, dk=rk, dv=rv, db=rb, dg=rg)
    if case["h0"]:
        got["dh0"], refs["dh0"] = dh0, rh0
    for name, r in refs.items():
        assert rel(got[name].double().numpy(), r) < 1e-5, name


def test_torch_cpu_kda_planted_mistake_fails():
    """The WY inverse left out (T = I, so u = beta v and w = beta exp(G) k) must fail."""
    from oracle import kda as KO
    from _inputs import kda_inputs
    d = kda_inputs(1, 128, 2, 32, 32, seed=6, h0=True)
    q, k, v, g, beta, h0 = _t(d, "q", "k", "v", "g", "beta", "h0")
    orig = torch.linalg.solve_triangular
    torch.linalg.solve_triangular = lambda A, B, **kw: B.clone()
    try:
        o, ht = TC.chunk_kda_fwd_bwd(q, k, v, g, beta, 32 ** -0.5, h0, backward=False)
    finally:
        torch.linalg.solve_triangular = orig
    ro, rht = KO.chunk_kda(d["q"], d["k"], d["v"], d["g"], d["beta"], 32 ** -0.5, d["h0"], True)
    assert rel(o.double().numpy(), ro) > 1e-2
