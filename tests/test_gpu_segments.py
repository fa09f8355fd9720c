"""Sequence-parallel chunk sweeps on MI355X (tops_chunk_state_pass / _combine + the segment
sweep): chunk_gla and chunk_simple_gla forward + backward with sequences cut into segments,
against the float64 oracle (tops/cpu/ops/gla/chunk.py, tops/cpu/ops/simple_gla/chunk.py
restated) and against the same call swept whole.  Cases cover ragged sequences, a
one-token sequence, h0 / dht, all three gate modes and the automatic split of one long
sequence.  Tolerance: fp32 1e-4, bf16 2e-3 (relative L2) against the oracle; 1e-4 between
the split and unsplit runs (fp32 state rounding only), except dq / dk / dg of bf16 calls,
1e-3: those read the fp16 state checkpoints, and a state that differs in its last fp32 bit
between the two runs can round to the neighbouring fp16 value (2^-12 of that entry), which
flips some bf16 outputs by one ulp.
"""
import numpy as np
import pytest
import torch

from oracle import gla as O
from oracle import simple_gla as S
from _inputs import gla_inputs, simple_gla_inputs
from _gpu import to_dev, seen, host, rel, tol

pytestmark = pytest.mark.gpu


def _split_bound(name, dtype):
    return 1e-3 if dtype == torch.bfloat16 and name in ("dq", "dk", "dg") else 1e-4


@pytest.fixture
def split_mode():
    from tops.utils import set_sequence_split
    yield set_sequence_split
    set_sequence_split(None)


def _gla(d, cu, dtype, device, scale=None):
    from tops.ops.gla import chunk_gla
    q, k, v = (to_dev(d[x], dtype, device).requires_grad_() for x in "qkv")
    g = to_dev(d["g"], torch.float32, device).requires_grad_()
    h0 = to_dev(d["h0"], torch.float32, device).requires_grad_()
    o, ht = chunk_gla(q, k, v, g, scale=scale, initial_state=h0, output_final_state=True,
                      cu_seqlens=cu)
    torch.autograd.backward((o, ht), (to_dev(d["do"], dtype, device),
                                      to_dev(d["dht"], torch.float32, device)))
    torch.cuda.synchronize()
    return dict(o=host(o), ht=host(ht), dq=host(q.grad), dk=host(k.grad), dv=host(v.grad),
                dg=host(g.grad), dh0=host(h0.grad))


def _gla_oracle(d, cu, dtype, scale):
    sq, sk, sv, sdo = (seen(d[x], dtype) for x in ("q", "k", "v", "do"))
    K = sq.shape[-1]
    sc = K ** -0.5 if scale is None else scale
    ro, rht = O.chunk_gla(sq, sk, sv, d["g"], scale=sc, initial_state=d["h0"],
                          output_final_state=True, cu_seqlens=cu)
    rq, rk, rv, rg, rh0 = O.chunk_gla_bwd(sq, sk, sv, d["g"], sc, d["h0"], sdo, d["dht"],
                                         chunk_size=64, cu_seqlens=cu)
    return dict(o=ro, ht=rht, dq=rq, dk=rk, dv=rv, dg=rg, dh0=rh0)


GLA_CASES = [
    dict(B=2, T=700, H=2, K=64, V=64, split=3),
    dict(B=1, T=900, H=2, K=128, V=128, split=2, cu=[0, 10, 300, 301, 900]),
    dict(B=1, T=1000, H=3, K=32, V=64, split=1, cu=[0, 640, 1000]),
    dict(B=1, T=1500, H=1, K=128, V=128, split=4, scale=0.2),
]


def _id(c):
    return "-".join(f"{k}{v}" for k, v in c.items() if k != "cu") + ("-varlen" if "cu" in c else "")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("cfg", GLA_CASES, ids=[_id(c) for c in GLA_CASES])
def test_chunk_gla_segments(cfg, dtype, cuda_device, split_mode):
    from tops.utils import ChunkPlan
    B, T, H, K, V = (cfg[x] for x in "BTHKV")
    cu = cfg.get("cu")
    n = len(cu) - 1 if cu else B
    # weak gates (a chunk keeps about half of the state) so the state handed from segment to
    # segment reaches far into the next one
    d = gla_inputs(B, T, H, K, V, seed=T + H, gate_div=64.0, h0=True, N=n, grads=True)
    split_mode(cfg["split"])
    sp = ChunkPlan(B, T, cu, cuda_device).segments(H, V)
    assert sp is not None and sp.fwd.n > 0 and sp.rev.n > 0
    got = _gla(d, cu, dtype, cuda_device, cfg.get("scale"))
    split_mode(0)
    whole = _gla(d, cu, dtype, cuda_device, cfg.get("scale"))
    ref = _gla_oracle(d, cu, dtype, cfg.get("scale"))
    errs = {x: rel(got[x], ref[x]) for x in got}
    diffs = {x: rel(got[x], whole[x]) for x in got}
    print(f"segments={sp.Nv}", " ".join(f"{x}={errs[x]:.2e}/{diffs[x]:.1e}" for x in got))
    for x in got:
        assert errs[x] < tol(dtype), (x, errs[x])
        assert diffs[x] < _split_bound(x, dtype), (x, diffs[x])


SIMPLE_CASES = [
    dict(B=1, T=1000, H=2, K=64, V=128, gate="g", split=2, cu=[0, 1, 500, 1000]),
    dict(B=2, T=600, H=2, K=128, V=64, gate="gamma", split=3),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("cfg", SIMPLE_CASES, ids=[_id(c) for c in SIMPLE_CASES])
def test_chunk_simple_gla_segments(cfg, dtype, cuda_device, split_mode):
    from tops.ops.simple_gla import chunk_simple_gla
    B, T, H, K, V = (cfg[x] for x in "BTHKV")
    cu = cfg.get("cu")
    n = len(cu) - 1 if cu else B
    d = simple_gla_inputs(B, T, H, K, V, seed=T + 3 * H, gate_div=64.0, h0=True, N=n, grads=True)
    d["g_gamma"] = d["g_gamma"] / 8

    def run():
        q, k, v = (to_dev(d[x], dtype, cuda_device).requires_grad_() for x in "qkv")
        g = to_dev(d["g"], torch.float32, cuda_device).requires_grad_() if cfg["gate"] == "g" else None
        gg = to_dev(d["g_gamma"], torch.float32, cuda_device) if cfg["gate"] == "gamma" else None
        h0 = to_dev(d["h0"], torch.float32, cuda_device).requires_grad_()
        o, ht = chunk_simple_gla(q, k, v, gg, initial_state=h0, output_final_state=True, g=g,
                                 cu_seqlens=cu)
        torch.autograd.backward((o, ht), (to_dev(d["do"], dtype, cuda_device),
                                          to_dev(d["dht"], torch.float32, cuda_device)))
        torch.cuda.synchronize()
        out = dict(o=host(o), ht=host(ht), dq=host(q.grad), dk=host(k.grad), dv=host(v.grad),
                   dh0=host(h0.grad))
        if g is not None:
            out["dg"] = host(g.grad)
        return out

    split_mode(cfg["split"])
    got = run()
    split_mode(0)
    whole = run()
    gs = d["g"] if cfg["gate"] == "g" else None
    gam = d["g_gamma"] if cfg["gate"] == "gamma" else None
    sq, sk, sv, sdo = (seen(d[x], dtype) for x in ("q", "k", "v", "do"))
    ro, rht = S.chunk_simple_gla(sq, sk, sv, g=gs, g_gamma=gam, initial_state=d["h0"],
                                 output_final_state=True, cu_seqlens=cu)
    rq, rk, rv, rg, rh0 = S.chunk_simple_gla_bwd(sq, sk, sv, gs, gam, d["h0"], sdo, d["dht"],
                                                 K ** -0.5, cu_seqlens=cu)
    ref = dict(o=ro, ht=rht, dq=rq, dk=rk, dv=rv, dg=rg, dh0=rh0)
    for x in got:
        e, df = rel(got[x], ref[x]), rel(got[x], whole[x])
        print(f"{x}={e:.2e}/{df:.1e}", end=" ")
        assert e < tol(dtype), (x, e)
        assert df < _split_bound(x, dtype), (x, df)


def test_automatic_split_of_one_long_sequence(cuda_device, split_mode):
    """B=1, T=4096 on 2 heads: 128 workgroups would sweep 64 chunks each on a 256-CU chip;
    the automatic plan cuts the sequence and the result still matches the oracle."""
    from tops.utils import ChunkPlan
    B, T, H, K, V = 1, 4096, 2, 128, 128
    split_mode(None)
    sp = ChunkPlan(B, T, None, cuda_device).segments(H, V)
    assert sp is not None and sp.Nv > 1, "expected an automatic split"
    d = gla_inputs(B, T, H, K, V, seed=77, gate_div=64.0, h0=True, grads=True)
    got = _gla(d, None, torch.bfloat16, cuda_device)
    ref = _gla_oracle(d, None, torch.bfloat16, None)
    for x in got:
        e = rel(got[x], ref[x])
        print(f"{x}={e:.2e}", end=" ")
        assert e < 2e-3, (x, e)


def test_more_segments_than_the_dispatch_ranking(cuda_device, split_mode):
    """301 one-chunk segments of one sequence: the segment sweep runs with more sequences
    than its in-kernel longest-first ranking covers (256) and the combine scans 300 states."""
    B, T, H, K, V = 1, 64 * 300 + 17, 1, 32, 32
    split_mode(1)
    d = gla_inputs(B, T, H, K, V, seed=301, gate_div=64.0, h0=True, grads=True)
    got = _gla(d, None, torch.float32, cuda_device)
    ref = _gla_oracle(d, None, torch.float32, None)
    for x in got:
        e = rel(got[x], ref[x])
        print(f"{x}={e:.2e}", end=" ")
        assert e < 1e-4, (x, e)
