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
