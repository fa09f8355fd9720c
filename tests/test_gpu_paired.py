"""The interleaved-checkpoint training path (tops_chunk_*_paired) on MI355X, the layout of
tops.utils.set_checkpoint_layout("paired").

chunk_fwd(keep_states=PAIRED) keeps the state before every even global chunk only; the
reverse sweep writes dh after every odd chunk into the same buffer, and the PAIR dq / dk / dg
kernel rebuilds each chunk's other state from its pair partner (one sweep step on MFMA).
Checked against the unpaired path on the same bf16 inputs:
  * o, ht, dv, dh0 and the forward's checkpoint slots are bitwise equal (the sweeps are the
    same kernels, only the checkpoint stores are skipped);
  * dq, dk, dg differ only by the rounding of the rebuilt states: dg (fp32) within 1e-5
    relative L2, dq / dk (bf16) within 2e-3;
and the gradients against the float64 oracle (2e-3) for the chunk_gla cases.  The shapes put
pair partners in different sequences (h0 / dht stand in), leave the last pair without a
second chunk, and cut long sequences into sequence-parallel segments.
"""
import numpy as np
import pytest
import torch

from oracle import gla as O
from _inputs import gla_inputs
from _gpu import to_dev, seen, host, rel

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _paired_layout():
    from tops import utils as U
    prev = U.checkpoint_layout()
    U.set_checkpoint_layout("paired")
    yield
    U.set_checkpoint_layout(prev)

CASES = [
    dict(B=2, T=130, H=3, K=64, V=64, seed=31),                       # 3 chunks per sequence
    dict(B=1, T=160, H=2, K=32, V=64, seed=32, cu=[0, 10, 64, 65, 160]),   # 5 chunks, odd
    dict(B=1, T=300, H=2, K=128, V=128, seed=33, cu=[0, 100, 300]),
    dict(B=2, T=64, H=2, K=32, V=32, seed=34),                        # one chunk per sequence
    dict(B=1, T=1000, H=2, K=128, V=128, seed=35, split=3),           # segments of 3 chunks
    dict(B=1, T=700, H=2, K=128, V=64, seed=36, cu=[0, 90, 91, 400, 700], split=2),
]
GATES = ["k", "s", "gamma", "gamma_k"]


def _id(c):
    return "-".join(f"{k}{v}" for k, v in c.items() if k != "seed")


def _gate(mode, d, H, K, device):
    rng = np.random.Generator(np.random.PCG64(7))
    if mode == "k":
        return to_dev(d["g"], torch.float32, device)
    if mode == "s":
        return to_dev(d["g"][..., 0], torch.float32, device).contiguous()
    if mode == "gamma":
        return torch.tensor(-np.abs(rng.standard_normal(H)) / 8, dtype=torch.float32, device=device)
    return torch.tensor(-np.abs(rng.standard_normal((H, K))) / 8, dtype=torch.float32,
                        device=device)


@pytest.mark.parametrize("gate", GATES)
@pytest.mark.parametrize("cfg", CASES, ids=[_id(c) for c in CASES])
def test_paired_matches_unpaired(cfg, gate, cuda_device):
    from tops import utils as U
    from tops.ops import _chunk_core as CC
    B, T, H, K, V = (cfg[x] for x in "BTHKV")
    cu = cfg.get("cu")
    n = len(cu) - 1 if cu else B
    d = gla_inputs(B, T, H, K, V, cfg["seed"], gate_div=4.0, h0=True, N=n, grads=True)
    bf = torch.bfloat16
    q, k, v, do = (to_dev(d[x], bf, cuda_device) for x in ("q", "k", "v", "do"))
    h0, dht = (to_dev(d[x], torch.float32, cuda_device) for x in ("h0", "dht"))
    gt = _gate(gate, d, H, K, cuda_device)
    mode = {"k": CC.GATE_K, "s": CC.GATE_S, "gamma": CC.GATE_GAMMA, "gamma_k": CC.GATE_GAMMA_K}[gate]
    scale = K ** -0.5
    U.set_sequence_split(cfg.get("split", 0))
    try:
        plan = U.ChunkPlan(B, T, cu, cuda_device)
        assert CC.paired_states(q, K, V)
        o1, ht1, hs1 = CC.chunk_fwd(q, k, v, (mode, gt), h0, scale, True, plan, keep_states=True)
        o2, ht2, hs2 = CC.chunk_fwd(q, k, v, (mode, gt), h0, scale, True, plan,
                                    keep_states=CC.PAIRED)
        hs1_copy = hs1.clone()
        r1 = CC.chunk_bwd(q, k, v, (mode, gt), do, dht, hs1, scale, plan, True)
        r2 = CC.chunk_bwd(q, k, v, (mode, gt), do, dht, hs2, scale, plan, True, h0=h0, paired=True)
        assert (plan.segments(H, V) is not None) == bool(cfg.get("split"))
    finally:
        U.set_sequence_split(None)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(ht1, ht2)
    ev = torch.arange(plan.total, device=cuda_device) % 2 == 0
    assert torch.equal(hs1_copy[ev], hs2[ev]), "even slots must be the forward's states"
    dq1, dk1, dv1, dg1, dh01 = r1
    dq2, dk2, dv2, dg2, dh02 = r2
    assert torch.equal(dv1, dv2) and torch.equal(dh01, dh02)
    for a, b in ((dq1, dq2), (dk1, dk2)):
        assert rel(host(b), host(a)) < 2e-3
    if dg1 is not None:
        # per-channel gates: the same arithmetic but for the rebuilt states (1e-5); one gate
        # per token: the unpaired kernel factors the gate out of q / k (exact planes, factors
        # in the dA tiles) while the paired one gates the planes, two fp32 formulations (1e-4)
        assert rel(host(dg2), host(dg1)) < (1e-5 if gate in ("k", "gamma_k") else 1e-4)


@pytest.mark.parametrize("cfg", CASES, ids=[_id(c) for c in CASES])
def test_paired_chunk_gla_vs_oracle(cfg, cuda_device):
    """chunk_gla's autograd (which keeps paired checkpoints for bf16) against the oracle."""
    from tops import utils as U
    from tops.ops.gla import chunk_gla
    B, T, H, K, V = (cfg[x] for x in "BTHKV")
    cu = cfg.get("cu")
    n = len(cu) - 1 if cu else B
    d = gla_inputs(B, T, H, K, V, cfg["seed"], gate_div=4.0, h0=True, N=n, grads=True)
    bf = torch.bfloat16
    q, k, v = (to_dev(d[x], bf, cuda_device).requires_grad_() for x in "qkv")
    g = to_dev(d["g"], torch.float32, cuda_device).requires_grad_()
    h0 = to_dev(d["h0"], torch.float32, cuda_device).requires_grad_()
    U.set_sequence_split(cfg.get("split", 0))
    try:
        o, ht = chunk_gla(q, k, v, g, initial_state=h0, output_final_state=True, cu_seqlens=cu)
        loss = (o.float() * to_dev(d["do"], bf, cuda_device).float()).sum() + \
            (ht * to_dev(d["dht"], torch.float32, cuda_device)).sum()
        loss.backward()
    finally:
        U.set_sequence_split(None)
    torch.cuda.synchronize()
    ref = O.chunk_gla_bwd(seen(d["q"], bf), seen(d["k"], bf), seen(d["v"], bf), d["g"], K ** -0.5,
                          d["h0"], seen(d["do"], bf), d["dht"], chunk_size=64, cu_seqlens=cu)
    for name, got, want in zip(("dq", "dk", "dv", "dg", "dh0"),
                               (q.grad, k.grad, v.grad, g.grad, h0.grad), ref):
        e = rel(host(got), want)
        assert e < 2e-3, f"{name}: rel {e:.2e}"
