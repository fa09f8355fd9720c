"""Long sequences on MI355X: chunk_gla and chunk_kda at T = 2^18 / 2^17 tokens (one sequence),
where the offsets into q / k / v and the per-chunk checkpoints run far past what the oracle
can check directly.  Checked through properties the recurrence fixes:

  * splitting the sequence at a chunk boundary and chaining the final state of the first
    part into the second as initial_state gives the same o, final state and gradients
    (dq, dk, dv, dg, dh0 through the chained autograd graph) as the whole sequence;
  * the first 2048 outputs depend only on the first 2048 tokens: they match the float64
    oracle run on that prefix.

The whole-sequence GLA run takes the sequence-parallel path (one sequence, few heads), so
this also checks the segment split at scale.  Tolerance: 2e-3 relative L2 (bf16 outputs).
"""
import numpy as np
import pytest
import torch

from oracle import gla as O
from oracle import kda as KO
from _gpu import host, rel

pytestmark = pytest.mark.gpu


def _rand(shape, gen, dev, dtype=torch.float32, scale=1.0):
    return (torch.randn(*shape, device=dev, generator=gen) * scale).to(dtype)


def _grads(fn, inputs, outs_grads):
    outs = fn(*inputs)
    return outs, torch.autograd.grad(outs, inputs, outs_grads)


def test_chunk_gla_long_sequence_split_and_prefix(cuda_device):
    from tops.ops.gla import chunk_gla
    dev = cuda_device
    gen = torch.Generator(device=dev).manual_seed(2024)
    B, T, H, K, V = 1, 1 << 18, 4, 128, 128
    T1 = 64 * 1537                              # split point: a chunk boundary near 0.37 T
    bf = torch.bfloat16
    q, k, v = (_rand((B, T, H, K), gen, dev, bf) for _ in range(3))
    # weak gates (a chunk keeps ~80% of the state): the state carried across the split
    # point, and across the whole run's segments, reaches thousands of tokens
    g = torch.nn.functional.logsigmoid(_rand((B, T, H, K), gen, dev)) / 256
    h0 = _rand((B, H, K, V), gen, dev, scale=0.1)
    do = _rand((B, T, H, V), gen, dev, bf)
    dht = _rand((B, H, K, V), gen, dev, scale=0.1)
    ins = [x.requires_grad_() for x in (q, k, v, g, h0)]
    print(f"chunk_gla B={B} T={T} H={H} split at {T1}", flush=True)

    (o, ht), gfull = _grads(lambda q_, k_, v_, g_, h_: chunk_gla(
        q_, k_, v_, g_, initial_state=h_, output_final_state=True), ins, (do, dht))

    def composed(q_, k_, v_, g_, h_):
        s1 = slice(None, T1)
        s2 = slice(T1, None)
        oa, ha = chunk_gla(q_[:, s1], k_[:, s1], v_[:, s1], g_[:, s1], initial_state=h_,
                           output_final_state=True)
        ob, hb = chunk_gla(q_[:, s2], k_[:, s2], v_[:, s2], g_[:, s2], initial_state=ha,
                           output_final_state=True)
        return torch.cat([oa, ob], 1), hb
    (o2, ht2), gsplit = _grads(composed, ins, (do, dht))
    torch.cuda.synchronize()
    from tops.utils import ChunkPlan
    sp = ChunkPlan(B, T, None, dev).segments(H, V)
    print("segments of the whole-sequence run:", None if sp is None else sp.Nv)
    errs = {"o": rel(host(o), host(o2)), "ht": rel(host(ht), host(ht2))}
    for name, a, b in zip(("dq", "dk", "dv", "dg", "dh0"), gfull, gsplit):
        assert float(a.float().norm()) > 0, name
        errs[name] = rel(host(a), host(b))
    print(" ".join(f"{n}={e:.2e}" for n, e in errs.items()))
    for n, e in errs.items():
        assert e < 2e-3, (n, e)

    P = 2048
    sq, sk, sv = (host(x[:, :P]) for x in (q, k, v))
    ro, _ = O.chunk_gla(sq, sk, sv, host(g[:, :P]), initial_state=host(h0),
                        output_final_state=False, chunk_size=64)
    e = rel(host(o[:, :P]), ro)
    print(f"prefix o vs oracle: {e:.2e}")
    assert e < 2e-3


def test_chunk_kda_long_sequence_split_and_prefix(cuda_device):
    from tops.ops.kda import chunk_kda
    dev = cuda_device
    gen = torch.Generator(device=dev).manual_seed(2025)
    B, T, H, K, V = 1, 1 << 17, 2, 128, 128
    T1 = 64 * 701
    bf = torch.bfloat16

    def l2n(x):
        return x / torch.sqrt((x * x).sum(-1, keepdim=True) + 1e-6)
    q, k = (l2n(_rand((B, T, H, K), gen, dev)).to(bf) for _ in range(2))
    v = _rand((B, T, H, V), gen, dev, bf)
    g = torch.nn.functional.logsigmoid(_rand((B, T, H, K), gen, dev)) / 256
    beta = torch.sigmoid(_rand((B, T, H), gen, dev))
    h0 = _rand((B, H, K, V), gen, dev, scale=0.1)
    do = _rand((B, T, H, V), gen, dev, bf)
    dht = _rand((B, H, K, V), gen, dev, scale=0.1)
    ins = [x.requires_grad_() for x in (q, k, v, g, beta, h0)]
    print(f"chunk_kda B={B} T={T} H={H} split at {T1}", flush=True)

    (o, ht), gfull = _grads(lambda q_, k_, v_, g_, b_, h_: chunk_kda(
        q_, k_, v_, g_, b_, initial_state=h_, output_final_state=True), ins, (do, dht))

    def composed(q_, k_, v_, g_, b_, h_):
        s1, s2 = slice(None, T1), slice(T1, None)
        oa, ha = chunk_kda(q_[:, s1], k_[:, s1], v_[:, s1], g_[:, s1], b_[:, s1],
                           initial_state=h_, output_final_state=True)
        ob, hb = chunk_kda(q_[:, s2], k_[:, s2], v_[:, s2], g_[:, s2], b_[:, s2],
                           initial_state=ha, output_final_state=True)
        return torch.cat([oa, ob], 1), hb
    (o2, ht2), gsplit = _grads(composed, ins, (do, dht))
    torch.cuda.synchronize()
    errs = {"o": rel(host(o), host(o2)), "ht": rel(host(ht), host(ht2))}
    for name, a, b in zip(("dq", "dk", "dv", "dg", "dbeta", "dh0"), gfull, gsplit):
        assert float(a.float().norm()) > 0, name
        errs[name] = rel(host(a), host(b))
    print(" ".join(f"{n}={e:.2e}" for n, e in errs.items()))
    for n, e in errs.items():
        assert e < 2e-3, (n, e)

    P = 1024
    ro, _ = KO.chunk_kda(host(q[:, :P]), host(k[:, :P]), host(v[:, :P]), host(g[:, :P]),
                         host(beta[:, :P]), K ** -0.5, host(h0), False)
    e = rel(host(o[:, :P]), ro)
    print(f"prefix o vs oracle: {e:.2e}")
    assert e < 2e-3
