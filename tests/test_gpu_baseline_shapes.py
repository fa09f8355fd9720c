"""Parity at the BASELINE shapes themselves (configs 2-5, full size), on MI355X.

Each case runs the op on the GPU at its config's exact shape and dtype and compares every
output and gradient with the torch-CPU float32 restatement of the reference
(oracle/torch_cpu.py: chunked GLA, simple GLA, KDA; pinned to the float64 oracle at 1e-5 by
tests/test_oracle_torch_cpu.py) evaluated on the same bf16-rounded inputs:
  config 2  fused_recurrent_gla fwd, B16 T2048 H8 K=V=128, gk, h0: o, ht
  config 3  chunk_gla fwd + bwd, B8 T4096 H16 K=V=128, h0, dht: o, ht, dq, dk, dv, dg, dh0
  config 4  chunk_simple_gla fwd + bwd, varlen T16384 (8 seeded sequences) H32 K=V=128,
            per-token g = logsigmoid(N(0,1)): o, dq, dk, dv, dg
  config 5  chunk_kda fwd + bwd, B4 T8192 H32 K=V=128, L2-normalised q, k: o, ht, dq, dk, dv,
            dbeta, dg
Inputs are drawn on the host with torch's CPU generator (seeds 1002-1005).  Tolerance:
north_star's bf16 bound, relative L2 error <= 2e-3 per tensor.
"""
import numpy as np
import pytest
import torch

from oracle import torch_cpu as TC

pytestmark = pytest.mark.gpu

TOL = 2e-3
BF = torch.bfloat16


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float(torch.linalg.norm(a - b) / torch.linalg.norm(b))


def _check(got, ref, tag):
    errs = {n: _rel(x, ref[n]) for n, x in got.items()}
    print(tag, " ".join(f"{n}={e:.3e}" for n, e in errs.items()), flush=True)
    bad = {n: e for n, e in errs.items() if not e <= TOL}
    assert not bad, f"{tag}: rel err over {TOL}: {bad}"


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _n(gen, *shape, std=1.0):
    return torch.randn(*shape, generator=gen) * std


def test_config2_full_shape(cuda_device):
    from tops.ops.gla import fused_recurrent_gla
    B, T, H, D = 16, 2048, 8, 128
    print("config 2 full shape: fused_recurrent_gla fwd B16 T2048 H8 K=V=128 bf16", flush=True)
    gen = _gen(1002)
    q, k, v = (_n(gen, B, T, H, D).to(BF) for _ in range(3))
    gk = torch.nn.functional.logsigmoid(_n(gen, B, T, H, D)) / 16
    h0 = _n(gen, B, H, D, D, std=0.1)
    dev = cuda_device
    with torch.no_grad():
        o, ht = fused_recurrent_gla(q.to(dev), k.to(dev), v.to(dev), gk.to(dev),
                                    initial_state=h0.to(dev), output_final_state=True)
    torch.cuda.synchronize()
    ro, rht = TC.chunk_gla_fwd_bwd(q.float(), k.float(), v.float(), gk, h0, None, None,
                                   D ** -0.5, backward=False)
    assert o.dtype == BF and ht.dtype == torch.float32
    _check(dict(o=o, ht=ht), dict(o=ro, ht=rht), "config 2")


def test_config3_full_shape(cuda_device):
    from tops.ops.gla import chunk_gla
    B, T, H, D = 8, 4096, 16, 128
    print("config 3 full shape: chunk_gla fwd+bwd B8 T4096 H16 K=V=128 bf16", flush=True)
    gen = _gen(1003)
    q, k, v = (_n(gen, B, T, H, D).to(BF) for _ in range(3))
    g = torch.nn.functional.logsigmoid(_n(gen, B, T, H, D)) / 16
    h0 = _n(gen, B, H, D, D, std=0.1)
    do = _n(gen, B, T, H, D).to(BF)
    dht = _n(gen, B, H, D, D, std=0.1)
    dev = cuda_device
    ins = [x.to(dev).requires_grad_() for x in (q, k, v, g, h0)]
    o, ht = chunk_gla(*ins[:4], initial_state=ins[4], output_final_state=True)
    grads = torch.autograd.grad((o, ht), ins, (do.to(dev), dht.to(dev)))
    torch.cuda.synchronize()
    ref = TC.chunk_gla_fwd_bwd(q.float(), k.float(), v.float(), g, h0, do.float(), dht, D ** -0.5)
    names = ("o", "ht", "dq", "dk", "dv", "dg", "dh0")
    got = dict(zip(names, (o, ht) + tuple(grads)))
    assert [x.dtype for x in grads] == [BF, BF, BF, torch.float32, torch.float32]
    _check(got, dict(zip(names, ref)), "config 3")


def test_config4_full_shape(cuda_device):
    from tops.ops.simple_gla import chunk_simple_gla
    T, H, D = 16384, 32, 128
    rng = np.random.Generator(np.random.PCG64(1004))
    cu = [0] + sorted(int(c) for c in rng.choice(np.arange(1, T), 7, replace=False)) + [T]
    print(f"config 4 full shape: chunk_simple_gla fwd+bwd varlen T16384 H32 K=V=128 bf16 cu={cu}",
          flush=True)
    gen = _gen(1004)
    q, k, v = (_n(gen, 1, T, H, D).to(BF) for _ in range(3))
    g = torch.nn.functional.logsigmoid(_n(gen, 1, T, H))
    do = _n(gen, 1, T, H, D).to(BF)
    dev = cuda_device
    ins = [x.to(dev).requires_grad_() for x in (q, k, v, g)]
    o, _ = chunk_simple_gla(ins[0], ins[1], ins[2], None, g=ins[3], cu_seqlens=cu)
    grads = torch.autograd.grad(o, ins, do.to(dev))
    torch.cuda.synchronize()
    r = TC.chunk_simple_gla_fwd_bwd(q.float(), k.float(), v.float(), g, D ** -0.5, do=do.float(),
                                    cu_seqlens=cu)
    ref = dict(o=r[0], dq=r[2], dk=r[3], dv=r[4], dg=r[5])
    got = dict(zip(("o", "dq", "dk", "dv", "dg"), (o,) + tuple(grads)))
    _check(got, ref, "config 4")


def test_config5_full_shape(cuda_device):
    from tops.ops.kda import chunk_kda
    B, T, H, D = 4, 8192, 32, 128
    print("config 5 full shape: chunk_kda fwd+bwd B4 T8192 H32 K=V=128 bf16", flush=True)
    gen = _gen(1005)

    def l2n(x):
        return x / torch.sqrt((x * x).sum(-1, keepdim=True) + 1e-6)
    q, k = (l2n(_n(gen, B, T, H, D)).to(BF) for _ in range(2))
    v = _n(gen, B, T, H, D).to(BF)
    beta = torch.sigmoid(_n(gen, B, T, H))
    g = torch.nn.functional.logsigmoid(_n(gen, B, T, H, D)) / 16
    do = _n(gen, B, T, H, D).to(BF)
    dev = cuda_device
    ins = [x.to(dev).requires_grad_() for x in (q, k, v, g, beta)]
    o, ht = chunk_kda(*ins, output_final_state=True)
    grads = torch.autograd.grad(o, ins, do.to(dev))
    torch.cuda.synchronize()
    got = dict(zip(("o", "ht", "dq", "dk", "dv", "dg", "dbeta"), (o, ht) + tuple(grads)))
    del ins, o, ht, grads
    r = TC.chunk_kda_fwd_bwd(q.float(), k.float(), v.float(), g, beta, D ** -0.5, do=do.float())
    ref = dict(zip(("o", "ht", "dq", "dk", "dv", "dbeta", "dg"), r[:7]))
    _check(got, ref, "config 5")
