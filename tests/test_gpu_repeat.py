"""Bitwise repeatability on MI355X: the kernels use no atomics and reduce in a fixed order,
so two runs of the same call give identical bits in every output and gradient (the
boundary's determinism requirement: the reference's JAX ops are pure functions).  chunk_gla
and chunk_kda forward + backward, bf16 and fp32, with varlen and the sequence-parallel
segment path."""
import numpy as np
import pytest
import torch

from _inputs import gla_inputs, kda_inputs
from _gpu import to_dev

pytestmark = pytest.mark.gpu


def _gla_once(d, dtype, dev, cu):
    from tops.ops.gla import chunk_gla
    q, k, v = (to_dev(d[x], dtype, dev).requires_grad_() for x in "qkv")
    g = to_dev(d["g"], torch.float32, dev).requires_grad_()
    h0 = to_dev(d["h0"], torch.float32, dev).requires_grad_()
    o, ht = chunk_gla(q, k, v, g, initial_state=h0, output_final_state=True, cu_seqlens=cu)
    torch.autograd.backward((o, ht), (to_dev(d["do"], dtype, dev), to_dev(d["dht"], torch.float32, dev)))
    torch.cuda.synchronize()
    return [x.detach().clone() for x in (o, ht, q.grad, k.grad, v.grad, g.grad, h0.grad)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("case", ["fixed", "varlen", "segments"])
def test_chunk_gla_bitwise_repeat(case, dtype, cuda_device):
    B, T, H, K, V, cu, n = 2, 300, 4, 128, 128, None, 2
    if case == "varlen":
        B, T, cu, n = 1, 700, [0, 13, 140, 141, 700], 4
    elif case == "segments":
        B, T, H, n = 1, 4096, 2, 1          # few heads, one long sequence: split into segments
    d = gla_inputs(B, T, H, K, V, 500, gate_div=8.0, h0=True, N=n, grads=True)
    print(f"repeat chunk_gla {case} {dtype}", flush=True)
    a = _gla_once(d, dtype, cuda_device, cu)
    b = _gla_once(d, dtype, cuda_device, cu)
    for name, x, y in zip(("o", "ht", "dq", "dk", "dv", "dg", "dh0"), a, b):
        assert torch.equal(x, y), name


def _kda_once(d, dtype, dev, cu):
    from tops.ops.kda import chunk_kda
    q, k, v = (to_dev(d[x], dtype, dev).requires_grad_() for x in "qkv")
    g = to_dev(d["g"], torch.float32, dev).requires_grad_()
    beta = to_dev(d["beta"], torch.float32, dev).requires_grad_()
    h0 = to_dev(d["h0"], torch.float32, dev).requires_grad_()
    o, ht = chunk_kda(q, k, v, g, beta, initial_state=h0, output_final_state=True, cu_seqlens=cu)
    torch.autograd.backward((o, ht), (to_dev(d["do"], dtype, dev), to_dev(d["dht"], torch.float32, dev)))
    torch.cuda.synchronize()
    return [x.detach().clone() for x in (o, ht, q.grad, k.grad, v.grad, g.grad, beta.grad, h0.grad)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("varlen", [False, True], ids=["fixed", "varlen"])
def test_chunk_kda_bitwise_repeat(varlen, dtype, cuda_device):
    B, T, H, K, V, cu, n = 2, 300, 4, 128, 128, None, 2
    if varlen:
        B, T, cu, n = 1, 700, [0, 13, 140, 141, 700], 4
    d = kda_inputs(B, T, H, K, V, 501, h0=True, grads=True, N=n)
    print(f"repeat chunk_kda varlen={varlen} {dtype}", flush=True)
    a = _kda_once(d, dtype, cuda_device, cu)
    b = _kda_once(d, dtype, cuda_device, cu)
    for name, x, y in zip(("o", "ht", "dq", "dk", "dv", "dg", "dbeta", "dh0"), a, b):
        assert torch.equal(x, y), name
