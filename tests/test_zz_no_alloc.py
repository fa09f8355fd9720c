"""tops_kda_chunk_fwd_noalloc (the allocation-free KDA forward, workspace in the library's
static scratch) through the C ABI against tops_kda_chunk_fwd with a caller workspace: o and
the final state bit-identical, on two calls in a row, the second with a smaller input (the
scratch keeps the first call's contents).  A call beyond the scratch is rejected on the host
before any launch."""
import ctypes

import numpy as np
import pytest
import torch

from _inputs import kda_inputs
from _gpu import to_dev

pytestmark = pytest.mark.gpu


def _call(name, q, k, v, g, beta, h0, o, ht, plan, B, T, H, K, V, scale, u=None, w=None):
    from tops import _native as N
    args = [N.ptr(q), N.ptr(k), N.ptr(v), N.ptr(g), N.ptr(beta), N.ptr(h0), N.ptr(o), N.ptr(ht)]
    if name == "tops_kda_chunk_fwd":
        args += [N.ptr(u), N.ptr(w), None, None, None]
    args += [N.ptr(plan.cu_dev), N.ptr(plan.offsets_dev), N.ptr(plan.chunk_map_dev), plan.total,
             B, T, H, K, V, plan.N, N.dtype_code(q.dtype), float(scale), N.stream()]
    N.call(name, *args)


def _case(dev, B, T, H, K, V, dtype, cu, seed):
    from tops.utils import ChunkPlan
    n = len(cu) - 1 if cu else B
    d = kda_inputs(B, T, H, K, V, seed, h0=True, N=n)
    q, k, v = (to_dev(d[x], dtype, dev) for x in "qkv")
    g = to_dev(d["g"], torch.float32, dev)
    beta = to_dev(d["beta"], torch.float32, dev)
    h0 = to_dev(d["h0"], torch.float32, dev)
    plan = ChunkPlan.get(B, T, cu, dev)
    scale = K ** -0.5
    outs = []
    for name in ("tops_kda_chunk_fwd", "tops_kda_chunk_fwd_noalloc"):
        o = torch.empty(B, T, H, V, device=dev, dtype=dtype)
        ht = torch.empty(n, H, K, V, device=dev, dtype=torch.float32)
        u = torch.empty(B, T, H, V, device=dev, dtype=torch.float32)
        w = torch.empty(B, T, H, K, device=dev, dtype=torch.float32)
        print(f"no-alloc case {name} B{B} T{T} H{H} K{K} V{V} {dtype} cu={cu}", flush=True)
        _call(name, q, k, v, g, beta, h0, o, ht, plan, B, T, H, K, V, scale, u, w)
        torch.cuda.synchronize()
        outs.append((o, ht))
    return outs


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
def test_kda_fwd_noalloc_matches_workspace_entry(dtype, cuda_device):
    # first call: larger; second call: smaller (and varlen), on the same scratch
    for (B, T, H, K, V, cu, seed) in ((2, 700, 8, 128, 128, None, 71),
                                      (1, 300, 2, 64, 32, [0, 13, 140, 141, 300], 72)):
        (o1, h1), (o2, h2) = _case(cuda_device, B, T, H, K, V, dtype, cu, seed)
        assert torch.equal(o1, o2), "o"
        assert torch.equal(h1, h2), "ht"
        assert torch.isfinite(o2.float()).all()


def test_kda_fwd_noalloc_rejects_oversize(cuda_device):
    from tops import _native as N
    L = N.lib()
    cap = L.tops_kda_chunk_fwd_noalloc_max_bytes()
    assert cap == 64 << 20
    T = cap // (8 * (128 + 128) * 4) + 64          # one size past the scratch
    fn = N._fn("tops_kda_chunk_fwd_noalloc")
    rc = fn(*([None] * 11), 0, 1, T, 8, 128, 128, 1, 1, ctypes.c_float(1.0), None)
    assert rc == -2 and b"static scratch" in L.tops_last_error()
