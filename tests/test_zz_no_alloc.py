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


def test_kda_fwd_noalloc_allocates_nothing_and_replays_in_a_graph(cuda_device):
    """After a first call (which resolves the scratch address on this device), a call changes
    neither the device's free memory nor torch's reserved pool, although the workspace it
    uses (u and w, 8 MiB here) is far larger than any allocation granule; the call also
    captures into a HIP graph whose replays, with eager work and synchronisations between
    them, reproduce the eager outputs bit for bit."""
    from tops.utils import ChunkPlan
    B, T, H, K, V = 2, 1024, 4, 128, 128
    dev = cuda_device
    d = kda_inputs(B, T, H, K, V, 91, h0=True)
    q, k, v = (to_dev(d[x], torch.bfloat16, dev) for x in "qkv")
    g, beta, h0 = (to_dev(d[x], torch.float32, dev) for x in ("g", "beta", "h0"))
    plan = ChunkPlan.get(B, T, None, dev)
    o = torch.empty(B, T, H, V, device=dev, dtype=torch.bfloat16)
    ht = torch.empty(B, H, K, V, device=dev, dtype=torch.float32)
    scale = K ** -0.5
    run = lambda: _call("tops_kda_chunk_fwd_noalloc", q, k, v, g, beta, h0, o, ht, plan,  # noqa: E731
                        B, T, H, K, V, scale)
    print("no-alloc: warm-up call", flush=True)
    run()
    torch.cuda.synchronize()
    free0, res0 = torch.cuda.mem_get_info(dev)[0], torch.cuda.memory_reserved(dev)
    run()
    torch.cuda.synchronize()
    free1, res1 = torch.cuda.mem_get_info(dev)[0], torch.cuda.memory_reserved(dev)
    assert res1 == res0 and abs(free1 - free0) < (1 << 20), (free0, free1, res0, res1)
    ref_o, ref_ht = o.clone(), ht.clone()
    print("no-alloc: graph capture", flush=True)
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            run()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for i in range(3):
        o.zero_()
        ht.fill_(float(i + 1))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        print(f"no-alloc: replay {i}", flush=True)
        assert torch.equal(o, ref_o) and torch.equal(ht, ref_ht), f"replay {i}"


_CHILD = r"""
import sys
sys.path[:0] = [ROOT + "/pallas-kernel_amd", ROOT + "/tests"]
import torch
from tops import _native as N
from tops.ops.gla import chunk_gla
from tops.ops.kda import chunk_kda
from tops.utils import ChunkPlan
torch.zeros(1, device="cuda")
torch.cuda.synchronize()
B, T, H, K, V = 1, 128, 2, 64, 64
q = torch.randn(B, T, H, K, device="cuda")
g = torch.nn.functional.logsigmoid(torch.randn(B, T, H, K, device="cuda")) / 16
beta = torch.sigmoid(torch.randn(B, T, H, device="cuda"))
qb = q.to(torch.bfloat16)
ob = torch.empty_like(qb)
plan = ChunkPlan.get(B, T, None, q.device)
torch.cuda.synchronize()
free0 = torch.cuda.mem_get_info()[0]
with torch.no_grad():
    chunk_gla(q, q, q, g)
    chunk_kda(q, q, q, g, beta)
torch.cuda.synchronize()
free1 = torch.cuda.mem_get_info()[0]
N.call("tops_kda_chunk_fwd_noalloc", N.ptr(qb), N.ptr(qb), N.ptr(qb), N.ptr(g), N.ptr(beta), None,
       N.ptr(ob), None, None, None, None, plan.total, B, T, H, K, V, plan.N,
       N.dtype_code(qb.dtype), 0.125, N.stream())
torch.cuda.synchronize()
free2 = torch.cuda.mem_get_info()[0]
print("FREE", free0, free1, free2, flush=True)
"""


def test_scratch_reserved_only_by_noalloc_callers(cuda_device):
    """The static scratch lives in the code object of the entry point's own source file, which
    the HIP runtime loads on a device the first time it is used there.  So a process that runs
    the other kernels (chunk_gla, chunk_kda) does not hold the 64 MiB; the first no-alloc call
    does.  Measured in a fresh child process (device free memory before and after)."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    print("no-alloc: child process for the scratch residency check", flush=True)
    r = subprocess.run([sys.executable, "-c", f"ROOT = {root!r}\n" + _CHILD], capture_output=True,
                       text=True, timeout=180)
    assert r.returncode == 0, r.stderr[-2000:]
    line = [x for x in r.stdout.splitlines() if x.startswith("FREE")][-1]
    free0, free1, free2 = (int(x) for x in line.split()[1:])
    MiB = 1 << 20
    print(f"other kernels: -{(free0 - free1) / MiB:.1f} MiB; no-alloc call: "
          f"-{(free1 - free2) / MiB:.1f} MiB")
    assert free0 - free1 < 32 * MiB
    assert free1 - free2 >= 64 * MiB
