"""The software-pipelined chunk sweep (gla_sweep_pipe.hip) against the serial sweep
(gla_sweep.hip) and the float64 oracle.

bf16 chunk_gla calls with per-channel gates run on the pipelined kernel;
TOPS_SWEEP_SERIAL=1 routes the same calls to the serial kernel.  Both perform the same
products in the same order, so they may differ only by fp32 contraction (the last bit of an
fp32 value, one bf16 ulp of a rounded output).  Each case runs forward + backward
(tops/ops/gla/chunk.py:1103-1199 and :1447-1509) under both schedules and checks
  * every output against the oracle at the north-star bf16 tolerance (2e-3; for tiny
    tensors the rounding floor of _gpu.out_bound), and
  * the two schedules against each other: relative L2 <= 1e-5 for fp32 outputs (ht, dg,
    dh0), <= 1e-3 for bf16 outputs (o, dq, dk, dv: a handful of one-ulp flips).
Cases cover K of 32 / 64 / 128 (the kernel's three row splits), ragged T, varlen with
one-token sequences, h0 / dht, and the fp32 and paired checkpoint layouts (empty sequences:
the oracle rejects them, as tops/cpu does; other modules run them).  The default layout keeps
fp16 checkpoints, which only the pipelined kernel writes: test_gpu_ckpt16.py covers it.
"""
import os

import numpy as np
import pytest
import torch

from oracle import gla as O
from _inputs import gla_inputs
from _gpu import to_dev, seen, host, rel, out_bound

pytestmark = pytest.mark.gpu

CASES = [
    dict(B=2, T=300, H=3, K=128, V=128, seed=11, h0=True),
    dict(B=1, T=513, H=2, K=64, V=64, seed=12, h0=True),
    dict(B=2, T=200, H=2, K=32, V=96, seed=13),
    dict(B=1, T=700, H=2, K=128, V=64, seed=14, cu=[0, 1, 129, 130, 700], h0=True),
    dict(B=1, T=1000, H=4, K=128, V=128, seed=15, cu=[0, 1, 64, 65, 300, 1000], h0=True),
    dict(B=1, T=64, H=2, K=128, V=128, seed=16, h0=True),
    dict(B=1, T=1, H=2, K=128, V=128, seed=17, h0=True),
]


def _id(c):
    return "-".join(f"{k}{v}" for k, v in c.items() if k != "seed")


def _run(cfg, device, serial, layout="full32"):
    from tops.ops.gla import chunk_gla
    from tops.utils import set_checkpoint_layout, checkpoint_layout
    B, T, H, K, V = (cfg[x] for x in "BTHKV")
    cu = cfg.get("cu")
    n = len(cu) - 1 if cu else B
    d = gla_inputs(B, T, H, K, V, cfg["seed"], gate_div=16.0, h0=cfg.get("h0", False), N=n,
                   grads=True)
    bf = torch.bfloat16
    q, k, v = (to_dev(d[x], bf, device).requires_grad_() for x in "qkv")
    g = to_dev(d["g"], torch.float32, device).requires_grad_()
    h0 = to_dev(d["h0"], torch.float32, device)
    if h0 is not None:
        h0.requires_grad_()
    prev_env = os.environ.get("TOPS_SWEEP_SERIAL")
    prev_layout = checkpoint_layout()
    os.environ["TOPS_SWEEP_SERIAL"] = "1" if serial else "0"
    set_checkpoint_layout(layout)
    try:
        o, ht = chunk_gla(q, k, v, g, initial_state=h0, output_final_state=True,
                          cu_seqlens=cu)
        do = to_dev(d["do"], bf, device)
        dht = to_dev(d["dht"], torch.float32, device)
        torch.autograd.backward((o, ht), (do, dht))
        torch.cuda.synchronize()
    finally:
        set_checkpoint_layout(prev_layout)
        if prev_env is None:
            os.environ.pop("TOPS_SWEEP_SERIAL", None)
        else:
            os.environ["TOPS_SWEEP_SERIAL"] = prev_env
    out = dict(o=o, ht=ht, dq=q.grad, dk=k.grad, dv=v.grad, dg=g.grad,
               dh0=None if h0 is None else h0.grad)
    return d, out


@pytest.mark.parametrize("layout", ["full32", "paired"])
@pytest.mark.parametrize("cfg", CASES, ids=_id)
def test_pipe_vs_serial_and_oracle(cfg, layout, cuda_device):
    print(f"case {_id(cfg)} layout={layout}", flush=True)
    d, a = _run(cfg, cuda_device, serial=False, layout=layout)
    _, b = _run(cfg, cuda_device, serial=True, layout=layout)
    bf = torch.bfloat16
    s = {x: seen(d[x], bf) for x in ("q", "k", "v", "do")}
    K = cfg["K"]
    ro, rht = O.chunk_gla(s["q"], s["k"], s["v"], d["g"], initial_state=d.get("h0"),
                          output_final_state=True, chunk_size=64, cu_seqlens=cfg.get("cu"))
    rq, rk, rv, rg, rh0 = O.chunk_gla_bwd(s["q"], s["k"], s["v"], d["g"], K ** -0.5,
                                          d.get("h0"), s["do"], d["dht"], chunk_size=64,
                                          cu_seqlens=cfg.get("cu"))
    ref = dict(o=ro, ht=rht, dq=rq, dk=rk, dv=rv, dg=rg, dh0=rh0)
    for name, r in ref.items():
        if a[name] is None:
            continue
        x, y = host(a[name]), host(b[name])
        stored = a[name].dtype
        e = rel(x, r)
        bound = out_bound(r, bf, stored)
        assert e < bound, f"{name}: pipelined rel-err {e:.3e} vs oracle (bound {bound:.2e})"
        lim = 1e-3 if stored == bf else 1e-5
        ab = rel(x, y)
        assert ab <= lim, f"{name}: pipelined vs serial rel {ab:.3e} > {lim}"
