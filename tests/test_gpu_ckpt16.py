"""fp16 state checkpoints (tops_gla_chunk_fwd_c16 / _bwd_dh_c16 / _bwd_dqkg_c16) against
fp32 checkpoints and the float64 oracle.

The default checkpoint layout of chunk_gla training on bf16 inputs with per-channel gates
keeps h (forward) and dh (reverse sweep) as fp16 times a power-of-two factor per (chunk,
head, 64 columns of V); set_checkpoint_layout("full32") keeps them as fp32.  Only the
dq / dk / dg kernel reads the checkpoints, so
  * o, ht (forward) and dv, dh0 (reverse sweep) equal those of the fp32 layout up to fp32
    contraction: the sweeps compute in fp32 either way and only the stored copies differ, but
    the two layouts run separately compiled kernel instances, whose fused multiply-adds may
    differ (relative L2 <= 1e-5 for fp32 outputs, <= 1e-3 for bf16 ones: one-ulp flips);
  * dq, dk, dg are within the north-star bf16 tolerance of the oracle (2e-3 relative L2,
    tops/ops/gla/chunk.py:1103-1199 forward and :1447-1509 backward), and within 2e-3 of
    the fp32 layout (fp16 keeps 11 significant bits of each scaled state; the factor keeps
    the largest entry of a tile in [2^14, 2^15));
  * the stage API (chunk_gla_fwd) hands back checkpoints scaled back to fp32 within 1e-3
    relative L2 of the fp32 layout's.
Cases: K of 32 / 64 / 128, V of 64 / 96 / 128 (a partial 64-column tile), ragged T,
varlen with one-token sequences, h0 / dht, and long sequences (segmented sweeps).
"""
import numpy as np
import pytest
import torch

from oracle import gla as O
from _inputs import gla_inputs
from _gpu import to_dev, seen, host, rel, out_bound

pytestmark = pytest.mark.gpu

CASES = [
    dict(B=2, T=300, H=3, K=128, V=128, seed=21, h0=True),
    dict(B=1, T=513, H=2, K=64, V=64, seed=22, h0=True),
    dict(B=2, T=200, H=2, K=32, V=96, seed=23),
    dict(B=1, T=700, H=2, K=128, V=64, seed=24, cu=[0, 1, 129, 130, 700], h0=True),
    dict(B=1, T=1000, H=4, K=128, V=128, seed=25, cu=[0, 1, 64, 65, 300, 1000], h0=True),
    dict(B=1, T=1, H=2, K=128, V=128, seed=26, h0=True),
    dict(B=1, T=8192, H=2, K=128, V=128, seed=27, h0=True),
]


def _id(c):
    return "-".join(f"{k}{v}" for k, v in c.items() if k != "seed")


def _run(cfg, device, layout):
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
    prev = checkpoint_layout()
    set_checkpoint_layout(layout)
    try:
        o, ht = chunk_gla(q, k, v, g, initial_state=h0, output_final_state=True, cu_seqlens=cu)
        do = to_dev(d["do"], bf, device)
        dht = to_dev(d["dht"], torch.float32, device)
        torch.autograd.backward((o, ht), (do, dht))
        torch.cuda.synchronize()
    finally:
        set_checkpoint_layout(prev)
    out = dict(o=o, ht=ht, dq=q.grad, dk=k.grad, dv=v.grad, dg=g.grad,
               dh0=None if h0 is None else h0.grad)
    return d, out


@pytest.mark.parametrize("cfg", CASES, ids=_id)
def test_ckpt16_vs_fp32_and_oracle(cfg, cuda_device):
    print(f"case {_id(cfg)}", flush=True)
    d, a = _run(cfg, cuda_device, "full")
    _, b = _run(cfg, cuda_device, "full32")
    for name in ("o", "ht", "dv", "dh0"):
        if a[name] is not None:
            lim = 1e-3 if a[name].dtype == torch.bfloat16 else 1e-5
            e = rel(host(a[name]), host(b[name]))
            assert e <= lim, f"{name}: differs from the fp32 layout by {e:.3e}"
    bf = torch.bfloat16
    big = cfg["T"] > 4096
    if not big:
        s = {x: seen(d[x], bf) for x in ("q", "k", "v", "do")}
        rq, rk, rv, rg, rh0 = O.chunk_gla_bwd(s["q"], s["k"], s["v"], d["g"], cfg["K"] ** -0.5,
                                              d.get("h0"), s["do"], d["dht"], chunk_size=64,
                                              cu_seqlens=cfg.get("cu"))
        for name, r in dict(dq=rq, dk=rk, dg=rg).items():
            e = rel(host(a[name]), r)
            bound = out_bound(r, bf, a[name].dtype)
            assert e < bound, f"{name}: fp16-checkpoint rel-err {e:.3e} vs oracle ({bound:.2e})"
    for name in ("dq", "dk", "dg"):
        ab = rel(host(a[name]), host(b[name]))
        assert ab <= 2e-3, f"{name}: fp16 vs fp32 checkpoints rel {ab:.3e}"


def test_stage_api_states_scaled_back(cuda_device):
    from tops.ops.gla.chunk import chunk_gla_fwd
    from tops.utils import set_checkpoint_layout, checkpoint_layout
    B, T, H, K, V = 2, 333, 2, 128, 96
    d = gla_inputs(B, T, H, K, V, 31, gate_div=16.0, h0=True)
    bf = torch.bfloat16
    q, k, v = (to_dev(d[x], bf, cuda_device) for x in "qkv")
    g = to_dev(d["g"], torch.float32, cuda_device)
    h0 = to_dev(d["h0"], torch.float32, cuda_device)
    hs = {}
    prev = checkpoint_layout()
    try:
        for layout in ("full", "full32"):
            set_checkpoint_layout(layout)
            _, _, h, _, _ = chunk_gla_fwd(q, k, v, g, None, None, K ** -0.5, h0, True)
            assert h.dtype == torch.float32
            hs[layout] = host(h)
    finally:
        set_checkpoint_layout(prev)
    assert hs["full"].shape == hs["full32"].shape
    e = rel(hs["full"], hs["full32"])
    assert e <= 1e-3, f"scaled-back fp16 checkpoints rel {e:.3e}"
