"""KDA with fp16 state checkpoints (tops_kda_chunk_fwd_c16 / _bwd_c16) against fp32
checkpoints and the float64 oracle.

For bf16 inputs chunk_kda keeps the forward's state per chunk and the reverse sweep's dS per
chunk as fp16 times a power-of-two factor per (chunk, head, 64 columns of V);
set_checkpoint_layout("full32") keeps them in fp32.  The sweeps compute in fp32 either way,
so o, ht (forward) and dh0 (reverse sweep) are bitwise those of the fp32 layout; the WY /
dq / dk / dg kernel reads the checkpoints, so dq, dk, dv, dbeta, dg are within the north-star
bf16 tolerance (2e-3 relative L2) of the oracle (tops/cpu/ops/kda restated) and within 2e-3
of the fp32 layout.  Cases: K, V of 32 / 64 / 128 and in between (partial passes and tiles),
ragged T, h0 / dht, varlen with one-token sequences, and a long sequence.
"""
import numpy as np
import pytest
import torch

from oracle import kda as KO
from _inputs import kda_inputs
from _gpu import to_dev, seen, host, rel

pytestmark = pytest.mark.gpu

CASES = [
    dict(B=1, T=200, H=2, K=128, V=128, h0=True),
    dict(B=2, T=128, H=3, K=64, V=128, h0=True),
    dict(B=1, T=150, H=2, K=40, V=120, h0=True),
    dict(B=1, T=96, H=2, K=24, V=128, h0=True),
    dict(B=1, T=300, H=2, K=128, V=128, h0=True, cu=[0, 1, 140, 141, 300]),
    dict(B=1, T=4096, H=2, K=128, V=128, h0=True),
]


def _id(c):
    return "-".join(f"{k}{v}" for k, v in c.items() if k != "cu") + ("-varlen" if "cu" in c else "")


def _run(cfg, device, layout):
    from tops.ops.kda import chunk_kda
    from tops.utils import set_checkpoint_layout, checkpoint_layout
    B, T, H, K, V = (cfg[x] for x in "BTHKV")
    cu = cfg.get("cu")
    n = len(cu) - 1 if cu else B
    d = kda_inputs(B, T, H, K, V, seed=T + K + 2 * V, h0=cfg.get("h0", False), grads=True, N=n)
    bf = torch.bfloat16
    q, k, v = (to_dev(d[x], bf, device).requires_grad_() for x in "qkv")
    g = to_dev(d["g"], torch.float32, device).requires_grad_()
    beta = to_dev(d["beta"], torch.float32, device).requires_grad_()
    h0 = to_dev(d["h0"], torch.float32, device)
    if h0 is not None:
        h0.requires_grad_()
    prev = checkpoint_layout()
    set_checkpoint_layout(layout)
    try:
        o, ht = chunk_kda(q, k, v, g, beta, scale=K ** -0.5, initial_state=h0,
                          output_final_state=True, cu_seqlens=cu)
        torch.autograd.backward((o, ht), (to_dev(d["do"], bf, device),
                                          to_dev(d["dht"], torch.float32, device)))
        torch.cuda.synchronize()
    finally:
        set_checkpoint_layout(prev)
    out = dict(o=o, ht=ht, dq=q.grad, dk=k.grad, dv=v.grad, db=beta.grad, dg=g.grad,
               dh0=None if h0 is None else h0.grad)
    return d, out


@pytest.mark.parametrize("cfg", CASES, ids=_id)
def test_kda_ckpt16_vs_fp32_and_oracle(cfg, cuda_device):
    print(f"case {_id(cfg)}", flush=True)
    d, a = _run(cfg, cuda_device, "full")
    _, b = _run(cfg, cuda_device, "full32")
    for name in ("o", "ht", "dh0"):
        if a[name] is not None:
            assert torch.equal(a[name], b[name]), f"{name}: differs from the fp32 layout"
    errs = {}
    for name in ("dq", "dk", "dv", "db", "dg"):
        errs[name + " vs fp32"] = rel(host(a[name]), host(b[name]))
    if cfg["T"] <= 1024:
        bf = torch.bfloat16
        cu = cfg.get("cu")
        sq, sk, sv, sdo = (seen(d[x], bf) for x in ("q", "k", "v", "do"))
        segs = [(0, cfg["T"], None)] if cu is None else [(cu[i], cu[i + 1], i) for i in range(len(cu) - 1)]
        parts = {x: [] for x in ("dq", "dk", "dv", "db", "dg")}
        for s, e, nn in segs:
            sl = (slice(None), slice(s, e))
            h0n = None if d["h0"] is None else (d["h0"] if nn is None else d["h0"][nn:nn + 1])
            dhtn = d["dht"] if nn is None else d["dht"][nn:nn + 1]
            r = KO.chunk_kda_bwd(sq[sl], sk[sl], sv[sl], d["g"][sl], d["beta"][sl], cfg["K"] ** -0.5,
                                 h0n, sdo[sl], dhtn)
            for key, val in zip(("dq", "dk", "dv", "db", "dg"), r[:5]):
                parts[key].append(val)
        for key, v in parts.items():
            errs[key + " vs oracle"] = rel(host(a[key]), np.concatenate(v, axis=1))
    print({k_: f"{e:.2e}" for k_, e in errs.items()})
    bad = {k_: e for k_, e in errs.items() if not e <= 2e-3}
    assert not bad, f"rel err over 2e-3: {bad}"
