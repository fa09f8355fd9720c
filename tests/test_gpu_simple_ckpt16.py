"""Simple GLA with fp16 state checkpoints (tops_simple_gla_chunk_fwd_c16 / _bwd_dh_c16 /
_bwd_dqkg_c16) against fp32 checkpoints and the float64 oracle.

For bf16 inputs with one gate per token (g [B,T,H]) or a scalar g_gamma [H], chunk_simple_gla
training keeps h and dh per chunk as fp16 times a power-of-two factor per (chunk, head, 64
columns of V); set_checkpoint_layout("full32") keeps fp32.  The sweeps compute in fp32
either way (separately compiled instances: fp32 contraction may differ in the last bit), so
o, ht, dv, dh0 match the fp32 layout to 1e-5 (fp32) / one bf16 ulp (bf16 outputs, 1e-3);
dq, dk, dg read the checkpoints and match the fp32 layout and the oracle
(tops/cpu/ops/simple_gla restated) within the north-star 2e-3.  fused_chunk_simple_gla
(g_gamma, its own autograd op) takes the same checkpoints.  Cases: K, V of 32 / 64 / 128,
ragged T, h0 / dht, varlen with one-token sequences, a long sequence (segmented sweeps).
"""
import numpy as np
import pytest
import torch

from oracle import simple_gla as S
from _inputs import simple_gla_inputs
from _gpu import to_dev, seen, host, rel

pytestmark = pytest.mark.gpu

CASES = [
    dict(B=2, T=200, H=2, K=128, V=128, gate="g", h0=True),
    dict(B=1, T=256, H=2, K=128, V=64, gate="gamma"),
    dict(B=2, T=100, H=3, K=64, V=64, gate="gamma", h0=True),
    dict(B=1, T=160, H=2, K=32, V=64, gate="g", h0=True, cu=[0, 1, 64, 65, 160]),
    dict(B=1, T=1000, H=4, K=128, V=128, gate="g", cu=[0, 100, 101, 460, 1000]),
    dict(B=1, T=8192, H=2, K=128, V=128, gate="g", h0=True),
]


def _id(c):
    return "-".join(f"{k}{v}" for k, v in c.items() if k != "cu") + ("-varlen" if "cu" in c else "")


def _run(cfg, device, layout):
    from tops.ops.simple_gla import chunk_simple_gla
    from tops.utils import set_checkpoint_layout, checkpoint_layout
    B, T, H, K, V = (cfg[x] for x in "BTHKV")
    cu = cfg.get("cu")
    n = len(cu) - 1 if cu else B
    d = simple_gla_inputs(B, T, H, K, V, seed=T + 3 * K + H, h0=cfg.get("h0", False), N=n,
                          grads=True)
    bf = torch.bfloat16
    q, k, v = (to_dev(d[x], bf, device).requires_grad_() for x in "qkv")
    g = to_dev(d["g"], torch.float32, device).requires_grad_() if cfg["gate"] == "g" else None
    gg = to_dev(d["g_gamma"], torch.float32, device) if cfg["gate"] == "gamma" else None
    h0 = to_dev(d["h0"], torch.float32, device)
    if h0 is not None:
        h0.requires_grad_()
    prev = checkpoint_layout()
    set_checkpoint_layout(layout)
    try:
        o, ht = chunk_simple_gla(q, k, v, gg, initial_state=h0, output_final_state=True, g=g,
                                 cu_seqlens=cu)
        torch.autograd.backward((o, ht), (to_dev(d["do"], bf, device),
                                          to_dev(d["dht"], torch.float32, device)))
        torch.cuda.synchronize()
    finally:
        set_checkpoint_layout(prev)
    out = dict(o=o, ht=ht, dq=q.grad, dk=k.grad, dv=v.grad,
               dg=None if g is None else g.grad, dh0=None if h0 is None else h0.grad)
    return d, out


@pytest.mark.parametrize("cfg", CASES, ids=_id)
def test_simple_ckpt16_vs_fp32_and_oracle(cfg, cuda_device):
    print(f"case {_id(cfg)}", flush=True)
    d, a = _run(cfg, cuda_device, "full")
    _, b = _run(cfg, cuda_device, "full32")
    errs = {}
    for name in ("o", "ht", "dv", "dh0"):
        if a[name] is not None:
            lim = 1e-3 if a[name].dtype == torch.bfloat16 else 1e-5
            e = rel(host(a[name]), host(b[name]))
            assert e <= lim, f"{name}: differs from the fp32 layout by {e:.3e}"
    for name in ("dq", "dk", "dg"):
        if a[name] is not None:
            errs[name + " vs fp32"] = rel(host(a[name]), host(b[name]))
    if cfg["T"] <= 1024:
        bf = torch.bfloat16
        gs = d["g"] if cfg["gate"] == "g" else None
        gam = d["g_gamma"] if cfg["gate"] == "gamma" else None
        sq, sk, sv, sdo = (seen(d[x], bf) for x in ("q", "k", "v", "do"))
        rq, rk, rv, rg, rh0 = S.chunk_simple_gla_bwd(sq, sk, sv, gs, gam, d["h0"], sdo, d["dht"],
                                                     cfg["K"] ** -0.5, cu_seqlens=cfg.get("cu"))
        for name, r in dict(dq=rq, dk=rk, dg=rg).items():
            if a[name] is not None and r is not None:
                errs[name + " vs oracle"] = rel(host(a[name]), r)
    print({k_: f"{e:.2e}" for k_, e in errs.items()})
    bad = {k_: e for k_, e in errs.items() if not e <= 2e-3}
    assert not bad, f"rel err over 2e-3: {bad}"


def test_fused_chunk_simple_gla_ckpt16(cuda_device):
    """fused_chunk_simple_gla (g_gamma) trains through the fp16 checkpoints: gradients match
    the fp32 layout within 2e-3."""
    from tops.ops.simple_gla import fused_chunk_simple_gla
    from tops.utils import set_checkpoint_layout, checkpoint_layout
    B, T, H, K, V = 2, 300, 2, 128, 128
    d = simple_gla_inputs(B, T, H, K, V, seed=41, h0=True, grads=True)
    bf = torch.bfloat16
    res = {}
    prev = checkpoint_layout()
    try:
        for layout in ("full", "full32"):
            set_checkpoint_layout(layout)
            q, k, v = (to_dev(d[x], bf, cuda_device).requires_grad_() for x in "qkv")
            gg = to_dev(d["g_gamma"], torch.float32, cuda_device)
            h0 = to_dev(d["h0"], torch.float32, cuda_device)
            o, ht = fused_chunk_simple_gla(q, k, v, gg, initial_state=h0, output_final_state=True)
            o.backward(to_dev(d["do"], bf, cuda_device))
            torch.cuda.synchronize()
            res[layout] = [host(x) for x in (o, q.grad, k.grad, v.grad)]
    finally:
        set_checkpoint_layout(prev)
    for name, x, y in zip(("o", "dq", "dk", "dv"), res["full"], res["full32"]):
        e = rel(x, y)
        assert e <= 2e-3, f"{name}: fp16 vs fp32 checkpoints rel {e:.3e}"
