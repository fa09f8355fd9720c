"""chunk_kda on MI355X vs the float64 KDA oracle (tops/cpu/ops/kda restated).

Stage checks of the forward (w, T, v_new, the per-chunk states) against the oracle's
exposed intermediates, then forward + backward through torch autograd (o, final state,
dq, dk, dv, dbeta, dg, dh0) for fp32 and bf16 inputs: aligned and ragged T, K != V,
h0 / dht, varlen packing with non-chunk-aligned segments (each sequence checked against
its own oracle run), and BASELINE config 5 at reduced T.  Inputs follow config 5:
L2-normalised q, k; beta = sigmoid(N(0,1)); g = logsigmoid(N(0,1)) / 16.
Error metric: relative L2 against the fp64 oracle on the (bf16-rounded) inputs the kernel
saw.  Tolerance: fp32 1e-4, bf16 2e-3.
"""
import numpy as np
import pytest
import torch

from oracle import kda as KO
from _inputs import kda_inputs, varlen_cu
from _gpu import to_dev, seen, host, rel, tol

pytestmark = pytest.mark.gpu

CASES = [
    dict(B=2, T=64, H=2, K=64, V=64),
    dict(B=1, T=200, H=2, K=128, V=128, h0=True),
    dict(B=2, T=128, H=3, K=64, V=128, h0=True),
    dict(B=1, T=130, H=2, K=128, V=32),
    dict(B=1, T=37, H=2, K=32, V=64, h0=True),
    dict(B=1, T=1, H=2, K=64, V=64, h0=True),
    dict(B=1, T=300, H=2, K=128, V=128, h0=True, cu=[0, 13, 140, 141, 300]),
    dict(B=1, T=1000, H=2, K=128, V=128, cu=varlen_cu(1000, 6, 77)),
    dict(B=1, T=1024, H=4, K=128, V=128),     # config 5 shape at reduced T
    # the remaining channel-pass / column-tile instances (K, V padded to 32, 64, 128), with
    # channels and columns past K / V in the last pass or tile
    dict(B=1, T=100, H=2, K=32, V=32),
    dict(B=1, T=150, H=2, K=40, V=120, h0=True),
    dict(B=2, T=70, H=1, K=64, V=24),
    dict(B=1, T=129, H=2, K=120, V=56, h0=True),
    dict(B=1, T=96, H=2, K=24, V=128, h0=True),
]


def _id(c):
    return "-".join(f"{k}{v}" for k, v in c.items() if k != "cu") + ("-varlen" if "cu" in c else "")


def _oracle(d, dtype, cu, scale):
    """fp64 oracle forward + backward, per sequence for varlen."""
    sq, sk, sv, sdo = (seen(d[x], dtype) for x in ("q", "k", "v", "do"))
    g, b, h0, dht = d["g"], d["beta"], d["h0"], d["dht"]
    segs = [(0, sq.shape[1], None)] if cu is None else [(cu[i], cu[i + 1], i) for i in range(len(cu) - 1)]
    outs = {x: [] for x in ("o", "dq", "dk", "dv", "db", "dg")}
    hts, dh0s = [], []
    for s, e, n in segs:
        sl = (slice(None), slice(s, e))
        h0n = None if h0 is None else (h0 if n is None else h0[n:n + 1])
        dhtn = dht if n is None else dht[n:n + 1]
        o, ht = KO.chunk_kda(sq[sl], sk[sl], sv[sl], g[sl], b[sl], scale, h0n, True)
        dq, dk, dv, db, dg, dh0 = KO.chunk_kda_bwd(sq[sl], sk[sl], sv[sl], g[sl], b[sl], scale, h0n,
                                                   sdo[sl], dhtn)
        for key, val in zip(("o", "dq", "dk", "dv", "db", "dg"), (o, dq, dk, dv, db, dg)):
            outs[key].append(val)
        hts.append(ht)
        dh0s.append(dh0)
    res = {key: np.concatenate(v, axis=1) for key, v in outs.items()}
    res["ht"] = np.concatenate(hts, axis=0)
    res["dh0"] = np.concatenate(dh0s, axis=0)
    return res


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
@pytest.mark.parametrize("cfg", CASES, ids=_id)
def test_chunk_kda_fwd_bwd(cfg, dtype, cuda_device):
    from tops.ops.kda import chunk_kda
    B, T, H, K, V = (cfg[x] for x in "BTHKV")
    cu = cfg.get("cu")
    n = len(cu) - 1 if cu else B
    print(f"case {_id(cfg)} {dtype}", flush=True)
    d = kda_inputs(B, T, H, K, V, seed=T + 3 * K + V, h0=cfg.get("h0", False), grads=True, N=n)
    q, k, v = (to_dev(d[x], dtype, cuda_device).requires_grad_() for x in "qkv")
    g = to_dev(d["g"], torch.float32, cuda_device).requires_grad_()
    beta = to_dev(d["beta"], torch.float32, cuda_device).requires_grad_()
    h0 = to_dev(d["h0"], torch.float32, cuda_device)
    if h0 is not None:
        h0.requires_grad_()
    scale = K ** -0.5
    o, ht = chunk_kda(q, k, v, g, beta, scale=scale, initial_state=h0, output_final_state=True,
                      cu_seqlens=cu)
    torch.autograd.backward((o, ht), (to_dev(d["do"], dtype, cuda_device),
                                      to_dev(d["dht"], torch.float32, cuda_device)))
    torch.cuda.synchronize()
    ref = _oracle(d, dtype, cu, scale)
    t = tol(dtype)
    errs = {"o": rel(host(o), ref["o"]), "ht": rel(host(ht), ref["ht"]),
            "dq": rel(host(q.grad), ref["dq"]), "dk": rel(host(k.grad), ref["dk"]),
            "dv": rel(host(v.grad), ref["dv"]), "dbeta": rel(host(beta.grad), ref["db"]),
            "dg": rel(host(g.grad), ref["dg"])}
    if h0 is not None:
        errs["dh0"] = rel(host(h0.grad), ref["dh0"])
    print({k_: f"{e:.2e}" for k_, e in errs.items()})
    bad = {k_: e for k_, e in errs.items() if not e <= t}
    assert not bad, f"rel err over {t}: {bad}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_kda_forward_stages(dtype, cuda_device):
    """w, T, v_new and the per-chunk states against the oracle's intermediates."""
    from tops.ops.kda.chunk import _fwd
    from tops.ops._chunk_core import states_fp32
    from tops.utils import ChunkPlan
    B, T, H, K, V = 2, 192, 2, 128, 64
    d = kda_inputs(B, T, H, K, V, seed=5, h0=True)
    q, k, v = (to_dev(d[x], dtype, cuda_device) for x in "qkv")
    g, beta, h0 = (to_dev(d[x], torch.float32, cuda_device) for x in ("g", "beta", "h0"))
    scale = K ** -0.5
    plan = ChunkPlan(B, T, None, cuda_device)
    o, ht, (w, tt, vn, hs) = _fwd(q, k, v, g, beta, h0, scale, True, plan, keep=True)
    hs = states_fp32(hs)          # bf16 inputs keep fp16 checkpoints with tile factors
    torch.cuda.synchronize()
    P = KO.chunk_kda_fwd_parts(seen(d["q"], dtype), seen(d["k"], dtype), seen(d["v"], dtype),
                               d["g"], d["beta"], scale, d["h0"])
    NT = T // 64
    t = tol(dtype)
    # oracle T is [B,NT,i,j,H]; the kernel stores T^T per (chunk, head): tt[b*NT+n, h, i, j] = T[j][i]
    T_ref = np.transpose(P["T"], (0, 1, 4, 3, 2)).reshape(B * NT, H, 64, 64)
    errs = {"T": rel(host(tt), T_ref),
            "w": rel(host(w), P["w"].reshape(B, T, H, K)),
            "v_new": rel(host(vn), P["v_new"].reshape(B, T, H, V)),
            "h": rel(host(hs), P["S"].reshape(B * NT, H, K, V)),
            "o": rel(host(o), P["o"]), "ht": rel(host(ht), P["ht"])}
    print({k_: f"{e:.2e}" for k_, e in errs.items()})
    bad = {k_: e for k_, e in errs.items() if not e <= t}
    assert not bad, f"rel err over {t}: {bad}"


def _intra_ref(d, C, scale, cu=None):
    """Oracle g_cumsum (log2, chunk-local at C), Aqk and Akk_inv [B,T,H,C]: the reference's
    chunk_kda_fwd outputs (tops/ops/kda/chunk.py:120-190), each sequence of a varlen batch
    padded to a multiple of C and chunked on its own."""
    from oracle import kda_gate as KG
    q, k, v, g, beta = (d[x] for x in ("q", "k", "v", "g", "beta"))
    B, T, H, K = q.shape
    gc = KG.kda_gate_chunk_cumsum(g, C, cu)
    spans = [(0, T)] if cu is None else list(zip(cu[:-1], cu[1:]))
    aqk = np.zeros((B, T, H, C))
    akk = np.zeros((B, T, H, C))
    for s, e in spans:
        n = e - s
        if n == 0:
            continue
        Tp = -(-n // C) * C
        def hf(x):
            y = np.zeros((B, Tp) + x.shape[2:])
            y[:, :n] = x[:, s:e]
            return np.swapaxes(y, 1, 2)
        *_, A, Ai = KO.kda_intra_chunk_fwd(hf(q), hf(k), hf(gc), hf(beta), hf(v), scale=scale,
                                           chunk_size=C)
        flat = lambda M: np.swapaxes(M.reshape(B, H, Tp, C), 1, 2)[:, :n]  # noqa: E731
        aqk[:, s:e], akk[:, s:e] = flat(A), flat(Ai)
    return gc, aqk, akk


FWD_EXTRA_CASES = [dict(T=128, C=32), dict(T=192, C=64), dict(T=256, C=128), dict(T=150, C=64),
                   dict(T=70, C=32), dict(T=300, C=64, cu=[0, 13, 140, 141, 300]),
                   dict(T=260, C=128, cu=[0, 200, 260])]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
@pytest.mark.parametrize("case", FWD_EXTRA_CASES,
                         ids=[f"T{c['T']}C{c['C']}{'v' if 'cu' in c else ''}" for c in FWD_EXTRA_CASES])
def test_chunk_kda_fwd_extras(case, dtype, cuda_device):
    """chunk_kda_fwd's (o, ht, g_cumsum, Aqk, Akk_inv) against the oracle at the caller's
    chunk size: g_cumsum the chunk-local log2 cumsum, Aqk and Akk_inv [B,T,H,C] in k.dtype
    (tops/ops/kda/chunk.py:180-190), ragged T and varlen included."""
    from tops.ops.kda import chunk_kda_fwd
    T, C, cu = case["T"], case["C"], case.get("cu")
    B, H, K, V = (1 if cu else 2), 2, 64, 64
    n = B if cu is None else len(cu) - 1
    d = kda_inputs(B, T, H, K, V, seed=8 + C, h0=True, N=n)
    q, k, v = (to_dev(d[x], dtype, cuda_device) for x in "qkv")
    g, beta, h0 = (to_dev(d[x], torch.float32, cuda_device) for x in ("g", "beta", "h0"))
    cut = None if cu is None else torch.tensor(cu, dtype=torch.int32, device=cuda_device)
    o, ht, gc, aqk, akk = chunk_kda_fwd(q, k, v, g, beta, initial_state=h0,
                                        output_final_state=True, cu_seqlens=cut, chunk_size=C)
    scale = K ** -0.5
    dd = dict(d, q=seen(d["q"], dtype), k=seen(d["k"], dtype), v=seen(d["v"], dtype))
    gc_ref, aqk_ref, akk_ref = _intra_ref(dd, C, scale, cu)
    assert aqk.dtype == k.dtype and akk.dtype == k.dtype
    assert tuple(aqk.shape) == (B, T, H, C) and tuple(akk.shape) == (B, T, H, C)
    if cu is None:
        ro, rht = KO.chunk_kda(dd["q"], dd["k"], dd["v"], d["g"], d["beta"], scale, d["h0"], True)
    else:
        parts = [KO.chunk_kda(dd["q"][:, s:e], dd["k"][:, s:e], dd["v"][:, s:e], d["g"][:, s:e],
                              d["beta"][:, s:e], scale, d["h0"][i:i + 1], True)
                 for i, (s, e) in enumerate(zip(cu[:-1], cu[1:]))]
        ro = np.concatenate([p[0] for p in parts], axis=1)
        rht = np.concatenate([p[1] for p in parts], axis=0)
    t = tol(dtype)
    errs = {"g_cumsum": rel(host(gc), gc_ref), "Aqk": rel(host(aqk), aqk_ref),
            "Akk_inv": rel(host(akk), akk_ref), "o": rel(host(o), ro), "ht": rel(host(ht), rht)}
    print({k_: f"{e:.2e}" for k_, e in errs.items()})
    assert errs["g_cumsum"] < 1e-6
    bad = {k_: e for k_, e in errs.items() if not e <= t}
    assert not bad, f"rel err over {t}: {bad}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_fused_recurrent_kda(dtype, cuda_device):
    """fused_recurrent_kda against the per-token recurrence (tops/cpu/ops/kda/naive.py:10-118)."""
    from tops.ops.kda import fused_recurrent_kda
    B, T, H, K, V = 2, 90, 2, 64, 64
    d = kda_inputs(B, T, H, K, V, seed=21, h0=True)
    q, k, v = (to_dev(d[x], dtype, cuda_device) for x in "qkv")
    g, beta, h0 = (to_dev(d[x], torch.float32, cuda_device) for x in ("g", "beta", "h0"))
    o, ht = fused_recurrent_kda(q, k, v, g, beta, initial_state=h0, output_final_state=True)
    assert o.dtype == q.dtype
    ro, rht = KO.naive_recurrent_kda(seen(d["q"], dtype), seen(d["k"], dtype), seen(d["v"], dtype),
                                     d["g"], d["beta"], None, d["h0"], True)
    t = tol(dtype)
    assert rel(host(o), ro) <= t and rel(host(ht), rht) <= t
