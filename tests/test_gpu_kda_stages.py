"""kda_intra_chunk_fwd and chunk_gated_delta_rule_fwd_h on MI355X vs the float64 oracle.

The oracle restates tops/ops/kda/chunk_intra.py:91-281 and
tops/cpu/ops/common/chunk_delta_h.py:22-118 (+ the scalar gate and varlen forms of
tops/ops/common/chunk_delta_h.py), pinned by tests/test_oracle_kda_stages.py.  Inputs are
KDA-style (L2-normalised q, k; sigmoid beta; logsigmoid gates, cumsummed per chunk in log2
units), compared on the values the kernels see (bf16-rounded for bf16 inputs).
Tolerance: fp32 1e-4, bf16 2e-3 (relative L2), every output.
"""
import numpy as np
import pytest
import torch

from oracle import kda as KD
from _inputs import kda_inputs
from _gpu import to_dev, seen, host, rel, tol

pytestmark = pytest.mark.gpu
LN2 = np.log(2.0)


def _log2_cumsum(g, C):
    B, T = g.shape[:2]
    return (np.cumsum(g.reshape(B, T // C, C, *g.shape[2:]), axis=2) / LN2).reshape(g.shape)


def _hf(x):
    return np.ascontiguousarray(np.swapaxes(x, 1, 2))


INTRA = [dict(B=1, H=2, T=128, K=32, V=32, C=64), dict(B=2, H=1, T=64, K=16, V=32, C=16),
         dict(B=1, H=2, T=96, K=64, V=48, C=32), dict(B=1, H=1, T=256, K=128, V=128, C=128),
         dict(B=1, H=2, T=128, K=128, V=64, C=64, seg=True),
         dict(B=2, H=2, T=64, K=16, V=16, C=32, seg=True)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("c", INTRA, ids=lambda c: "-".join(f"{k}{v}" for k, v in c.items()))
def test_kda_intra_chunk_fwd(c, dtype, cuda_device):
    from tops.ops.kda.chunk_intra import kda_intra_chunk_fwd
    B, H, T, K, V, C = (c[x] for x in ("B", "H", "T", "K", "V", "C"))
    d = kda_inputs(B, T, H, K, V, seed=T + K + C, gate_div=2.0)
    G = _log2_cumsum(np.float64(d["g"]), C).astype(np.float32)
    seg = None
    if c.get("seg"):
        rng = np.random.default_rng(T)
        seg = np.cumsum(rng.random((B, T)) < 0.05, axis=1).astype(np.int32)
    q, k, g, beta, v = (_hf(x) for x in (d["q"], d["k"], G, d["beta"], d["v"]))
    scale = K ** -0.5
    got = kda_intra_chunk_fwd(to_dev(q, dtype, cuda_device), to_dev(k, dtype, cuda_device),
                              to_dev(g, torch.float32, cuda_device),
                              to_dev(beta, torch.float32, cuda_device),
                              to_dev(v, dtype, cuda_device),
                              segment_ids=None if seg is None else torch.from_numpy(seg),
                              scale=scale, chunk_size=C)
    torch.cuda.synchronize()
    ref = KD.kda_intra_chunk_fwd(seen(q, dtype), seen(k, dtype), g, beta, seen(v, dtype),
                                 segment_ids=seg, scale=scale, chunk_size=C)
    for name, a, b in zip(("u", "w", "qg", "kg", "Aqk", "Akk_inv"), got, ref):
        assert a.dtype == dtype and tuple(a.shape) == b.shape, name
        e = rel(host(a), b)
        assert e < tol(dtype), f"{name}: rel {e:.2e}"


DELTA = [dict(B=2, T=128, H=2, K=64, V=64, C=64, gate="gk", h0=True),
         dict(B=1, T=256, H=2, K=128, V=128, C=64, gate="gk", h0=False),
         dict(B=1, T=128, H=3, K=32, V=96, C=32, gate="g", h0=True),
         dict(B=2, T=64, H=1, K=16, V=16, C=16, gate="both", h0=True),
         dict(B=1, T=64, H=2, K=32, V=32, C=64, gate="none", h0=True),
         dict(B=1, T=300, H=2, K=64, V=80, C=64, gate="gk", h0=True, cu=[0, 13, 140, 141, 300]),
         dict(B=1, T=200, H=2, K=32, V=32, C=32, gate="both", h0=False, cu=[0, 0, 64, 200])]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("c", DELTA, ids=lambda c: "-".join(f"{k}{v}" for k, v in c.items()))
def test_chunk_gated_delta_rule_fwd_h(c, dtype, cuda_device):
    from tops.ops.common import chunk_gated_delta_rule_fwd_h
    B, T, H, K, V, C = (c[x] for x in ("B", "T", "H", "K", "V", "C"))
    cu = c.get("cu")
    N = len(cu) - 1 if cu else B
    rng = np.random.default_rng(T + K)
    k = (rng.standard_normal((B, T, H, K)) * 0.3).astype(np.float32)
    w = (rng.standard_normal((B, T, H, K)) * 0.1).astype(np.float32)
    u = rng.standard_normal((B, T, H, V)).astype(np.float32)
    g = gk = None
    if c["gate"] in ("g", "both"):
        g = (-np.abs(rng.standard_normal((B, T, H))) / 8).astype(np.float32)
    if c["gate"] in ("gk", "both"):
        gk = (-np.abs(rng.standard_normal((B, T, H, K))) / 8).astype(np.float32)
    h0 = (0.1 * rng.standard_normal((N, H, K, V))).astype(np.float32) if c["h0"] else None
    f = lambda x: None if x is None else to_dev(x, torch.float32, cuda_device)   # noqa: E731
    h, vn, ht = chunk_gated_delta_rule_fwd_h(
        to_dev(k, dtype, cuda_device), to_dev(w, dtype, cuda_device), to_dev(u, dtype, cuda_device),
        g=f(g), gk=f(gk), initial_state=f(h0), output_final_state=True, chunk_size=C,
        cu_seqlens=cu)
    torch.cuda.synchronize()
    hr, vr, tr = KD.chunk_gated_delta_rule_fwd_h(seen(k, dtype), seen(w, dtype), seen(u, dtype),
                                                 g=g, gk=gk, initial_state=h0,
                                                 output_final_state=True, chunk_size=C,
                                                 cu_seqlens=cu)
    assert h.dtype == dtype and vn.dtype == torch.float32 and ht.dtype == torch.float32
    assert tuple(h.shape) == hr.shape and tuple(vn.shape) == vr.shape
    for name, a, b in (("h", h, hr), ("v_new", vn, vr), ("ht", ht, tr)):
        e = rel(host(a), b)
        assert e < tol(dtype), f"{name}: rel {e:.2e}"


def test_delta_rule_natural_gates_and_no_v_new(cuda_device):
    """use_exp2=False takes natural-log gates; save_new_value=False returns no v_new."""
    from tops.ops.common import chunk_gated_delta_rule_fwd_h
    rng = np.random.default_rng(1)
    B, T, H, K, V, C = 1, 128, 2, 32, 32, 64
    k, w = (rng.standard_normal((2, B, T, H, K)) * 0.2).astype(np.float32)
    u = rng.standard_normal((B, T, H, V)).astype(np.float32)
    gk = (-np.abs(rng.standard_normal((B, T, H, K))) / 8).astype(np.float32)
    d = lambda x: to_dev(x, torch.float32, cuda_device)                     # noqa: E731
    h, vn, ht = chunk_gated_delta_rule_fwd_h(d(k), d(w), d(u), gk=d(gk * LN2), chunk_size=C,
                                             save_new_value=False, use_exp2=False)
    hr, _, _ = KD.chunk_gated_delta_rule_fwd_h(k, w, u, gk=gk, chunk_size=C)
    assert vn is None and ht is None
    assert rel(host(h), hr) < 1e-4


def test_kda_stages_compose_to_chunk_kda(cuda_device):
    """The reference's chunk_kda_fwd pipeline from the stage functions (gate cumsum ->
    intra solve -> delta-rule state pass -> output) reproduces chunk_kda's o and ht."""
    from tops.ops.kda import chunk_kda
    from tops.ops.kda.chunk_intra import kda_intra_chunk_fwd
    from tops.ops.common import chunk_gated_delta_rule_fwd_h
    B, T, H, K, V, C = 1, 128, 2, 64, 64, 64
    d = kda_inputs(B, T, H, K, V, seed=7, gate_div=2.0, h0=True)
    dev = lambda x: to_dev(x, torch.float32, cuda_device)                   # noqa: E731
    G = _log2_cumsum(np.float64(d["g"]), C).astype(np.float32)
    scale = K ** -0.5
    u, w, qg, kg, Aqk, _ = kda_intra_chunk_fwd(*(dev(_hf(x)) for x in (d["q"], d["k"], G)),
                                               dev(_hf(d["beta"])), dev(_hf(d["v"])),
                                               scale=scale, chunk_size=C)
    tf = lambda x: x.transpose(1, 2).contiguous()                           # noqa: E731
    h, v_new, ht = chunk_gated_delta_rule_fwd_h(tf(kg), tf(w), tf(u), gk=dev(G),
                                                initial_state=dev(d["h0"]),
                                                output_final_state=True, chunk_size=C)
    # o = (scale q 2^G) h + Aqk v_new, per chunk
    NT = T // C
    qgs = tf(qg).reshape(B, NT, C, H, K) * scale
    o = torch.einsum("bnchk,bnhkv->bnchv", qgs, h.float()) + \
        torch.einsum("bhnij,bnjhv->bnihv", Aqk.float(), v_new.reshape(B, NT, C, H, V))
    o_ref, ht_ref = chunk_kda(dev(d["q"]), dev(d["k"]), dev(d["v"]), dev(d["g"]), dev(d["beta"]),
                              scale=scale, initial_state=dev(d["h0"]), output_final_state=True)
    torch.cuda.synchronize()
    assert rel(host(o.reshape(B, T, H, V)), host(o_ref)) < 1e-4
    assert rel(host(ht), host(ht_ref)) < 1e-4
