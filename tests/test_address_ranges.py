"""CPU check that every buffer access of the chunk kernels stays inside its tensor.

The launches are the ones the ops make (ChunkPlan / SegPlan of tops.utils decide the
sequence-parallel segments, the state passes and the varlen maps); tests/addr_model.py
replays each kernel's per-lane offset arithmetic over every workgroup and chunk.  Cases:
the shapes of test_gpu_reference_shapes.py, test_gpu_simple_gla.py and test_gpu_kda.py, plus
empty sequences.  A planted mistake (the 16-byte read of the per-token scalar gate, the read
that ran 12 bytes past a [B,T,H] gate) must be caught.
"""
import numpy as np
import pytest
import torch

import addr_model as M
from addr_model import C
from tops import utils as U

CUS = 256   # MI355X compute units (the segment planner sizes the split by them)


@pytest.fixture(autouse=True)
def _cus(monkeypatch):
    monkeypatch.setattr(U, "_device_cus", lambda device: CUS)


def _np(t):
    return None if t is None else (t.numpy() if isinstance(t, torch.Tensor) else np.asarray(t))


def chunk_op(B, T, H, K, V, es, cu=None, gate_mode=0, h0=True, dht=True, gate_width_bytes=4,
             paired=None):
    """Forward + backward launches of chunk_gla (gate_mode 0) / chunk_simple_gla (1: g [B,T,H],
    2: g_gamma [H]) on one K, V <= 128 tile, as _fwd_tile / _bwd_tile make them (bf16: the
    interleaved checkpoints and the PAIR dq / dk / dg kernel, unless paired says otherwise)."""
    if paired is None:
        paired = es == 2
    plan = U.ChunkPlan(B, T, cu, "cpu")
    N = plan.N
    sizes = dict(q=B * T * H * K * es, k=B * T * H * K * es, v=B * T * H * V * es,
                 o=B * T * H * V * es, do=B * T * H * V * es, dv=B * T * H * V * es,
                 dq=B * T * H * K * es, dk=B * T * H * K * es,
                 g={0: B * T * H * K * 4, 1: B * T * H * 4, 2: H * 4, 3: H * K * 4}[gate_mode],
                 dg={0: B * T * H * K * 4, 1: B * T * H * 4, 2: 0, 3: B * T * H * K * 4}[gate_mode],
                 hs=plan.total * H * K * V * 4, dhs=plan.total * H * K * V * 4,
                 h0=N * H * K * V * 4, ht=N * H * K * V * 4, dht=N * H * K * V * 4, dh0=N * H * K * V * 4)
    ck = M.Checker(sizes)
    base = dict(H=H, K=K, V=V, gate_mode=gate_mode, g="g")
    sp = plan.segments(H, V)
    for rev in (False, True):
        z, y = ("q", "do") if rev else ("k", "v")
        s_in, s_out = ("dht", "dh0") if rev else ("h0", "ht")
        if sp is None:
            p = dict(base, B=B, T=T, N=N, cu=plan.cu_host if plan.varlen else None,
                     offsets=_np(plan.offsets_dev), q="q", k="k", y=y,
                     out="dv" if rev else "o", ckpt="dhs" if rev else "hs",
                     s0=s_in if (dht if rev else h0) else None, s_fin=s_out)
            M.sweep(ck, p, es, rev, gate_width_bytes=gate_width_bytes)
            continue
        pc = sp.rev if rev else sp.fwd
        if pc.n:
            ck.sizes.update(s_loc=pc.n * H * K * V * 4, dec=pc.n * H * K * 4)
            p = dict(base, B=1, T=B * T, N=pc.n, cu=pc.start, seg_end=pc.end, q=z, k=z, y=y,
                     s_fin="s_loc", dec_fin="dec")
            M.sweep(ck, p, es, rev, st=True, gate_width_bytes=gate_width_bytes)
        ck.sizes.update(init=sp.Nv * H * K * V * 4, fin=sp.Nv * H * K * V * 4)
        p = dict(base, B=1, T=B * T, N=sp.Nv, cu=sp.cu_host, offsets=_np(sp.offsets_dev),
                 q="q", k="k", y=y, out="dv" if rev else "o", ckpt="dhs" if rev else "hs",
                 s0="init", s_fin="fin")
        M.sweep(ck, p, es, rev, gate_width_bytes=gate_width_bytes)
    p = dict(base, B=B, T=T, total=plan.total, cu=plan.cu_host if plan.varlen else None,
             offsets=_np(plan.offsets_dev), chunk_map=_np(plan.chunk_map_dev),
             q="q", k="k", v="v", do="do", hs="hs", dhs="dhs", dq="dq", dk="dk",
             dg="dg" if gate_mode != 2 else None,
             h0="h0" if h0 else None, dht="dht" if dht else None)
    M.dqkg(ck, p, es, es, pair=paired)
    if paired:
        M.dqkg(ck, p, es, es, pair=False)      # the unpaired instance serves the stage API
    return ck


def kda_op(B, T, H, K, V, es, cu=None, h0=True):
    """Forward + backward launches of chunk_kda (tops_kda_chunk_fwd / _bwd)."""
    plan = U.ChunkPlan(B, T, cu, "cpu")
    N, tot = plan.N, plan.total
    rK, rV = B * T * H * K, B * T * H * V
    sizes = dict(q=rK * es, k=rK * es, v=rV * es, o=rV * es, do=rV * es, dv=rV * es, dq=rK * es,
                 dk=rK * es, g=rK * 4, beta=B * T * H * 4, dbeta=B * T * H * 4, u=rV * 4, w=rK * 4,
                 vnew=rV * 4, tt=tot * H * C * C * 4, hs=tot * H * K * V * 4, dhs=tot * H * K * V * 4,
                 dvnt=tot * H * V * C * 4, dk_wy=rK * 4, dg_wy=rK * 4, dg=rK * 4,
                 h0=N * H * K * V * 4, ht=N * H * K * V * 4, dht=N * H * K * V * 4, dh0=N * H * K * V * 4)
    ck = M.Checker(sizes)
    vl = dict(cu=plan.cu_host if plan.varlen else None, offsets=_np(plan.offsets_dev),
              chunk_map=_np(plan.chunk_map_dev))
    M.kda_prep(ck, dict(vl, H=H, K=K, V=V, B=B, T=T, total=tot, k="k", g="g", v="v", beta="beta",
                        u="u", w="w", tt="tt"), es)
    sw = dict(vl, B=B, T=T, H=H, K=K, V=V, N=N, gate_mode=0, q="q", k="k", g="g", w="w")
    M.sweep(ck, dict(sw, u="u", y32="vnew", out="o", ckpt="hs", s0="h0" if h0 else None, s_fin="ht"),
            es, rev=False, delta=True)
    M.sweep(ck, dict(sw, y="do", y32="dvnt", ckpt="dhs", s0="dht", s_fin="dh0"), es, rev=True, delta=True)
    # bf16: the WY backward and dq / dk / dg run as one kernel (kda_bwd_fused.hip)
    fused = es == 2
    M.kda_wy(ck, dict(vl, H=H, K=K, V=V, B=B, T=T, total=tot, k="k", g="g", v="v", beta="beta",
                      tt="tt", dvnt="dvnt", vnew="vnew", hs="hs", dv="dv", dbeta="dbeta",
                      dk_wy="dk_wy", dg_wy="dg_wy"), es, fused=fused)
    M.dqkg(ck, dict(vl, B=B, T=T, H=H, K=K, V=V, total=tot, gate_mode=0, q="q", k="k", v="vnew",
                    g="g", do="do", hs="hs", dhs="dhs", dq="dq", dk="dk", dg="dg",
                    dk_add=None if fused else "dk_wy", dg_add=None if fused else "dg_wy"), es, 4)
    return ck


def _tile(K, V):
    """The per-tile K, V the ops launch (K, V > 128 run as equal slices)."""
    nk, nv = -(-K // 128), -(-V // 128)
    return K // nk, V // nv


# test_gpu_reference_shapes.py: chunk_gla's reference shapes (fp32 / bf16) and the g_gamma forms
def _ref_cases():
    import test_gpu_reference_shapes as R
    return R.REF


@pytest.mark.parametrize("es", [4, 2], ids=["f32", "bf16"])
def test_reference_chunk_gla_shapes_in_bounds(es):
    for c in _ref_cases():
        B, T, H, K, V = (c[x] for x in "BTHKV")
        ck = chunk_op(B, T, H, K, V, es, cu=c.get("cu"), gate_mode=0, h0=c.get("h0", False))
        assert ck.count > 0


SIMPLE = [  # test_gpu_simple_gla.py CASES (+ the reference module's K / V = 256, chunk 128)
    dict(B=2, T=64, H=2, K=32, V=32, gate=1), dict(B=2, T=100, H=3, K=64, V=64, gate=2),
    dict(B=1, T=37, H=2, K=16, V=32, gate=1), dict(B=1, T=1, H=2, K=32, V=64, gate=2),
    dict(B=2, T=200, H=2, K=128, V=128, gate=1), dict(B=1, T=256, H=2, K=128, V=64, gate=2),
    dict(B=1, T=1000, H=4, K=128, V=128, gate=1, cu=[0, 86, 203, 419, 430, 611, 700, 951, 1000]),
    dict(B=1, T=300, H=2, K=64, V=128, gate=2, cu=[0, 13, 140, 141, 300]),
    dict(B=1, T=160, H=2, K=32, V=64, gate=1, cu=[0, 10, 64, 65, 160]),
    dict(B=2, T=512, H=2, K=256, V=128, gate=2), dict(B=1, T=512, H=4, K=128, V=256, gate=2),
]


@pytest.mark.parametrize("es", [4, 2], ids=["f32", "bf16"])
@pytest.mark.parametrize("c", SIMPLE, ids=lambda c: "B{B}-T{T}-H{H}-K{K}-V{V}-gate{gate}".format(**c))
def test_simple_gla_in_bounds(c, es):
    K, V = _tile(c["K"], c["V"])
    chunk_op(c["B"], c["T"], c["H"], K, V, es, cu=c.get("cu"), gate_mode=c["gate"])


@pytest.mark.parametrize("es", [4, 2], ids=["f32", "bf16"])
def test_constant_gate_chunk_gla_in_bounds(es):
    """chunk_gla with g = None or a g_gamma constant over (B, T): the [H, K] gate mode."""
    chunk_op(2, 130, 3, 64, 64, es, gate_mode=3)
    chunk_op(1, 300, 2, 128, 128, es, cu=[0, 13, 140, 141, 300], gate_mode=3)


def test_planted_wide_scalar_gate_read_is_caught():
    """The 16-byte read of the one-word gate [B,T,H] runs past the tensor on its last row."""
    with pytest.raises(M.OOBError, match="g"):
        chunk_op(2, 64, 2, 32, 32, 4, gate_mode=1, gate_width_bytes=16)


def test_planted_rows_range_past_end_is_caught():
    ck = M.Checker(dict(x=100 * 4))
    ck.acc("x", 96 * 4, 0, 0, 16, "last four elements")          # ends at the tensor end
    with pytest.raises(M.OOBError):
        ck.acc("x", 97 * 4, 0, 0, 16, "one element past the end")


KDA = [dict(B=2, T=64, H=2, K=32, V=32), dict(B=1, T=100, H=3, K=64, V=128),
       dict(B=2, T=130, H=2, K=128, V=64), dict(B=1, T=1, H=2, K=16, V=32),
       dict(B=1, T=300, H=2, K=64, V=64, cu=[0, 13, 140, 141, 300]),
       dict(B=1, T=256, H=4, K=128, V=128, cu=[0, 64, 128, 192, 256]),
       dict(B=1, T=150, H=2, K=40, V=120), dict(B=2, T=70, H=1, K=64, V=24),
       dict(B=1, T=129, H=2, K=120, V=56), dict(B=1, T=96, H=2, K=24, V=128)]


@pytest.mark.parametrize("es", [4, 2], ids=["f32", "bf16"])
@pytest.mark.parametrize("c", KDA, ids=lambda c: "B{B}-T{T}-H{H}-K{K}-V{V}".format(**c))
def test_kda_in_bounds(c, es):
    kda_op(c["B"], c["T"], c["H"], c["K"], c["V"], es, cu=c.get("cu"))


@pytest.mark.parametrize("cu", [[0, 0, 64, 64], [0, 0, 0, 37], [0, 50, 50, 130, 130]])
def test_empty_sequences_in_bounds(cu):
    """Zero-length sequences (0 chunks, the reference's prepare_chunk_indices) walk no chunk,
    in either direction."""
    idx = U.prepare_chunk_indices(np.array(cu), 64)
    lens = np.diff(cu)
    assert idx.shape[0] == int(sum(-(-x // 64) for x in lens))
    for es in (4, 2):
        chunk_op(1, cu[-1], 2, 64, 64, es, cu=cu, gate_mode=0)
        chunk_op(1, cu[-1], 2, 32, 64, es, cu=cu, gate_mode=1)
        kda_op(1, cu[-1], 2, 32, 32, es, cu=cu)


def test_planted_unguarded_empty_prefetch_is_caught():
    """Prefetching chunk cidx(0) = -1 of an empty first sequence reads before the tensor."""
    plan = U.ChunkPlan(1, 64, [0, 0, 64], "cpu")
    ck = M.Checker(dict(q=64 * 2 * 32 * 2, k=64 * 2 * 32 * 2, g=64 * 2 * 32 * 4, do=64 * 2 * 32 * 2))
    p = dict(B=1, T=64, H=2, K=32, V=32, N=2, cu=plan.cu_host, offsets=_np(plan.offsets_dev),
             gate_mode=0, g="g", q="q", k="k", y="do")
    M.sweep(ck, p, 2, rev=True, st=True)
    with pytest.raises(M.OOBError):
        M.sweep(ck, p, 2, rev=True, st=True, unguarded_prefetch=True)


def test_planted_paired_partner_past_end_is_caught():
    """With an odd number of chunks the last pair has no second chunk: reading the partner
    slot of its first chunk without the same-sequence test runs past the checkpoints."""
    B, T, H, K, V = 1, 192, 2, 32, 32          # 3 chunks
    plan = U.ChunkPlan(B, T, None, "cpu")
    sizes = dict(q=B * T * H * K * 2, k=B * T * H * K * 2, v=B * T * H * V * 2, do=B * T * H * V * 2,
                 dq=B * T * H * K * 2, dk=B * T * H * K * 2, g=B * T * H * K * 4, dg=B * T * H * K * 4,
                 hs=plan.total * H * K * V * 4, h0=H * K * V * 4, dht=H * K * V * 4)
    p = dict(B=B, T=T, H=H, K=K, V=V, total=plan.total, cu=None, gate_mode=0, g="g", q="q", k="k",
             v="v", do="do", hs="hs", dq="dq", dk="dk", dg="dg", h0="h0", dht="dht")
    M.dqkg(M.Checker(sizes), p, 2, 2, pair=True)
    with pytest.raises(M.OOBError, match="hs"):
        M.dqkg(M.Checker(sizes), p, 2, 2, pair=True, planted_link=True)


def test_segment_split_in_bounds():
    """Long sequences cut into segments (state pass + combine + segment sweeps)."""
    U.set_sequence_split(None)
    ck = chunk_op(1, 2048, 2, 128, 128, 2, gate_mode=0)
    assert ck.count > 0
    chunk_op(1, 3000, 2, 64, 64, 4, cu=[0, 100, 3000], gate_mode=1)


def reverse_op(B, T, H, K, V, es, cu=None, gate_mode=0, h0=True, planted_shift=False):
    """The launch of tops_chunk_reverse_fwd (fused_recurrent reverse=True without gradients):
    the reverse sweep with q and k exchanged, v as Y, the gate read one token later, no
    checkpoints."""
    plan = U.ChunkPlan(B, T, cu, "cpu")
    N = plan.N
    sizes = dict(q=B * T * H * K * es, k=B * T * H * K * es, v=B * T * H * V * es,
                 o=B * T * H * V * es,
                 g={0: B * T * H * K * 4, 1: B * T * H * 4, 2: H * 4, 3: H * K * 4}[gate_mode],
                 h0=N * H * K * V * 4, ht=N * H * K * V * 4)
    ck = M.Checker(sizes)
    p = dict(B=B, T=T, H=H, K=K, V=V, N=N, cu=plan.cu_host if plan.varlen else None, offsets=None,
             gate_mode=gate_mode, g="g", q="k", k="q", y="v", out="o",
             s0="h0" if h0 else None, s_fin="ht")
    M.sweep(ck, p, es, rev=True, gshift=True, planted_shift=planted_shift)
    return ck


# test_gpu_reverse_native.py's launches
REVERSE = [dict(B=2, T=64, H=2, K=32, V=32), dict(B=2, T=50, H=2, K=64, V=64),
           dict(B=1, T=1, H=2, K=32, V=64), dict(B=2, T=200, H=3, K=16, V=40),
           dict(B=1, T=150, H=2, K=32, V=32, cu=[0, 13, 13, 64, 65, 150]),
           dict(B=1, T=4, H=2, K=8, V=16, cu=[0, 1, 2, 3, 4]),
           dict(B=2, T=256, H=2, K=128, V=128), dict(B=1, T=70, H=1, K=128, V=200),
           dict(B=1, T=150, H=2, K=32, V=48, cu=[0, 40, 40, 99, 150])]


@pytest.mark.parametrize("es", [4, 2], ids=["f32", "bf16"])
@pytest.mark.parametrize("c", REVERSE, ids=lambda c: "B{B}-T{T}-H{H}-K{K}-V{V}".format(**c))
def test_reverse_native_in_bounds(c, es):
    for gm in (0, 1, 2, 3):
        ck = reverse_op(c["B"], c["T"], c["H"], c["K"], c["V"], es, cu=c.get("cu"), gate_mode=gm)
        assert ck.count > 0


def test_planted_reverse_first_chunk_shift_is_caught():
    """Reading the first chunk's gate rows one token early runs before the tensor for the
    first sequence."""
    reverse_op(1, 100, 2, 32, 32, 4, gate_mode=0)
    with pytest.raises(M.OOBError, match="g"):
        reverse_op(1, 100, 2, 32, 32, 4, gate_mode=0, planted_shift=True)
    with pytest.raises(M.OOBError, match="g"):
        reverse_op(1, 100, 2, 32, 32, 4, gate_mode=1, planted_shift=True)


def gv_op(B, T, H, K, V, cu=None, h0=True):
    """The launch of tops_gla_chunk_fwd_gv (fused_recurrent_gla with gv, no gk, no gradients):
    the bf16 forward sweep with g = gv [B,T,H,V], no checkpoints."""
    plan = U.ChunkPlan(B, T, cu, "cpu")
    N, es = plan.N, 2
    sizes = dict(q=B * T * H * K * es, k=B * T * H * K * es, v=B * T * H * V * es,
                 o=B * T * H * V * es, g=B * T * H * V * 4, h0=N * H * K * V * 4,
                 ht=N * H * K * V * 4)
    ck = M.Checker(sizes)
    p = dict(B=B, T=T, H=H, K=K, V=V, N=N, cu=plan.cu_host if plan.varlen else None, offsets=None,
             gate_mode=2, g="g", q="q", k="k", y="v", out="o", s0="h0" if h0 else None,
             s_fin="ht")
    M.sweep(ck, p, es, rev=False, gv=True)
    return ck


# test_gpu_gv_native.py's launches
GV = [dict(B=2, T=64, H=2, K=32, V=32), dict(B=2, T=50, H=2, K=64, V=64),
      dict(B=1, T=1, H=2, K=32, V=64), dict(B=2, T=200, H=3, K=16, V=40),
      dict(B=1, T=150, H=2, K=32, V=32, cu=[0, 13, 13, 64, 65, 150]),
      dict(B=2, T=256, H=2, K=128, V=128), dict(B=1, T=70, H=1, K=128, V=200),
      dict(B=1, T=100, H=2, K=24, V=72)]


@pytest.mark.parametrize("c", GV, ids=lambda c: "B{B}-T{T}-H{H}-K{K}-V{V}".format(**c))
def test_gv_native_in_bounds(c):
    assert gv_op(c["B"], c["T"], c["H"], c["K"], c["V"], cu=c.get("cu")).count > 0


DECODE = [dict(B=3, T=1, H=2, K=128, V=128), dict(B=2, T=5, H=1, K=64, V=20),
          dict(B=1, T=9, H=2, K=36, V=100, cu=[0, 1, 1, 4, 9]), dict(B=2, T=16, H=1, K=128, V=64),
          dict(B=1, T=3, H=3, K=4, V=7), dict(B=2, T=3, H=2, K=64, V=160)]


@pytest.mark.parametrize("es", [4, 2], ids=["f32", "bf16"])
@pytest.mark.parametrize("c", DECODE, ids=lambda c: "B{B}-T{T}-H{H}-K{K}-V{V}".format(**c))
def test_fr_decode_in_bounds(c, es):
    """The decode kernel's state, input and output accesses, both directions, all optional
    tensors bound."""
    B, T, H, K, V = (c[x] for x in "BTHKV")
    cu = c.get("cu")
    N = len(cu) - 1 if cu else B
    rK, rV = B * T * H * K, B * T * H * V
    sizes = dict(q=rK * es, k=rK * es, gk=rK * 4, v=rV * es, gv=rV * 4, o=rV * es, o32=rV * 4,
                 h0=N * H * K * V * 4, ht=N * H * K * V * 4, beta=B * T * H * 4)
    for rev in (False, True):
        ck = M.Checker(sizes)
        M.fr_decode(ck, dict(B=B, T=T, H=H, K=K, V=V, cu=cu, gk="gk", gv="gv", s0="h0",
                             s_fin="ht", o32="o32", reverse=rev), es)
        assert ck.count > 0
    ck = M.Checker(sizes)        # the KDA instance (tops_kda_fused_recurrent_fwd_decode)
    M.fr_decode(ck, dict(B=B, T=T, H=H, K=K, V=V, cu=cu, gk="gk", beta="beta", s0="h0",
                         s_fin="ht"), es)
