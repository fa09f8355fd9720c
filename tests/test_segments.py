"""Sequence-parallel segmentation (tops.utils.SegPlan) on the CPU.

1. The host plan: segments are chunk-aligned, cover every sequence exactly once in token
   order, carry the global chunk numbering of the unsplit plan, and list the state-pass
   segments the forward / reverse sweeps need.
2. The decomposition the segment kernels implement, checked with the oracle's serial state
   recurrences (tops/cpu/ops/common/chunk_h.py:179-226 forward, :387-427 reverse): every
   segment swept from a zero state gives (sum of log-gates, local end state); the scan over
   those, indexed exactly as tops_chunk_state_combine indexes them (seg_first / st_first),
   reproduces the state entering every segment and the sequence's final state / dh0.
"""
import numpy as np
import pytest

from oracle.common import chunk_fwd_h, chunk_bwd_dh, chunk_local_cumsum
from tops.utils import SegPlan, ChunkPlan, set_sequence_split

C = 64


def _plan(cu, m, per=None, cus=None):
    cu = np.asarray(cu, np.int64)
    chunks = -(-(cu[1:] - cu[:-1]) // C)
    return SegPlan(cu, chunks, np.asarray(m), C, "cpu", per=per, cus=cus), chunks


LAYOUTS = [
    ([0, 700], [4]),
    ([0, 15, 1960, 2132, 2269, 3173, 11907, 12437, 16384], [1, 2, 1, 1, 1, 3, 1, 5]),
    ([0, 64, 128, 1000], [1, 1, 7]),
    ([0, 1, 640, 641], [1, 10, 1]),
]


@pytest.mark.parametrize("pieces", [None, (1, 40), (4, 16)], ids=["whole", "fine", "coarse"])
@pytest.mark.parametrize("cu,m", LAYOUTS)
def test_plan_layout(cu, m, pieces):
    per, cus = pieces if pieces else (None, None)
    sp, chunks = _plan(cu, m, per, cus)
    cuv = sp.cu_host
    assert sp.Nv == int(np.sum(m)) and cuv[0] == 0 and cuv[-1] == cu[-1]
    assert np.all(np.diff(cuv) > 0)
    offs = sp.offsets_dev.numpy()
    coff = np.concatenate([[0], np.cumsum(chunks)])
    assert offs[-1] == coff[-1]
    sf = sp.seg_first
    for n in range(len(cu) - 1):
        segs = range(sf[n], sf[n + 1])
        assert len(segs) == m[n]
        assert cuv[sf[n]] == cu[n] and cuv[sf[n + 1]] == cu[n + 1]
        for j in segs:
            # chunk-aligned inside the sequence; numbering continues the sequence's chunks
            assert (cuv[j] - cu[n]) % C == 0
            assert offs[j] == coff[n] + (cuv[j] - cu[n]) // C
        seg_chunks = -(-np.diff(cuv[sf[n]:sf[n + 1] + 1]) // C)
        assert seg_chunks.max() - seg_chunks.min() <= 1            # near-equal segments
        for rev, pc in ((False, sp.fwd), (True, sp.rev)):
            st, en, dst = pc.start[pc.first[n]:pc.first[n + 1]], pc.end[pc.first[n]:pc.first[n + 1]], \
                pc.dst[pc.first[n]:pc.first[n + 1]]
            # the pieces tile, in sweep order, exactly the segments that hand a state on
            handing = range(sf[n], sf[n + 1] - 1) if not rev else range(sf[n + 1] - 1, sf[n], -1)
            lo = [cuv[j] for j in handing]
            hi = [cuv[j + 1] for j in handing]
            if not rev:
                assert list(st[:1]) == lo[:1] and np.all(st[1:] == en[:-1])
                assert (en[-1] if len(en) else None) == (hi[-1] if hi else None)
            else:
                assert list(en[:1]) == hi[:1] and np.all(en[1:] == st[:-1])
                assert (st[-1] if len(st) else None) == (lo[-1] if lo else None)
            assert np.all((st - cu[n]) % C == 0) and np.all(en > st)
            # a piece hands into the next segment in sweep order exactly when it ends one
            want = []
            for j in handing:
                k = np.sum((st >= cuv[j]) & (en <= cuv[j + 1]))
                want += [-1] * (k - 1) + [j + 1 if not rev else j - 1]
            assert list(dst) == want
            if pieces:
                assert np.all(-(-(en - st) // C) <= sp.sub + 1)
    assert np.array_equal(sp.first_dev.numpy(), sf[:-1])
    assert np.array_equal(sp.last_dev.numpy(), sf[1:] - 1)


def test_split_counts():
    ch = np.array([1, 31, 3, 3, 15, 137, 9, 62])
    assert list(SegPlan.split_counts(ch, 4, None)) == [1, 1, 1, 1, 1, 3, 1, 1]
    assert list(SegPlan.split_counts(ch, 4, 0)) == [1] * 8
    assert list(SegPlan.split_counts(ch, 4, 40)) == [1, 1, 1, 1, 1, 4, 1, 2]
    # enough slots for everything: nothing split below MIN_SEG_CHUNKS
    assert list(SegPlan.split_counts(np.array([8, 8]), 1000, None)) == [1, 1]
    # one long sequence on an idle chip is cut toward total / slots chunks
    assert list(SegPlan.split_counts(np.array([512]), 8, None)) == [8]
    # pieces: one round of state-pass workgroups, never below MIN_PIECE_CHUNKS
    assert SegPlan.piece_chunks(91, 64, 256) == 23
    assert SegPlan.piece_chunks(10, 1, 256) == 4


def test_no_split_without_gpu_when_forced_off():
    set_sequence_split(0)
    try:
        assert ChunkPlan(1, 4096, None, "cpu").segments(2, 128) is None
    finally:
        set_sequence_split(None)
    with pytest.raises(ValueError):
        set_sequence_split(-1)


def _gates(rng, T, H, K):
    return -np.logaddexp(0.0, -rng.standard_normal((1, T, H, K))) / 4


@pytest.mark.parametrize("pieces", [None, (1, 40)], ids=["whole", "fine"])
@pytest.mark.parametrize("reverse", [False, True], ids=["fwd", "rev"])
def test_segment_scan_matches_serial_recurrence(reverse, pieces):
    rng = np.random.default_rng(5)
    H, K, V = 2, 8, 4
    cu = [0, 300, 320, 960]          # ragged first sequence, a one-chunk one, a 10-chunk one
    m = [3, 1, 4]
    per, cus = pieces if pieces else (None, None)
    sp, _ = _plan(cu, m, per, cus)
    T = cu[-1]
    z = rng.standard_normal((1, T, H, K))
    y = rng.standard_normal((1, T, H, V))
    g = _gates(rng, T, H, K)
    s_in = 0.1 * rng.standard_normal((len(cu) - 1, H, K, V))

    def sweep(lo, hi, s0):
        """Oracle recurrence over rows [lo, hi) (padded to whole chunks with zero rows)."""
        L = hi - lo
        P = -(-L // C) * C
        zz, yy, gg = (np.zeros((1, P) + a.shape[2:]) for a in (z, y, g))
        zz[:, :L], yy[:, :L], gg[:, :L] = z[:, lo:hi], y[:, lo:hi], g[:, lo:hi]
        gc = chunk_local_cumsum(gg, C)
        if reverse:
            _, s = chunk_bwd_dh(zz, yy, gk=gc, dht=s0, scale=0.5, C=C)
        else:
            _, s = chunk_fwd_h(zz, yy, gk=gc, h0=s0, C=C)
        return s[0], gg[0, :L].sum(0)          # end state, summed log-gates [H,K]

    pc = sp.rev if reverse else sp.fwd
    # 1. state pass over the pieces, from a zero state
    loc = [sweep(a, b, None) for a, b in zip(pc.start, pc.end)]
    # 2. the combine scan, as tops_chunk_state_combine runs it
    cuv, sf = sp.cu_host, sp.seg_first
    init = np.full((sp.Nv, H, K, V), np.nan)
    for n in range(len(cu) - 1):
        S = s_in[n].copy()
        init[sf[n + 1] - 1 if reverse else sf[n]] = S
        for e in range(pc.first[n], pc.first[n + 1]):
            s_loc, dec = loc[e]
            S = np.exp(dec)[:, :, None] * S + s_loc
            if pc.dst[e] >= 0:
                init[pc.dst[e]] = S
    # every segment's incoming state equals the serial sweep's state at its boundary, and the
    # last segment in sweep order, swept from it, ends in the sequence's final state
    for n in range(len(cu) - 1):
        for j in range(sf[n], sf[n + 1]):
            lo, hi = cuv[j], cuv[j + 1]
            if reverse:
                want, _ = sweep(hi, cu[n + 1], s_in[n][None]) if hi < cu[n + 1] else (s_in[n], None)
            else:
                want, _ = sweep(cu[n], lo, s_in[n][None]) if lo > cu[n] else (s_in[n], None)
            np.testing.assert_allclose(init[j], want, rtol=1e-12, atol=1e-12)
        full, _ = sweep(cu[n], cu[n + 1], s_in[n][None])
        j = sf[n] if reverse else sf[n + 1] - 1
        fin, _ = sweep(cuv[j], cuv[j + 1], init[j][None])
        np.testing.assert_allclose(fin, full, rtol=1e-12, atol=1e-12)
