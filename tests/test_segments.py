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


def _plan(cu, m):
    cu = np.asarray(cu, np.int64)
    chunks = -(-(cu[1:] - cu[:-1]) // C)
    return SegPlan(cu, chunks, np.asarray(m), C, "cpu"), chunks


@pytest.mark.parametrize("cu,m", [
    ([0, 700], [4]),
    ([0, 15, 1960, 2132, 2269, 3173, 11907, 12437, 16384], [1, 2, 1, 1, 1, 3, 1, 5]),
    ([0, 64, 128, 1000], [1, 1, 7]),
    ([0, 1, 640, 641], [1, 10, 1]),
])
def test_plan_layout(cu, m):
    sp, chunks = _plan(cu, m)
    cuv = sp.cu_host
    assert sp.Nv == int(np.sum(m)) and cuv[0] == 0 and cuv[-1] == cu[-1]
    assert np.all(np.diff(cuv) > 0)
    offs = sp.offsets_dev.numpy()
    coff = np.concatenate([[0], np.cumsum(chunks)])
    assert offs[-1] == coff[-1]
    sf = sp.seg_first
    st = sp.st_first_dev.numpy()
    fs, fe = sp.fwd_start_dev.numpy(), sp.fwd_end_dev.numpy()
    rs, re = sp.rev_start_dev.numpy(), sp.rev_end_dev.numpy()
    assert sp.n_state == int(np.sum(np.asarray(m) - 1)) == len(fs) == len(rs)
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
        assert st[n + 1] - st[n] == m[n] - 1
        for i, j in enumerate(range(sf[n], sf[n + 1] - 1)):
            e = st[n] + i
            assert (fs[e], fe[e]) == (cuv[j], cuv[j + 1])          # all but the last
            assert (rs[e], re[e]) == (cuv[j + 1], cuv[j + 2])      # all but the first
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


@pytest.mark.parametrize("reverse", [False, True], ids=["fwd", "rev"])
def test_segment_scan_matches_serial_recurrence(reverse):
    rng = np.random.default_rng(5)
    H, K, V = 2, 8, 4
    cu = [0, 300, 320, 960]          # ragged first sequence, a one-chunk one, a 10-chunk one
    m = [3, 1, 4]
    sp, _ = _plan(cu, m)
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

    # 1. state pass over the segments that hand a state on, from a zero state
    starts = sp.rev_start_dev.numpy() if reverse else sp.fwd_start_dev.numpy()
    ends = sp.rev_end_dev.numpy() if reverse else sp.fwd_end_dev.numpy()
    loc = [sweep(a, b, None) for a, b in zip(starts, ends)]
    # 2. the combine scan, indexed as tops_chunk_state_combine does
    cuv, sf, st = sp.cu_host, sp.seg_first, sp.st_first_dev.numpy()
    for n in range(len(cu) - 1):
        j0, mm, e0 = sf[n], sf[n + 1] - sf[n], st[n]
        S = s_in[n][None].copy()
        for i in range(mm):
            j = mm - 1 - i if reverse else i
            lo, hi = cuv[j0 + j], cuv[j0 + j + 1]
            # the state entering segment j equals the serial sweep's state at its boundary
            if reverse:
                want, _ = sweep(hi, cu[n + 1], s_in[n][None])
            else:
                want, _ = sweep(cu[n], lo, s_in[n][None]) if lo > cu[n] else (s_in[n], None)
            np.testing.assert_allclose(S[0], want, rtol=1e-12, atol=1e-12)
            if i + 1 < mm:
                s_loc, dec = loc[e0 + (j - 1 if reverse else j)]
                S = np.exp(dec)[None, :, :, None] * S + s_loc[None]
        full, _ = sweep(cu[n], cu[n + 1], s_in[n][None])
        last_lo, last_hi = (cuv[j0], cuv[j0 + 1]) if reverse else (cuv[j0 + mm - 1], cuv[j0 + mm])
        fin, _ = sweep(last_lo, last_hi, S)
        np.testing.assert_allclose(fin, full, rtol=1e-12, atol=1e-12)
