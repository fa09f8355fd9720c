"""Host-side checks of the stage / export surface (CPU, no kernel calls): the names each
package exports at the reference's import paths and the argument errors raised before
any device work."""
import pytest
import torch


def test_gla_exports_match_reference_names():
    import tops.ops.gla as G
    # tops/ops/gla/__init__.py:19-35
    names = ["naive_recurrent_gla", "chunk_gla", "chunk_local_cumsum", "chunk_fwd_h",
             "chunk_gla_fwd_intra_gk", "chunk_gla_fwd_o_gk", "chunk_gla_fwd",
             "chunk_gla_bwd_dA_ref", "chunk_gla_bwd_dv_ref", "chunk_gla_bwd_dqk_intra_ref",
             "chunk_gla_bwd_dqkg_ref", "chunk_gla_bwd", "chunk_gla_bwd_with_pl", "fused_chunk_gla",
             "fused_recurrent_gla", "fused_recurrent_gla_bwd"]
    for n in names:
        assert n in G.__all__ and callable(getattr(G, n)), n


def test_simple_gla_and_ops_exports():
    import importlib
    import tops.ops as OPS
    # tops.ops re-exports the simple_gla function under the subpackage's name (as the
    # reference does), so fetch the subpackage itself from the import system
    S = importlib.import_module("tops.ops.simple_gla")
    assert OPS.__all__ == ["chunk_kda", "chunk_kda_fwd", "fused_recurrent_kda", "simple_gla"]
    for n in ("simple_gla", "chunk_simple_gla", "chunk_simple_gla_fwd",
              "chunk_simple_gla_fwd_varlen", "chunk_simple_gla_bwd", "fused_chunk_simple_gla",
              "fused_chunk_simple_gla_fwd", "fused_chunk_simple_gla_bwd",
              "fused_recurrent_simple_gla", "simple_gla_naive", "SimpleGLAKernelMode",
              "simple_gla_fwd", "simple_gla_bwd"):
        assert hasattr(S, n), n
    assert [m.value for m in S.SimpleGLAKernelMode] == ["chunk", "fused_chunk"]


def test_kda_exports_match_reference_names():
    import tops.ops.kda as KD
    for n in ("chunk_kda", "chunk_kda_fwd", "fused_recurrent_kda", "chunk_kda_bwd_intra"):
        assert n in KD.__all__ and callable(getattr(KD, n)), n


def test_common_exports():
    from tops.ops.common import chunk_h, cumsum
    for n in ("chunk_fwd_h_ref", "chunk_fwd_h_kernel", "chunk_fwd_h_kernel_varlen", "chunk_bwd_dh_ref", "chunk_bwd_dh_kernel"):
        assert callable(getattr(chunk_h, n))
    assert callable(cumsum.chunk_local_cumsum_vector)
    # the KDA stages at the reference's module paths
    from tops.ops.common import chunk_delta_h
    from tops.ops.kda import chunk_intra
    for n in ("chunk_gated_delta_rule_fwd_h", "chunk_gated_delta_rule_fwd_h_ref"):
        assert callable(getattr(chunk_delta_h, n))
    assert callable(chunk_intra.kda_intra_chunk_fwd)


def test_argument_errors_before_device_work():
    from tops.ops.common.cumsum import chunk_local_cumsum_vector
    from tops.ops.simple_gla import simple_gla_bwd
    g = torch.zeros(1, 8, 1, 4)
    with pytest.raises(AssertionError, match="power of 2"):
        chunk_local_cumsum_vector(g, 12)
    with pytest.raises(AssertionError, match="4-D"):
        chunk_local_cumsum_vector(torch.zeros(8, 4), 8)
    with pytest.raises(Exception, match="not support"):
        simple_gla_bwd(g, g, g, g, g_gamma=torch.zeros(1), mode="bogus")


def test_tiling_and_slice_views():
    """The K / V slicing of the chunk core (host only): slice widths, the accumulation mode of
    each slice, and state views that address a slice of [.., K, V] without a copy."""
    from tops.ops._chunk_core import _acc, _kv_view, tiling
    assert tiling(256, 128, True) == (2, 128, 1, 128)
    assert tiling(192, 256, True) == (2, 96, 2, 128)
    assert tiling(64, 512, False) == (1, 64, 1, 512)
    with pytest.raises(NotImplementedError):
        tiling(200, 64, True)                   # 2 slices of 100: not a multiple of 8
    assert [_acc(i, 1) for i in range(1)] == [0]
    assert [_acc(i, 2) for i in range(2)] == [1, 3]
    assert [_acc(i, 4) for i in range(4)] == [1, 2, 2, 3]
    hs = torch.randn(3, 2, 256, 192)
    t = _kv_view(hs, 128, 128, 96, 96)
    assert t.data_ptr() == hs.data_ptr() + (128 * 192 + 96) * 4
    assert t.stride() == hs.stride()
    assert torch.equal(t, hs[:, :, 128:, 96:])
    assert _kv_view(None, 0, 8) is None


def test_reference_utils_helpers():
    import numpy as np
    from tops.utils import (align_up, assert_shape, assert_shape_or_none, next_power_of_2,
                            pad_to_multiple)
    assert [next_power_of_2(n) for n in (1, 2, 3, 64, 65)] == [1, 2, 4, 64, 128]
    assert align_up(65, 64) == 128 and align_up(64, 64) == 64
    t = torch.ones(2, 5, 3)
    p = pad_to_multiple(t, [4, 2], [1, 2], 0.0)
    assert p.shape == (2, 8, 4) and float(p.sum()) == 30.0
    assert pad_to_multiple(np.ones((3, 2)), 4, 0, -1).shape == (4, 2)
    assert_shape([t, t], (2, 5, 3), ("a", "b"))
    assert_shape_or_none([t, None], (2, 5, 3))
    with pytest.raises(AssertionError, match=r"\[x\]"):
        assert_shape(t, (2, 5), "x")
