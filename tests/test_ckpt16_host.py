"""Host side of the fp16 state checkpoints: the layout switch and the scale-back of the
stage API (no GPU)."""
import pytest
import torch

from tops import utils as U
from tops.ops._chunk_core import (GATE_K, GATE_S, GATE_GAMMA, GATE_GAMMA_K, States16, _c16,
                                  pack_states, states_fp32,
                                  unpack_states)


def test_layout_switch():
    prev = U.checkpoint_layout()
    try:
        for layout in ("full", "full32", "paired"):
            U.set_checkpoint_layout(layout)
            assert U.checkpoint_layout() == layout
        with pytest.raises(ValueError):
            U.set_checkpoint_layout("fp16")
    finally:
        U.set_checkpoint_layout(prev)


def test_c16_selection():
    bf = torch.zeros(1, dtype=torch.bfloat16)
    f32 = torch.zeros(1)
    prev = U.checkpoint_layout()
    try:
        U.set_checkpoint_layout("full")
        assert _c16(bf, GATE_K, 128, 128)
        assert not _c16(f32, GATE_K, 128, 128)          # fp32 inputs keep fp32 states
        assert _c16(bf, GATE_S, 128, 128)               # one gate per token: fp16 too
        assert _c16(bf, GATE_GAMMA, 128, 128)
        assert not _c16(bf, GATE_GAMMA_K, 128, 128)     # per-channel constants: fp32
        assert not _c16(bf, GATE_K, 256, 128)           # channel slices: fp32
        assert not _c16(bf, GATE_K, 128, 192)
        U.set_checkpoint_layout("full32")
        assert not _c16(bf, GATE_K, 128, 128)
    finally:
        U.set_checkpoint_layout(prev)


def test_states_fp32_applies_tile_factors():
    # 3 chunks, 2 heads, K = 4, V = 96: two 64-column tiles, the second one partial
    h = torch.arange(3 * 2 * 4 * 96, dtype=torch.float32).remainder(7.0).sub(3.0)
    h = h.reshape(3, 2, 4, 96).to(torch.float16)
    scale = torch.tensor([0.5, 8.0]).repeat(3, 2, 1) * torch.arange(1, 4).view(3, 1, 1)
    s = States16(h, scale)
    out = states_fp32(s)
    assert out.dtype == torch.float32 and out.shape == (3, 2, 4, 96)
    for c in range(3):
        for hh in range(2):
            for vt, (lo, hi) in enumerate(((0, 64), (64, 96))):
                want = h[c, hh, :, lo:hi].float() * scale[c, hh, vt]
                assert torch.equal(out[c, hh, :, lo:hi], want)
    plain = torch.randn(2, 2, 4, 8)
    assert states_fp32(plain) is plain


def test_pack_unpack_round_trip():
    s = States16(torch.zeros(2, 1, 4, 8, dtype=torch.float16), torch.ones(2, 1, 1))
    a, b = pack_states(s)
    assert a is s.h and b is s.scale
    t = unpack_states(a, b)
    assert isinstance(t, States16) and t.h is s.h and t.scale is s.scale
    plain = torch.zeros(2, 1, 4, 8)
    a, b = pack_states(plain)
    assert a is plain and b is None and unpack_states(a, b) is plain
