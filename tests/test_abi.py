"""The C-ABI library loads without a GPU, exports every entry point include/tops_hip.h
declares, and its host-only routines behave (no kernel launches here)."""
import ctypes
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER_DIR = os.path.join(ROOT, "include")


def _declared():
    names = set()
    for f in os.listdir(HEADER_DIR):
        if f.endswith(".h"):
            text = open(os.path.join(HEADER_DIR, f)).read()
            text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
            names |= set(re.findall(r"\b(tops_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_header_declares_entry_points():
    names = _declared()
    for n in ("tops_gla_chunk_fwd", "tops_gla_chunk_bwd", "tops_gla_chunk_bwd_dh",
              "tops_gla_chunk_bwd_dqkg", "tops_prepare_chunk_indices"):
        assert n in names


def test_library_exports_every_declared_symbol():
    from tops import _native as N
    lib = N.lib()
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, missing
    for n in N.SIGNATURES:
        assert n in _declared(), f"binding {n} has no declaration in include/"


def test_version_and_error_channel():
    from tops import _native as N
    lib = N.lib()
    assert b"gfx950" in lib.tops_version()
    # a shape error is reported before anything touches a device
    rc = lib.tops_gla_chunk_fwd(ctypes.c_void_p(8), ctypes.c_void_p(8), ctypes.c_void_p(8),
                                ctypes.c_void_p(8), None, ctypes.c_void_p(8), None, None, None,
                                None, 1, 16, 1, 200, 64, 1, 0, ctypes.c_float(1.0), None)
    assert rc == -2
    assert b"K <= 128" in lib.tops_last_error()


def test_prepare_chunk_indices_matches_oracle():
    from tops.utils import prepare_chunk_indices
    from oracle.common import prepare_chunk_indices as ref
    for cu, C in (([0, 13, 37, 50], 16), ([0, 64, 128], 64), ([0, 1, 2, 200, 201], 64)):
        np.testing.assert_array_equal(prepare_chunk_indices(cu, C), ref(cu, C))


def test_prepare_chunk_indices_empty_and_negative_segments():
    """An empty sequence gets no chunk (tops/utils.py:71-90: repeat by cdiv(0, C) = 0); a
    negative length is an error."""
    from tops.utils import prepare_chunk_indices
    from oracle.common import prepare_chunk_indices as ref
    for cu in ([0, 10, 10, 20], [0, 0, 64, 64], [0, 0, 0, 5]):
        got = prepare_chunk_indices(cu, 16)
        np.testing.assert_array_equal(got, ref(cu, 16))
        assert 0 not in np.diff(cu) or got.shape[0] == sum(-(-int(x) // 16) for x in np.diff(cu))
    np.testing.assert_array_equal(prepare_chunk_indices([0, 10, 10, 20], 16), [[0, 0], [2, 0]])
    with pytest.raises(ValueError):
        prepare_chunk_indices([0, 10, 5, 20], 16)


def test_kda_noalloc_rejects_oversize_on_host():
    """The allocation-free KDA forward checks its workspace against the static scratch before
    any HIP call: an oversize call returns TOPS_ERR_SHAPE (no device needed)."""
    from tops import _native as N
    L = N.lib()
    cap = L.tops_kda_chunk_fwd_noalloc_max_bytes()
    T = cap // (8 * (128 + 128) * 4) + 64
    rc = N._fn("tops_kda_chunk_fwd_noalloc")(*([None] * 11), 0, 1, T, 8, 128, 128, 1, 1,
                                              ctypes.c_float(1.0), None)
    assert rc == -2 and b"static scratch" in L.tops_last_error()


def test_ptr_keeps_its_tensor_alive():
    """A pointer taken from a temporary (ptr(f(x)) inside a call's argument list) holds the
    tensor until the pointer itself is dropped, so a later argument's allocation cannot take
    the block before the kernel that reads it is queued."""
    import gc
    import weakref
    import torch
    from tops import _native as N
    t = torch.arange(6, dtype=torch.float32) * 2
    w = weakref.ref(t)
    p = N.ptr(t)
    del t
    gc.collect()
    assert w() is not None and int(p) == w().data_ptr()
    assert ctypes.c_void_p.from_param(p) is not None     # still a plain address for ctypes
    del p
    gc.collect()
    assert w() is None
    assert N.ptr(None) is None


def test_decode_routing_reads_no_device_boundaries():
    """The decode route decides on host boundaries exactly and on device boundaries by the mean
    length, without reading them back (a meta tensor has no data: reading it would raise)."""
    import torch
    from tops.ops.gla.fused_recurrent import decode_sized
    assert decode_sized(4, None) and not decode_sized(5, None)
    assert decode_sized(8, [0, 4, 8]) and not decode_sized(8, [0, 1, 8])
    assert decode_sized(8, torch.tensor([0, 4, 8])) and not decode_sized(8, np.array([0, 1, 8]))
    assert decode_sized(8, torch.empty(3, dtype=torch.int32, device="meta"))       # mean 4
    assert not decode_sized(9, torch.empty(3, dtype=torch.int32, device="meta"))   # mean 4.5
    assert not decode_sized(0, torch.empty(1, dtype=torch.int32, device="meta"))   # no sequence


def test_phase_clock_library_is_separate_and_checks_arguments():
    """The instrumented sweep (phase clocks) is its own library: the regular one does not
    export its entry, and the entry rejects missing buffers and unsupported shapes on the
    host, before any launch."""
    from tops import _native as N
    assert not hasattr(N.lib(), "tops_pipe_phase_clocks")
    path = os.path.join(ROOT, "pallas-kernel_amd", "tops", "_lib", "libtops_pipe_clocks.so")
    if not os.path.exists(path):
        pytest.skip("instrumented library not built (build.py --phase-clocks)")
    f = ctypes.CDLL(path).tops_pipe_phase_clocks
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_void_p] * 8 + [ctypes.c_int] * 6 + [ctypes.c_float, ctypes.c_void_p]
    p = ctypes.c_void_p(8)
    # no clock buffer; a checkpoint buffer without its factors; K over one tile
    assert f(p, p, p, p, p, None, None, None, 1, 64, 1, 64, 64, 0, 1.0, None) != 0
    assert f(p, p, p, p, p, p, None, p, 1, 64, 1, 64, 64, 0, 1.0, None) != 0
    assert f(p, p, p, p, p, None, None, p, 1, 64, 1, 256, 64, 0, 1.0, None) != 0
