"""Host-side helpers mirroring tops/utils.py (varlen chunk maps, ceil-div)."""
from __future__ import annotations

import numpy as np
import torch

from . import _native as N

CHUNK = 64  # tile length of every chunked kernel


def cdiv(x: int, y: int) -> int:
    """tops/utils.py:19-26."""
    return (x + y - 1) // y


def _host_cu(cu_seqlens) -> np.ndarray:
    if isinstance(cu_seqlens, torch.Tensor):
        cu_seqlens = cu_seqlens.detach().cpu().numpy()
    return np.ascontiguousarray(np.asarray(cu_seqlens, dtype=np.int32))


def prepare_lens(cu_seqlens) -> np.ndarray:
    """tops/utils.py:63-68."""
    cu = _host_cu(cu_seqlens)
    return cu[1:] - cu[:-1]


def prepare_chunk_indices(cu_seqlens, chunk_size: int) -> np.ndarray:
    """[total_NT, 2] int32 (sequence id, chunk id): tops/utils.py:71-90, built by the
    native host routine tops_prepare_chunk_indices."""
    cu = _host_cu(cu_seqlens)
    n = len(cu) - 1
    cap = int(cu[-1]) // chunk_size + n
    offs = np.empty(n + 1, np.int32)
    idx = np.empty((max(cap, 1), 2), np.int32)
    total = N._fn("tops_prepare_chunk_indices")(cu.ctypes.data, n, chunk_size, offs.ctypes.data,
                                               idx.ctypes.data, cap)
    if total < 0:
        raise ValueError(N.lib().tops_last_error().decode())
    return idx[:total].copy()


class ChunkPlan:
    """Chunk bookkeeping of one call: sequences, global chunk offsets, device maps."""

    def __init__(self, B: int, T: int, cu_seqlens, device, C: int = CHUNK):
        self.C = C
        self.varlen = cu_seqlens is not None
        if self.varlen:
            cu = _host_cu(cu_seqlens)
            self.N = len(cu) - 1
            idx = prepare_chunk_indices(cu, C)
            self.total = idx.shape[0]
            offs = np.zeros(self.N + 1, np.int32)
            np.cumsum(np.bincount(idx[:, 0], minlength=self.N), out=offs[1:])
            self.cu_dev = torch.from_numpy(cu).to(device)
            self.offsets_dev = torch.from_numpy(offs).to(device)
            self.chunk_map_dev = torch.from_numpy(np.ascontiguousarray(idx[:, 0])).to(device)
        else:
            self.N = B
            self.total = B * cdiv(T, C)
            self.cu_dev = self.offsets_dev = self.chunk_map_dev = None
