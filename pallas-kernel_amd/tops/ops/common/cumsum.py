"""Chunk-local gate cumsum on MI355X (mirrors tops/ops/common/cumsum.py:472-540 and
tops/ops/gla/chunk.py:110-198).

One HIP kernel (tops_chunk_local_cumsum) serves every layout and mode the reference
dispatches to separate back ends (jnp.cumsum, triangular matmul, Hillis-Steele Pallas
kernel): one thread per (chunk, head, column) carries the running sum down its chunk.
"""
from __future__ import annotations

import torch

from ... import _native as N
from ...utils import ChunkPlan
from ._stage import require

_OUT_KERNEL = (torch.float32, torch.bfloat16)


def chunk_local_cumsum_vector(g: torch.Tensor, chunk_size: int, reverse: bool = False,
                              scale: float | None = None, cu_seqlens=None,
                              head_first: bool = False,
                              output_dtype: torch.dtype | None = torch.float32,
                              chunk_indices=None) -> torch.Tensor:
    """Inclusive prefix sum (suffix sum when ``reverse``) of ``g`` inside each chunk of
    ``chunk_size`` tokens, then ``* scale`` when given.

    g: [B, T, H, S] (or [B, H, T, S] with ``head_first``); a 3-D [B, T, H] scalar gate is
    treated as S = 1.  ``cu_seqlens`` ([N+1], B == 1): chunks restart at every sequence
    start and a sequence's last chunk may be short.  ``chunk_indices`` is accepted for
    signature compatibility (the chunk map is derived from ``cu_seqlens``).  Returns the
    same shape in ``output_dtype`` (``None``: g's dtype).
    """
    del chunk_indices
    C = int(chunk_size)
    require(C > 0 and C & (C - 1) == 0, "chunk_size must be power of 2")
    require(g.ndim in (3, 4), f"g must be 4-D (or a 3-D scalar gate), got {g.ndim}-D")
    N.require_cuda(g)
    g4 = g if g.ndim == 4 else g.unsqueeze(-1)
    if head_first:
        B, H, T, S = g4.shape
    else:
        B, T, H, S = g4.shape
    out_dt = output_dtype or g.dtype
    kin = g4 if g4.dtype in _OUT_KERNEL else g4.float()
    kin = kin.contiguous()
    kout_dt = out_dt if out_dt in _OUT_KERNEL else torch.float32
    out = torch.empty(g4.shape, device=g.device, dtype=kout_dt)
    if g.numel() == 0:
        return out.to(out_dt).reshape(g.shape)
    if cu_seqlens is not None:
        require(B == 1, f"cu_seqlens requires B=1, got {B}")
    plan = ChunkPlan.get(B, T, cu_seqlens, g.device, C)
    with torch.no_grad():
        N.call("tops_chunk_local_cumsum", N.ptr(kin), N.dtype_code(kin.dtype), N.ptr(out),
               N.dtype_code(kout_dt), N.ptr(plan.cu_dev), N.ptr(plan.offsets_dev),
               N.ptr(plan.chunk_map_dev), plan.total, B, T, H, S, C, int(bool(head_first)),
               int(bool(reverse)), 1.0 if scale is None else float(scale), N.stream())
    if kout_dt != out_dt:
        out = out.to(out_dt)
    return out.reshape(g.shape)


def chunk_local_cumsum(g: torch.Tensor, chunk_size: int, reverse: bool = False,
                       cu_seqlens=None, chunk_indices=None, scale: float | None = None,
                       head_first: bool = False, output_dtype: torch.dtype | None = torch.float32):
    """tops/ops/common/chunk_o.py:22-112 form ([B,T,H] or [B,T,H,K] gates, float32 out)."""
    return chunk_local_cumsum_vector(g, chunk_size, reverse=reverse, scale=scale,
                                     cu_seqlens=cu_seqlens, head_first=head_first,
                                     output_dtype=output_dtype, chunk_indices=chunk_indices)


__all__ = ["chunk_local_cumsum_vector", "chunk_local_cumsum"]
