"""fused_chunk_fwd on MI355X (mirrors tops/ops/common/fused_chunk.py:286-365): the simple-GLA
forward from chunk-local cumsummed scalar gates, as the state recurrence followed by the
output stage (the reference fuses the two into one kernel; chunk_simple_gla's HIP sweep is
the fused form here)."""
from __future__ import annotations

import torch

from .chunk_h import _recurrence
from .chunk_o import chunk_fwd_o


def fused_chunk_fwd(q, k, v, *, g=None, g_gamma=None, h0=None, scale=None, use_ht: bool = False,
                    chunk_size: int = 64, interpret=None):
    """g [B,T,H] chunk-local cumsum of the scalar gate, g_gamma [H], h0 [B,H,K,V].
    Returns (o in v.dtype, ht [B,H,K,V] fp32 or None)."""
    del interpret
    K = q.shape[-1]
    if scale is None:
        scale = K ** -0.5
    C = int(chunk_size)
    h, ht = _recurrence(k, v, g, g_gamma, None, h0, None, C, False, 1.0, 1, torch.float32,
                        bool(use_ht))
    o = chunk_fwd_o(q, k, v, h, g=g, g_gamma=g_gamma, scale=scale, chunk_size=C)
    return o, (ht if use_ht else None)


__all__ = ["fused_chunk_fwd"]
