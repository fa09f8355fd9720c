"""fused_recurrent_kda on MI355X (tops/ops/kda/fused_recurrent.py:18-105).

The reference runs the per-token delta rule as a lax.scan.  Here the same recurrence
runs through the chunked KDA kernels (the chunk form is an exact rewrite of the per-token
recurrence, equal up to fp32 rounding), which keeps the state on chip across a chunk
instead of re-reading it per token.  Differentiable through `chunk_kda`.
"""
from __future__ import annotations

import torch

from .chunk import chunk_kda


def fused_recurrent_kda(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor,
                        beta: torch.Tensor, scale: float | None = None,
                        initial_state: torch.Tensor | None = None,
                        output_final_state: bool = False):
    """q, k [B,T,H,K]; v [B,T,H,V]; g [B,T,H,K] natural-log gates; beta [B,T,H];
    initial_state [B,H,K,V].  Returns (o in q.dtype, final_state or None)."""
    o, ht = chunk_kda(q, k, v, g, beta, scale=scale, initial_state=initial_state,
                      output_final_state=output_final_state)
    return o.to(q.dtype), ht
