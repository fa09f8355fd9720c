"""naive_recurrent_gla (mirrors tops/ops/gla/naive.py:6-105): the per-token recurrence
h_t = h_{t-1} * exp(gk_t) + k_t^T v_t, o_t = scale * q_t h_t, on the HIP fused-recurrent
kernels (the same equations; the reference runs them as a Python loop in JAX)."""
from __future__ import annotations

from .fused_recurrent import _FusedRecurrentGLA, _check


def naive_recurrent_gla(q, k, v, gk, scale=None, initial_state=None, output_final_state=False,
                        cu_seqlens=None):
    """Returns (o [B,T,H,V] in q.dtype, final state [N,H,K,V] float32 or None)."""
    _check(q, k, v, gk, None, initial_state, cu_seqlens)
    if scale is None:
        scale = q.shape[-1] ** -0.5
    o, ht = _FusedRecurrentGLA.apply(q, k, v, gk, None, initial_state, float(scale),
                                     bool(output_final_state), False, cu_seqlens)
    return o.to(q.dtype), (ht if output_final_state else None)


__all__ = ["naive_recurrent_gla"]
