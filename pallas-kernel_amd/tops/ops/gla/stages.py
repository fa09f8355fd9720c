"""The stage functions of chunked GLA on MI355X (mirrors tops/ops/gla/chunk.py:20-760 and
:1411-1440): the pieces the reference composes into chunk_gla_fwd / chunk_gla_bwd, each
callable on its own with the reference's shapes and meaning.

chunk_gla itself does not go through these (its fused sweeps never write A, h or dh to
HBM); they serve callers that drive the stages one by one.  Each runs one HIP kernel of
csrc/gla_stages.hip in fp32 (v_mfma_f32_16x16x4_f32, the reference's Precision.HIGHEST).
Layout [B, T, H, D] with T a multiple of chunk_size (16, 32, 64 or 128); varlen input
with chunk-aligned cu_seqlens has the same layout, so these stages ignore cu_seqlens as
the reference's do.
"""
from __future__ import annotations

import torch

from ... import _native as N
from ..common._stage import act, chunk_size_ok, f32, finish, promoted, require
from ..common.chunk_h import _recurrence
from ..common.cumsum import chunk_local_cumsum_vector


def _dims(x, C):
    B, T, H, D = x.shape
    chunk_size_ok(C)
    require(T % C == 0, f"T ({T}) must be a multiple of chunk_size ({C})")
    return B, T, H, D


def chunk_local_cumsum(g, chunk_size: int, reverse: bool = False, scale: float | None = None,
                       cu_seqlens=None, head_first: bool = False,
                       output_dtype: torch.dtype | None = torch.float32, chunk_indices=None):
    """tops/ops/gla/chunk.py:110-198 (exported as tops.ops.gla.chunk_local_cumsum)."""
    return chunk_local_cumsum_vector(g, chunk_size, reverse=reverse, scale=scale,
                                     cu_seqlens=cu_seqlens, head_first=head_first,
                                     output_dtype=output_dtype, chunk_indices=chunk_indices)


def chunk_fwd_h(k, v, gk=None, h0=None, output_final_state: bool = False, cu_seqlens_cpu=None,
                chunk_size: int = 64):
    """tops/ops/gla/chunk.py:206-292: h [B, NT, H, K, V] in k.dtype (the state before each
    chunk; gk is the chunk-local gate cumsum) and ht [N, H, K, V] float32, which is zeros
    unless ``output_final_state`` (the reference returns its zero-initialised buffer)."""
    h, ht = _recurrence(k, v, None, None, gk, h0, cu_seqlens_cpu, int(chunk_size), False, 1.0,
                        1, k.dtype, True)
    if not output_final_state:
        ht = torch.zeros_like(ht)
    return h, ht


def chunk_gla_fwd_intra_gk(q, k, g, scale: float, chunk_size: int = 64):
    """A [B, T, H, C] float32: A[i, j] = scale * sum_c q_ic k_jc exp(g_ic - g_jc) within each
    chunk, full square (tops/ops/gla/chunk.py:390-438; the consumer masks it)."""
    C = int(chunk_size)
    B, T, H, K = _dims(q, C)
    (qk, kk), code = act(q, k)
    A = torch.empty((B, T, H, C), device=q.device, dtype=torch.float32)
    N.call("tops_gla_stage_attn", N.ptr(qk), N.ptr(kk), code, N.ptr(f32(g)), N.ptr(A),
           B, T, H, K, C, float(scale), N.stream())
    return A


def chunk_gla_fwd_intra_gk_ref(q, k, g, scale: float, cu_seqlens_dev=None, chunk_size: int = 64):
    """tops/ops/gla/chunk.py:300-343 (same result as chunk_gla_fwd_intra_gk)."""
    del cu_seqlens_dev
    return chunk_gla_fwd_intra_gk(q, k, g, scale, chunk_size)


def chunk_gla_fwd_o_gk(q, v, g, A, h, scale: float, cu_seqlens=None, chunk_indices=None,
                       chunk_size: int = 64, use_exp2: bool = False):
    """o [B, T, H, V] in v.dtype: scale * (q exp(g)) h_c + tril(A) v per chunk
    (tops/ops/gla/chunk.py:1279-1440; exp2 with ``use_exp2``)."""
    del cu_seqlens, chunk_indices
    C = int(chunk_size)
    B, T, H, K = _dims(q, C)
    V = v.shape[-1]
    require(tuple(A.shape) == (B, T, H, C), f"A must be {(B, T, H, C)}")
    require(tuple(h.shape) == (B, T // C, H, K, V), f"h must be {(B, T // C, H, K, V)}")
    (qk, vk), code = act(q, v)
    o = torch.empty((B, T, H, V), device=q.device, dtype=vk.dtype)
    N.call("tops_gla_stage_o", N.ptr(qk), N.ptr(vk), code, N.ptr(f32(g)), N.ptr(f32(A)),
           N.ptr(f32(h)), N.ptr(o), B, T, H, K, V, C, float(scale), int(bool(use_exp2)),
           N.stream())
    return finish(o, v.dtype)


def chunk_gla_fwd_o_gk_ref(q, v, gk, A, h, scale: float, cu_seqlens_cpu=None,
                           chunk_size: int = 64):
    """tops/ops/gla/chunk.py:446-501 (o in the promoted dtype of the inputs)."""
    o = chunk_gla_fwd_o_gk(q, v, gk, A, h, scale, chunk_size=chunk_size)
    return finish(o, promoted(q, v, gk, A, h))


def chunk_gla_bwd_dA_ref(v, do, scale: float, cu_seqlens_cpu=None, chunk_size: int = 64):
    """dA [B, T, H, C] = scale * tril(do v^T) per chunk, in the promoted dtype of v and do
    (tops/ops/gla/chunk.py:509-549)."""
    del cu_seqlens_cpu
    C = int(chunk_size)
    B, T, H, V = _dims(v, C)
    (vk, dok), code = act(v, do)
    dt = vk.dtype
    dA = torch.empty((B, T, H, C), device=v.device, dtype=dt)
    N.call("tops_gla_stage_dattn", N.ptr(vk), N.ptr(dok), code, N.ptr(dA), N.dtype_code(dt),
           B, T, H, V, C, float(scale), N.stream())
    return finish(dA, promoted(v, do))


def chunk_gla_bwd_dv_ref(k, g_cumsum, A, do, dh, cu_seqlens_cpu=None, chunk_size: int = 64):
    """dv [B, T, H, V] = tril(A)^T do + (k exp(g_last - g)) dh per chunk
    (tops/ops/gla/chunk.py:552-605)."""
    del cu_seqlens_cpu
    C = int(chunk_size)
    B, T, H, K = _dims(k, C)
    V = do.shape[-1]
    require(tuple(dh.shape) == (B, T // C, H, K, V), f"dh must be {(B, T // C, H, K, V)}")
    (kk, dok), code = act(k, do)
    dv = torch.empty((B, T, H, V), device=k.device, dtype=torch.float32)
    N.call("tops_gla_stage_dv", N.ptr(kk), N.ptr(dok), code, N.ptr(f32(g_cumsum)),
           N.ptr(f32(A)), N.ptr(f32(dh)), N.ptr(dv), B, T, H, K, V, C, N.stream())
    return finish(dv, promoted(k, g_cumsum, A, do, dh))


def chunk_gla_bwd_dqk_intra_ref(q, k, g_cumsum, dA, cu_seqlens_cpu=None, chunk_size: int = 64):
    """Intra-chunk (dq, dk) from dA, used as given (tops/ops/gla/chunk.py:608-662)."""
    del cu_seqlens_cpu
    C = int(chunk_size)
    B, T, H, K = _dims(q, C)
    require(tuple(dA.shape) == (B, T, H, C), f"dA must be {(B, T, H, C)}")
    (qk, kk), code = act(q, k)
    dq = torch.empty((B, T, H, K), device=q.device, dtype=torch.float32)
    dk = torch.empty_like(dq)
    N.call("tops_gla_stage_dqk_intra", N.ptr(qk), N.ptr(kk), code, N.ptr(f32(g_cumsum)),
           N.ptr(f32(dA)), N.ptr(dq), N.ptr(dk), B, T, H, K, C, N.stream())
    dt = promoted(q, k, g_cumsum, dA)
    return finish(dq, dt), finish(dk, dt)


def chunk_gla_bwd_dqkg_ref(q, k, v, h, g_cumsum, do, dh, dq, dk, scale: float,
                           cu_seqlens_cpu=None, chunk_size: int = 64):
    """Inter-chunk dq / dk added to the intra parts, and the gate gradient dg
    (tops/ops/gla/chunk.py:665-760).  Returns (dq, dk, dg)."""
    del cu_seqlens_cpu
    C = int(chunk_size)
    B, T, H, K = _dims(q, C)
    V = v.shape[-1]
    for name, t in (("h", h), ("dh", dh)):
        require(tuple(t.shape) == (B, T // C, H, K, V), f"{name} must be {(B, T // C, H, K, V)}")
    (qk, kk, vk, dok), code = act(q, k, v, do)
    dq_o = torch.empty((B, T, H, K), device=q.device, dtype=torch.float32)
    dk_o = torch.empty_like(dq_o)
    dg = torch.empty_like(dq_o)
    N.call("tops_gla_stage_dqkg", N.ptr(qk), N.ptr(kk), N.ptr(vk), N.ptr(dok), code,
           N.ptr(f32(g_cumsum)), N.ptr(f32(h)), N.ptr(f32(dh)), N.ptr(f32(dq)), N.ptr(f32(dk)),
           N.ptr(dq_o), N.ptr(dk_o), N.ptr(dg), B, T, H, K, V, C, float(scale), N.stream())
    dt = promoted(q, k, v, h, g_cumsum, do, dh, dq, dk)
    return finish(dq_o, dt), finish(dk_o, dt), finish(dg, dt)


__all__ = [
    "chunk_local_cumsum",
    "chunk_fwd_h",
    "chunk_gla_fwd_intra_gk",
    "chunk_gla_fwd_intra_gk_ref",
    "chunk_gla_fwd_o_gk",
    "chunk_gla_fwd_o_gk_ref",
    "chunk_gla_bwd_dA_ref",
    "chunk_gla_bwd_dv_ref",
    "chunk_gla_bwd_dqk_intra_ref",
    "chunk_gla_bwd_dqkg_ref",
]
