"""tops.ops.simple_gla on MI355X (mirrors tops/ops/simple_gla/__init__.py:1-239)."""
from __future__ import annotations

import enum

from .chunk import (chunk_simple_gla, chunk_simple_gla_bwd, chunk_simple_gla_fwd,
                    chunk_simple_gla_fwd_varlen)
from .fused_chunk import fused_chunk_simple_gla, fused_chunk_simple_gla_bwd, fused_chunk_simple_gla_fwd
from .fused_recurrent import fused_recurrent_simple_gla


def simple_gla(q, k, v, *args, g=None, g_gamma=None, scale=None, initial_state=None,
               output_final_state=False, chunk_size=64, reverse=False, cu_seqlens_cpu=None,
               mode="chunk", **kwargs):
    """Unified simple-GLA entry point (tops/ops/simple_gla/__init__.py:15-158), with the
    reference's argument checks and ValueErrors per mode."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    assert tuple(k.shape) == (B, T, H, K), f"k shape {tuple(k.shape)} != {(B, T, H, K)}"
    assert tuple(v.shape) == (B, T, H, V), f"v shape {tuple(v.shape)} != {(B, T, H, V)}"
    assert g is None or tuple(g.shape) == (B, T, H), f"g shape {tuple(g.shape)} != {(B, T, H)}"
    assert g_gamma is None or tuple(g_gamma.shape) == (H,), f"g_gamma shape must be ({H},)"
    if mode in ("chunk", "fused_chunk"):
        if g is not None:
            raise ValueError(f"mode={mode!r} does not support per-token gate `g`; "
                             "use 'fused_recurrent' or 'naive' instead")
        if reverse:
            raise ValueError(f"mode={mode!r} does not support `reverse`")
        if cu_seqlens_cpu is not None:
            raise ValueError(f"mode={mode!r} does not support `cu_seqlens`")
        assert g_gamma is not None, f"mode={mode!r} requires g_gamma"
        fn = chunk_simple_gla if mode == "chunk" else fused_chunk_simple_gla
        return fn(q, k, v, g_gamma, initial_state=initial_state, scale=scale,
                  output_final_state=output_final_state, chunk_size=chunk_size)
    if mode == "fused_recurrent":
        return fused_recurrent_simple_gla(q, k, v, g=g, g_gamma=g_gamma, scale=scale,
                                          initial_state=initial_state,
                                          output_final_state=output_final_state, reverse=reverse,
                                          cu_seqlens=cu_seqlens_cpu)
    if mode == "naive":
        return simple_gla_naive(q, k, v, g=g, g_gamma=g_gamma, scale=scale,
                                initial_state=initial_state, output_final_state=output_final_state,
                                chunk_size=chunk_size, cu_seqlens_cpu=cu_seqlens_cpu)
    raise ValueError(f"Unknown mode {mode!r}; expected one of "
                     "'chunk', 'fused_chunk', 'fused_recurrent', 'naive'")


__all__ = [
    "simple_gla",
    "chunk_simple_gla",
    "chunk_simple_gla_fwd",
    "chunk_simple_gla_fwd_varlen",
    "chunk_simple_gla_bwd",
    "fused_chunk_simple_gla",
    "fused_chunk_simple_gla_fwd",
    "fused_chunk_simple_gla_bwd",
    "fused_recurrent_simple_gla",
    "simple_gla_naive",
    "SimpleGLAKernelMode",
    "simple_gla_fwd",
    "simple_gla_bwd",
]


def simple_gla_naive(q, k, v, g=None, g_gamma=None, scale=None, initial_state=None,
                     output_final_state=False, chunk_size=64, cu_seqlens_cpu=None):
    """The reference's pure-JAX testing form (tops/ops/simple_gla/naive.py:5-100); here the
    per-token recurrence on the HIP fused_recurrent kernels (same equations).  Returns
    (o [B,T,H,V] float32, final state float32 or None) as the reference does."""
    q, k, v = (x.float() for x in (q, k, v))      # the reference computes in fp32 throughout
    o, ht = fused_recurrent_simple_gla(q, k, v, g=g, g_gamma=g_gamma, scale=scale,
                                       initial_state=initial_state,
                                       output_final_state=output_final_state,
                                       cu_seqlens=cu_seqlens_cpu)
    return o, ht


class SimpleGLAKernelMode(enum.Enum):
    """Kernel family for simple_gla_fwd / simple_gla_bwd (tops/ops/simple_gla/__init__.py:160-164);
    both run the same HIP chunk sweep here."""
    CHUNK = "chunk"
    FUSED_CHUNK = "fused_chunk"


def simple_gla_fwd(q, k, v, *, g=None, g_gamma=None, scale=None, h0=None, use_ht=False,
                   cu_seqlens_cpu=None, cu_seqlens_dev=None, chunk_size=64,
                   mode=SimpleGLAKernelMode.FUSED_CHUNK):
    """tops/ops/simple_gla/__init__.py:167-201: forward by kernel mode (a device cu_seqlens
    selects the varlen forward).  Returns (o, ht)."""
    if mode not in (SimpleGLAKernelMode.CHUNK, SimpleGLAKernelMode.FUSED_CHUNK) \
            and cu_seqlens_dev is None:
        raise Exception(f"mode {mode} not support")
    if cu_seqlens_dev is not None:
        fn = chunk_simple_gla_fwd_varlen
    elif mode == SimpleGLAKernelMode.CHUNK:
        fn = chunk_simple_gla_fwd
    else:
        fn = fused_chunk_simple_gla_fwd
    return fn(q, k, v, g=g, g_gamma=g_gamma, scale=scale, h0=h0, use_ht=use_ht,
              cu_seqlens_cpu=cu_seqlens_cpu, cu_seqlens_dev=cu_seqlens_dev,
              chunk_size=chunk_size)


def simple_gla_bwd(q, k, v, do, *, g=None, g_gamma=None, scale=None, h0=None, dht=None,
                   cu_seqlens_cpu=None, cu_seqlens_dev=None, chunk_size=64,
                   mode=SimpleGLAKernelMode.FUSED_CHUNK):
    """tops/ops/simple_gla/__init__.py:204-239: backward by kernel mode.  Returns
    (dq, dk, dv, dh0)."""
    if mode == SimpleGLAKernelMode.CHUNK:
        fn = chunk_simple_gla_bwd
    elif mode == SimpleGLAKernelMode.FUSED_CHUNK:
        fn = fused_chunk_simple_gla_bwd
    else:
        raise Exception(f"mode {mode} not support")
    return fn(q, k, v, do, g=g, g_gamma=g_gamma, scale=scale, h0=h0, dht=dht,
              cu_seqlens_cpu=cu_seqlens_cpu, cu_seqlens_dev=cu_seqlens_dev,
              chunk_size=chunk_size)
