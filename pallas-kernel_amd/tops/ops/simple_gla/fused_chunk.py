"""fused_chunk_simple_gla on MI355X (tops/ops/simple_gla/fused_chunk.py:28-555).

The reference's fused-chunk variant keeps the state on-chip across chunks; the
tops-hip chunk sweep already does that for every chunk op, so the fused-chunk
entry points run the same kernels as chunk_simple_gla."""
from __future__ import annotations

from .chunk import chunk_simple_gla, chunk_simple_gla_fwd, chunk_simple_gla_bwd


def fused_chunk_simple_gla(q, k, v, g_gamma, initial_state=None, scale=None,
                           output_final_state=False, chunk_size=64):
    """tops/ops/simple_gla/fused_chunk.py:503-555 (custom_vjp; g_gamma only)."""
    return chunk_simple_gla(q, k, v, g_gamma, initial_state=initial_state, scale=scale,
                            output_final_state=output_final_state, chunk_size=chunk_size)


def fused_chunk_simple_gla_fwd(q, k, v, g_gamma=None, scale=None, initial_state=None,
                               output_final_state=False, chunk_size=64, *, g=None, h0=None,
                               use_ht=None, cu_seqlens_cpu=None, cu_seqlens_dev=None,
                               interpret=None):
    """tops/ops/simple_gla/fused_chunk.py:28-60 forward: returns (o, ht).  Accepts the
    accelerator keywords (g, h0, use_ht, cu_seqlens_cpu / _dev) as chunk_simple_gla_fwd."""
    return chunk_simple_gla_fwd(q, k, v, g=g, g_gamma=g_gamma, scale=scale,
                                initial_state=initial_state, output_final_state=output_final_state,
                                chunk_size=chunk_size, h0=h0, use_ht=use_ht,
                                cu_seqlens_cpu=cu_seqlens_cpu, cu_seqlens_dev=cu_seqlens_dev,
                                interpret=interpret)


def fused_chunk_simple_gla_bwd(q, k, v, do, g_gamma=None, scale=None, h0=None, dht=None,
                               chunk_size=64, *, g=None, cu_seqlens_cpu=None,
                               cu_seqlens_dev=None, interpret=None):
    """tops/ops/simple_gla/fused_chunk.py:307-402 backward: returns (dq, dk, dv, dh0)."""
    assert g is None, "per-element gating not supported in fused_chunk_simple_gla_bwd"
    return chunk_simple_gla_bwd(q, k, v, do, g_gamma=g_gamma, scale=scale, h0=h0, dht=dht,
                                chunk_size=chunk_size, cu_seqlens_cpu=cu_seqlens_cpu,
                                cu_seqlens_dev=cu_seqlens_dev, interpret=interpret)
