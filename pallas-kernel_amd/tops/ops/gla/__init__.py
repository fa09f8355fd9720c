"""tops.ops.gla on MI355X (mirrors tops/ops/gla/__init__.py:1-34)."""
from .naive import naive_recurrent_gla
from .chunk import chunk_gla, chunk_gla_fwd, chunk_gla_bwd, chunk_gla_bwd_with_pl
from .stages import (chunk_local_cumsum, chunk_fwd_h, chunk_gla_fwd_intra_gk, chunk_gla_fwd_o_gk,
                     chunk_gla_bwd_dA_ref, chunk_gla_bwd_dv_ref, chunk_gla_bwd_dqk_intra_ref,
                     chunk_gla_bwd_dqkg_ref)
from .fused_chunk import fused_chunk_gla
from .fused_recurrent import (fused_recurrent_gla, fused_recurrent_gla_fwd, fused_recurrent_gla_bwd,
                              fused_recurrent_gla_norm_gate, fused_recurrent_gla_conv_norm_gate)

__all__ = [
    "naive_recurrent_gla",
    "chunk_gla",
    "chunk_local_cumsum",
    "chunk_fwd_h",
    "chunk_gla_fwd_intra_gk",
    "chunk_gla_fwd_o_gk",
    "chunk_gla_fwd",
    "chunk_gla_bwd_dA_ref",
    "chunk_gla_bwd_dv_ref",
    "chunk_gla_bwd_dqk_intra_ref",
    "chunk_gla_bwd_dqkg_ref",
    "chunk_gla_bwd",
    "chunk_gla_bwd_with_pl",
    "fused_chunk_gla",
    "fused_recurrent_gla",
    "fused_recurrent_gla_fwd",
    "fused_recurrent_gla_bwd",
    "fused_recurrent_gla_norm_gate",
    "fused_recurrent_gla_conv_norm_gate",
]
