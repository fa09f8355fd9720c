"""Shared chunk stages (mirrors tops/ops/common/): gate cumsum, the state recurrences (GLA
and the KDA delta rule), and the simple-GLA output / backward stages."""
from .cumsum import chunk_local_cumsum, chunk_local_cumsum_vector
from .chunk_h import (chunk_bwd_dh_kernel, chunk_bwd_dh_ref, chunk_fwd_h_kernel,
                      chunk_fwd_h_kernel_varlen, chunk_fwd_h_ref)
from .chunk_o import (chunk_bwd_dqkwg, chunk_bwd_dv, chunk_fwd_o, chunk_fwd_o_ref,
                      chunk_simple_gla_bwd_o_pl)
from .chunk_delta_h import chunk_gated_delta_rule_fwd_h, chunk_gated_delta_rule_fwd_h_ref
from .fused_chunk import fused_chunk_fwd

__all__ = [
    "chunk_local_cumsum",
    "chunk_local_cumsum_vector",
    "chunk_fwd_h_ref",
    "chunk_fwd_h_kernel",
    "chunk_fwd_h_kernel_varlen",
    "chunk_bwd_dh_ref",
    "chunk_bwd_dh_kernel",
    "chunk_fwd_o",
    "chunk_fwd_o_ref",
    "chunk_bwd_dv",
    "chunk_bwd_dqkwg",
    "chunk_simple_gla_bwd_o_pl",
    "fused_chunk_fwd",
    "chunk_gated_delta_rule_fwd_h",
    "chunk_gated_delta_rule_fwd_h_ref",
]
