"""Shared chunk stages (mirrors tops/ops/common/): gate cumsum and the state recurrence."""
from .cumsum import chunk_local_cumsum, chunk_local_cumsum_vector
from .chunk_h import chunk_bwd_dh_kernel, chunk_bwd_dh_ref, chunk_fwd_h_kernel, chunk_fwd_h_ref

__all__ = [
    "chunk_local_cumsum",
    "chunk_local_cumsum_vector",
    "chunk_fwd_h_ref",
    "chunk_fwd_h_kernel",
    "chunk_bwd_dh_ref",
    "chunk_bwd_dh_kernel",
]
