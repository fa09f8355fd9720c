"""tops.ops.gla on MI355X (mirrors tops/ops/gla/__init__.py:1-34)."""
from .chunk import chunk_gla, chunk_gla_fwd, chunk_gla_bwd
from .fused_chunk import fused_chunk_gla
from .fused_recurrent import fused_recurrent_gla, fused_recurrent_gla_fwd, fused_recurrent_gla_bwd

__all__ = [
    "chunk_gla",
    "chunk_gla_fwd",
    "chunk_gla_bwd",
    "fused_chunk_gla",
    "fused_recurrent_gla",
    "fused_recurrent_gla_fwd",
    "fused_recurrent_gla_bwd",
]
