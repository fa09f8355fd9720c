"""tops.ops.kda on MI355X (mirrors tops/ops/kda/__init__.py)."""
from .chunk import chunk_kda, chunk_kda_fwd
from .fused_recurrent import fused_recurrent_kda

__all__ = ["chunk_kda", "chunk_kda_fwd", "fused_recurrent_kda"]
