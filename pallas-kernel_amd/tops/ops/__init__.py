"""Public operator API (mirrors tops/ops/__init__.py:1-16): every public interface is
re-exported here."""
from .kda import chunk_kda, chunk_kda_fwd, fused_recurrent_kda
from .simple_gla import simple_gla

__all__ = [
    "chunk_kda",
    "chunk_kda_fwd",
    "fused_recurrent_kda",
    "simple_gla",
]
