"""Public operator API (mirrors tops/ops/__init__.py:8-16)."""
from .kda import chunk_kda, chunk_kda_fwd, fused_recurrent_kda  # noqa: F401
from .simple_gla import simple_gla  # noqa: F401
