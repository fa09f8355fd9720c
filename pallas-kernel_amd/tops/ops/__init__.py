"""Public operator API (mirrors tops/ops/__init__.py:8-16)."""
from .simple_gla import simple_gla  # noqa: F401
