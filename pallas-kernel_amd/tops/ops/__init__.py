"""Public operator API (mirrors tops/ops/__init__.py)."""
