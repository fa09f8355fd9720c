"""tops.ops.kda on MI355X (mirrors tops/ops/kda/__init__.py, plus the gate and recurrent
entry points of tops/cpu/ops/kda/__init__.py)."""
from .chunk import chunk_kda, chunk_kda_fwd
from .chunk_intra import chunk_kda_bwd_intra, kda_intra_chunk_fwd
from .fused_recurrent import fused_recurrent_kda, fused_recurrent_kda_bwd, fused_recurrent_kda_fwd
from .gate import (fused_kda_gate, kda_gate_bwd, kda_gate_chunk_cumsum, kda_gate_fwd,
                   naive_kda_gate, naive_kda_lowerbound_gate)
from .l2norm import l2norm

__all__ = [
    "chunk_kda",
    "chunk_kda_fwd",
    "fused_recurrent_kda",
    "chunk_kda_bwd_intra",
    "kda_intra_chunk_fwd",
    "fused_recurrent_kda_fwd",
    "fused_recurrent_kda_bwd",
    "fused_kda_gate",
    "kda_gate_fwd",
    "kda_gate_bwd",
    "kda_gate_chunk_cumsum",
    "naive_kda_gate",
    "naive_kda_lowerbound_gate",
    "l2norm",
]
