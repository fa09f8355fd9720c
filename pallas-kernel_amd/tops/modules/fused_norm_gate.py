"""FusedRMSNormGated on MI355X (tops/modules/fused_norm_gate.py:6-37):
output = RMSNorm(x) * silu(g), in float32, returned in x's dtype, on the HIP kernels
tops_rmsnorm_gated_fwd / _bwd (differentiable in x, g and the weight)."""
from __future__ import annotations

import torch
from torch import nn

from .layernorm import rms_norm_gated


class FusedRMSNormGated(nn.Module):
    def __init__(self, hidden_size: int, elementwise_affine: bool = True, eps: float = 1e-5,
                 *, rngs=None, device=None, dtype=None):
        super().__init__()
        self.hidden_size = hidden_size
        self.eps = eps
        self.elementwise_affine = elementwise_affine
        if elementwise_affine:
            self.weight = nn.Parameter(torch.ones(hidden_size, device=device,
                                                  dtype=dtype or torch.float32))
        else:
            self.register_parameter("weight", None)

    def forward(self, x: torch.Tensor, g: torch.Tensor) -> torch.Tensor:
        return rms_norm_gated(x, g, self.weight, self.eps)
