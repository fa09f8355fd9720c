"""RMSNorm on MI355X (tops/modules/layernorm.py:6-35), and the functional RMSNorm with an
optional SiLU gate shared with FusedRMSNormGated.

y = x * rsqrt(mean(x^2) + eps) * weight [* silu(g)], in float32, returned in x's dtype.
Forward and backward run on tops_rmsnorm_gated_fwd / _bwd (one wave64 per row, D <= 2048);
the weight gradient is reduced deterministically.
"""
from __future__ import annotations

import torch
from torch import nn

from .. import _native as N


def _kin(t):
    if t is None:
        return None
    if t.dtype not in (torch.float32, torch.bfloat16):
        t = t.to(torch.float32)
    return t.contiguous()


class _RMSNormGated(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, g, weight, eps):
        N.require_cuda(x, g, weight)
        D = x.shape[-1]
        if g is not None and tuple(g.shape) != tuple(x.shape):
            raise AssertionError(f"g shape {tuple(g.shape)} != x shape {tuple(x.shape)}")
        if weight is not None and tuple(weight.shape) != (D,):
            raise AssertionError(f"weight shape {tuple(weight.shape)} != ({D},)")
        xk, gk = _kin(x), _kin(g)
        w32 = None if weight is None else weight.detach().to(torch.float32).contiguous()
        rows = x.numel() // D if D else 0
        y = torch.empty_like(xk)
        N.call("tops_rmsnorm_gated_fwd", N.ptr(xk), N.dtype_code(xk.dtype), N.ptr(gk),
               0 if gk is None else N.dtype_code(gk.dtype), N.ptr(w32), N.ptr(y), rows, D,
               float(eps), N.stream())
        ctx.save_for_backward(xk, gk, w32)
        ctx.eps = float(eps)
        ctx.dtypes = (x.dtype, None if g is None else g.dtype,
                      None if weight is None else weight.dtype)
        return y.to(x.dtype)

    @staticmethod
    def backward(ctx, dy):
        xk, gk, w32 = ctx.saved_tensors
        D = xk.shape[-1]
        rows = xk.numel() // D if D else 0
        dy = dy.to(xk.dtype).contiguous()
        dx = torch.empty_like(xk)
        dg = None if gk is None else torch.empty_like(gk)
        dw = ws = None
        n_ws = 0
        if w32 is not None:
            dw = torch.empty(D, device=xk.device, dtype=torch.float32)
            n_ws = int(N.lib().tops_rmsnorm_gated_bwd_workspace(rows, D))
            ws = torch.empty(max(n_ws, 1), device=xk.device, dtype=torch.float32)
        N.call("tops_rmsnorm_gated_bwd", N.ptr(xk), N.dtype_code(xk.dtype), N.ptr(gk),
               0 if gk is None else N.dtype_code(gk.dtype), N.ptr(w32), N.ptr(dy), N.ptr(dx),
               N.ptr(dg), N.ptr(dw), N.ptr(ws), n_ws, rows, D, ctx.eps, N.stream())
        x_dt, g_dt, w_dt = ctx.dtypes
        return (dx.to(x_dt), None if dg is None else dg.to(g_dt),
                None if dw is None else dw.to(w_dt), None)


def rms_norm_gated(x: torch.Tensor, g: torch.Tensor | None = None,
                   weight: torch.Tensor | None = None, eps: float = 1e-5) -> torch.Tensor:
    """x * rsqrt(mean(x^2, -1) + eps) * weight * silu(g) (g / weight optional), in x's dtype;
    differentiable in x, g and weight."""
    return _RMSNormGated.apply(x, g, weight, eps)


class RMSNorm(nn.Module):
    """Root mean square layer normalisation: x * rsqrt(mean(x^2) + eps) * weight."""

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

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return rms_norm_gated(x, None, self.weight, self.eps)
