"""Row L2 normalisation of q / k for KDA on MI355X.

y = x / sqrt(sum x^2 + 1e-6) over the last axis, in float32: the `_l2_normalize_last_dim`
that fused_recurrent_kda applies with use_qk_l2norm_in_kernel=True
(tops/cpu/ops/kda/fused_recurrent.py:14-18).  One wave64 per row on the HIP kernels
tops_l2norm_fwd / tops_l2norm_bwd; differentiable (dx = r (dy - y (y . dy)) with
r = 1 / sqrt(sum x^2 + 1e-6), in the input dtype).
"""
from __future__ import annotations

import torch

from ... import _native as N


def _kernel_input(x: torch.Tensor) -> torch.Tensor:
    if x.dtype not in (torch.float32, torch.bfloat16):
        x = x.to(torch.float32)
    return x.contiguous()


class _L2Norm(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x):
        N.require_cuda(x)
        xk = _kernel_input(x)
        D = x.shape[-1]
        rows = x.numel() // D if D else 0
        y = torch.empty(x.shape, device=x.device, dtype=torch.float32)
        N.call("tops_l2norm_fwd", N.ptr(xk), N.dtype_code(xk.dtype), N.ptr(y), rows, D,
               N.stream())
        ctx.save_for_backward(xk)
        ctx.in_dtype = x.dtype
        return y

    @staticmethod
    def backward(ctx, dy):
        (xk,) = ctx.saved_tensors
        D = xk.shape[-1]
        rows = xk.numel() // D if D else 0
        dy = dy.contiguous().to(torch.float32)
        dx = torch.empty_like(xk)
        N.call("tops_l2norm_bwd", N.ptr(xk), N.dtype_code(xk.dtype), N.ptr(dy), N.ptr(dx),
               rows, D, N.stream())
        return dx.to(ctx.in_dtype)


def l2norm(x: torch.Tensor) -> torch.Tensor:
    """float32 x / sqrt(sum(x^2, -1) + 1e-6); D = x.shape[-1] <= 256."""
    return _L2Norm.apply(x)


__all__ = ["l2norm"]
