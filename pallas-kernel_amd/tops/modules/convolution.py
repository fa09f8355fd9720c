"""ShortConvolution on MI355X (tops/modules/convolution.py:6-173): causal depthwise
convolution over time with optional SiLU, packed varlen sequences, the final-state window
and single-step decoding with a cache.

    y[t, d] = act(sum_j x[t - W + 1 + j, d] * weight[d, 0, j] + bias[d])

with W - 1 zeros of left padding per sequence.  The parameters follow PyTorch's depthwise
Conv1d (weight [D, 1, W], bias [D]); caches and final states are [N, D, W].  As in the
reference, a prefill call does not read `cache` (it pads with zeros), its final state is
the last W inputs of each sequence, and a call whose B*T equals the number of sequences
is a decode step.  The output dtype is the promotion of x's and the weight's dtypes (fp32
for bf16 inputs with fp32 parameters, as the reference's Conv promotes).
Prefill forward / backward run on tops_short_conv_fwd / _bwd (differentiable in x, weight
and bias, deterministic weight / bias gradients); the decode step on tops_short_conv_step.
"""
from __future__ import annotations

import math

import torch
from torch import nn

from .. import _native as N
from ..utils import _host_cu, _upload

_CU = {}


def _cu_dev(cu_seqlens, device):
    if cu_seqlens is None:
        return None, None
    cu = _host_cu(cu_seqlens)
    key = (cu.tobytes(), str(device))
    t = _CU.get(key)
    if t is None:
        if len(_CU) > 64:
            _CU.clear()
        t = _CU[key] = _upload(cu, device)
    return t, len(cu) - 1


def _act(activation) -> int:
    return 1 if activation in ("silu", "swish") else 0


def _out_dtype(x, weight):
    dt = torch.promote_types(x.dtype, weight.dtype)
    return dt if dt in (torch.float32, torch.bfloat16) else torch.float32


def _kin(t):
    if t.dtype not in (torch.float32, torch.bfloat16):
        t = t.to(torch.float32)
    return t.contiguous()


class _ShortConv(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, bias, act, cu, n, want_state):
        B, T, D = x.shape
        W = weight.shape[-1]
        xk = _kin(x)
        w32 = weight.detach().reshape(D, W).to(torch.float32).contiguous()
        b32 = None if bias is None else bias.detach().to(torch.float32).contiguous()
        ydt = _out_dtype(x, weight)
        y = torch.empty(B, T, D, device=x.device, dtype=ydt)
        fs = torch.empty(n, D, W, device=x.device, dtype=xk.dtype) if want_state else None
        N.call("tops_short_conv_fwd", N.ptr(xk), N.dtype_code(xk.dtype), N.ptr(w32), N.ptr(b32),
               N.ptr(y), N.dtype_code(ydt), N.ptr(fs), N.ptr(cu), B, T, D, W, n, act, N.stream())
        ctx.save_for_backward(xk, w32, b32, cu)
        ctx.meta = (act, n, x.dtype, weight.dtype, None if bias is None else bias.dtype,
                    tuple(weight.shape))
        if fs is not None:
            fs = fs.to(x.dtype)
            ctx.mark_non_differentiable(fs)
        return y, fs

    @staticmethod
    def backward(ctx, dy, _dfs):
        xk, w32, b32, cu = ctx.saved_tensors
        act, n, x_dt, w_dt, b_dt, w_shape = ctx.meta
        B, T, D = xk.shape
        W = w32.shape[1]
        dy = _kin(dy)
        dx = torch.empty_like(xk)
        dw = torch.empty(D, W, device=xk.device, dtype=torch.float32)
        db = None if b32 is None else torch.empty(D, device=xk.device, dtype=torch.float32)
        n_ws = int(N.lib().tops_short_conv_bwd_workspace(B, T, D, W))
        ws = torch.empty(max(n_ws, 1), device=xk.device, dtype=torch.float32)
        N.call("tops_short_conv_bwd", N.ptr(xk), N.dtype_code(xk.dtype), N.ptr(w32), N.ptr(b32),
               N.ptr(dy), N.dtype_code(dy.dtype), N.ptr(dx), N.ptr(dw), N.ptr(db), N.ptr(ws),
               n_ws, N.ptr(cu), B, T, D, W, n, act, N.stream())
        return (dx.to(x_dt), dw.reshape(w_shape).to(w_dt),
                None if db is None else db.to(b_dt), None, None, None, None)


def short_conv(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None,
               activation: str | None = "silu", cu_seqlens=None,
               output_final_state: bool = False):
    """Causal depthwise conv over time: x [B,T,D], weight [D,1,W] (or [D,W]), bias [D].
    Returns (y [B,T,D], final_state [N,D,W] in x's dtype or None)."""
    if x.ndim != 3:
        raise AssertionError(f"x must be [B,T,D], got shape {tuple(x.shape)}")
    B, T, D = x.shape
    if weight.shape[0] != D or weight.numel() % D:
        raise AssertionError(f"weight shape {tuple(weight.shape)} incompatible with D={D}")
    if cu_seqlens is not None and B != 1:
        raise AssertionError("cu_seqlens requires B=1")
    N.require_cuda(x, weight, bias)
    cu, n = _cu_dev(cu_seqlens, x.device)
    if cu is None:
        n = B
    return _ShortConv.apply(x, weight, bias, _act(activation), cu, n, bool(output_final_state))


@torch.no_grad()
def short_conv_step(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None,
                    activation: str | None = "silu", cache: torch.Tensor | None = None,
                    output_final_state: bool = False, cu_seqlens=None):
    """One decode step of ShortConvolution (tops/modules/convolution.py:82-126): x [B,1,D] (or
    [1,N,D] with cu_seqlens), weight [D,1,W] or [D,W], cache [N,D,W].  The cache rolls by one
    token and takes x; y = act(sum_j cache[.., j] w[.., j] + bias), or act(x w[.., W-1] + bias)
    without a cache.  Returns (y shaped like x, the rolled cache or None).  Inference only."""
    D = x.shape[-1]
    W = weight.numel() // D
    n = x.shape[0] if cu_seqlens is None else len(cu_seqlens) - 1
    N.require_cuda(x, cache)
    if output_final_state and cache is None:
        cache = torch.zeros(n, D, W, device=x.device, dtype=torch.float32)
    xs = _kin(x[0] if cu_seqlens is not None else x[:, 0])
    if cache is not None and tuple(cache.shape) != (n, D, W):
        raise AssertionError(f"cache shape {tuple(cache.shape)} != {(n, D, W)}")
    cin = None if cache is None else cache.to(torch.float32).contiguous()
    cout = None if cache is None else torch.empty_like(cin)
    w32 = weight.reshape(D, W).to(torch.float32).contiguous()
    b32 = None if bias is None else bias.to(torch.float32).contiguous()
    ydt = _out_dtype(x, weight)
    y = torch.empty(n, D, device=x.device, dtype=ydt)
    N.call("tops_short_conv_step", N.ptr(xs), N.dtype_code(xs.dtype), N.ptr(cin), N.ptr(cout),
           N.ptr(w32), N.ptr(b32), N.ptr(y), N.dtype_code(ydt), n, D, W, _act(activation),
           N.stream())
    return y.reshape(x.shape), None if cout is None else cout.to(cache.dtype)


class ShortConvolution(nn.Module):
    """Causal depthwise 1D convolution (groups = hidden_size, W - 1 left padding), optional
    SiLU activation."""

    def __init__(self, hidden_size: int, kernel_size: int, bias: bool = False,
                 activation: str | None = "silu", *, rngs=None, device=None, dtype=None):
        super().__init__()
        self.hidden_size = hidden_size
        self.kernel_size = kernel_size
        self.activation = activation
        f = dict(device=device, dtype=dtype or torch.float32)
        self.weight = nn.Parameter(torch.empty(hidden_size, 1, kernel_size, **f))
        nn.init.kaiming_uniform_(self.weight, a=math.sqrt(5))   # torch Conv1d's default
        if bias:
            bound = 1.0 / math.sqrt(kernel_size)
            self.bias = nn.Parameter(torch.empty(hidden_size, **f).uniform_(-bound, bound))
        else:
            self.register_parameter("bias", None)

    def forward(self, x: torch.Tensor, cache: torch.Tensor | None = None,
                output_final_state: bool = False, cu_seqlens=None, **kwargs):
        """x [B,T,D]; cache [N,D,W] (read by decode steps only).  Returns (y [B,T,D],
        final_state [N,D,W] or None)."""
        B, T, D = x.shape
        n = B if cu_seqlens is None else len(cu_seqlens) - 1
        if B * T == n:
            return self.step(x, cache, output_final_state, cu_seqlens)
        return short_conv(x, self.weight, self.bias, self.activation, cu_seqlens,
                          output_final_state)

    @torch.no_grad()
    def step(self, x: torch.Tensor, cache: torch.Tensor | None,
             output_final_state: bool = False, cu_seqlens=None):
        """One decode step: x [B,1,D] (or [1,N,D] with cu_seqlens), cache [N,D,W].  Returns
        (y shaped like x, the rolled cache or None).  Inference only (no autograd)."""
        return short_conv_step(x, self.weight.detach(),
                               None if self.bias is None else self.bias.detach(),
                               self.activation, cache, output_final_state, cu_seqlens)
