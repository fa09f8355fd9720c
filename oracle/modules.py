"""Float64 oracle for the GLA layer's neighbour modules (test infrastructure only: imported
by tests/ and nothing else).

Restates:
  - tops/modules/layernorm.py:28-35        RMSNorm:  x * rsqrt(mean(x^2) + eps) * w
  - tops/modules/fused_norm_gate.py:28-37  FusedRMSNormGated:  RMSNorm(x) * silu(g)
  - tops/modules/convolution.py:44-80      ShortConvolution._causal_conv1d: depthwise causal
        conv over time with W - 1 zero left padding per sequence (varlen: per segment),
        then SiLU (activation "silu" / "swish") or identity
  - tops/modules/convolution.py:128-173    the final-state window: the last W inputs of each
        sequence, zero left-padded; prefill ignores any cache passed in (as the reference does)
  - tops/modules/convolution.py:82-126     ShortConvolution.step: cache rolled by one with the
        new token appended, y = act(sum(cache * w) + b); without a cache y = act(x w[-1] + b)
The weight is the depthwise kernel as w[d, j] (tap j multiplies x[t - W + 1 + j]); caches
and final states are [N, D, W] (PyTorch channels-first).  The backward functions are the
gradients of these forwards, written out here; tests pin them with torch autograd.
"""

from __future__ import annotations

import numpy as np

from .common import f64


def _silu(x):
    return x / (1.0 + np.exp(-x))


def _dsilu(x):
    s = 1.0 / (1.0 + np.exp(-x))
    return s * (1.0 + x * (1.0 - s))


def rmsnorm_gated(x, g=None, w=None, eps=1e-5):
    """RMSNorm(x) * w * silu(g) over the last axis (g / w optional)."""
    x = f64(x)
    r = 1.0 / np.sqrt((x * x).mean(-1, keepdims=True) + eps)
    y = x * r
    if w is not None:
        y = y * f64(w)
    if g is not None:
        y = y * _silu(f64(g))
    return y


def rmsnorm_gated_bwd(x, g, w, dy, eps=1e-5):
    """(dx, dg or None, dw or None) of rmsnorm_gated."""
    x, dy = f64(x), f64(dy)
    D = x.shape[-1]
    r = 1.0 / np.sqrt((x * x).mean(-1, keepdims=True) + eps)
    xh = x * r
    wv = np.ones(D) if w is None else f64(w)
    s = np.ones_like(x) if g is None else _silu(f64(g))
    dxh = dy * wv * s
    dx = r * (dxh - xh * (dxh * xh).mean(-1, keepdims=True))
    dg = None if g is None else dy * xh * wv * _dsilu(f64(g))
    dw = None if w is None else (dy * xh * s).reshape(-1, D).sum(0)
    return dx, dg, dw


def _segments(B, T, cu):
    if cu is None:
        return [(b, 0, T) for b in range(B)]
    return [(0, int(cu[i]), int(cu[i + 1])) for i in range(len(cu) - 1)]


def short_conv(x, w, b=None, activation="silu", cu_seqlens=None):
    """x [B,T,D], w [D,W], b [D] -> y [B,T,D]."""
    x, w = f64(x), f64(w)
    B, T, D = x.shape
    W = w.shape[1]
    pre = np.zeros_like(x)
    for bi, s, e in _segments(B, T, cu_seqlens):
        seg = np.concatenate([np.zeros((W - 1, D)), x[bi, s:e]], 0)
        for t in range(e - s):
            pre[bi, s + t] = (seg[t:t + W] * w.T).sum(0)
    if b is not None:
        pre = pre + f64(b)
    return _silu(pre) if activation in ("silu", "swish") else pre


def short_conv_bwd(x, w, b, dy, activation="silu", cu_seqlens=None):
    """(dx, dw [D,W], db [D] or None) of short_conv."""
    x, w, dy = f64(x), f64(w), f64(dy)
    B, T, D = x.shape
    W = w.shape[1]
    pre = short_conv(x, w, b, None, cu_seqlens)
    dpre = dy * _dsilu(pre) if activation in ("silu", "swish") else dy
    dx = np.zeros_like(x)
    dw = np.zeros_like(w)
    for bi, s, e in _segments(B, T, cu_seqlens):
        L = e - s
        for t in range(L):
            for j in range(W):
                p = t - W + 1 + j          # input position feeding output t through tap j
                if p >= 0:
                    dx[bi, s + p] += dpre[bi, s + t] * w[:, j]
                    dw[:, j] += dpre[bi, s + t] * x[bi, s + p]
    db = None if b is None else dpre.reshape(-1, D).sum(0)
    return dx, dw, db


def short_conv_final_state(x, W, cu_seqlens=None):
    """[N, D, W]: the last W inputs of each sequence, zero left-padded."""
    x = f64(x)
    B, T, D = x.shape
    out = []
    for bi, s, e in _segments(B, T, cu_seqlens):
        seg = x[bi, s:e]
        if seg.shape[0] < W:
            seg = np.concatenate([np.zeros((W - seg.shape[0], D)), seg], 0)
        out.append(seg[-W:].T)
    return np.stack(out, 0)


def short_conv_step(x, cache, w, b=None, activation="silu"):
    """x [N,D], cache [N,D,W] or None -> (y [N,D], new cache or None)."""
    x, w = f64(x), f64(w)
    if cache is not None:
        c = np.concatenate([f64(cache)[..., 1:], x[..., None]], -1)
        pre = (c * w).sum(-1)
    else:
        c = None
        pre = x * w[:, -1]
    if b is not None:
        pre = pre + f64(b)
    y = _silu(pre) if activation in ("silu", "swish") else pre
    return y, c
