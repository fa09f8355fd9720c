"""Float64 oracle for the KDA gate activation and the q / k L2 normalisation (test
infrastructure only: imported by tests/ and nothing else).

Restates:
  - tops/cpu/ops/kda/gate.py:22-58   _expand_headwise_params (A_log / dt_bias head broadcast)
  - tops/cpu/ops/kda/gate.py:61-96   naive_kda_gate, naive_kda_lowerbound_gate
        standard:     y = -exp(A[h]) * softplus(g + b[h,k])
        lower bound:  y = lower_bound * sigmoid(exp(A[h]) * (g + b[h,k]))
  - tops/ops/kda/gate.py:54-119      kda_gate_bwd (analytic gradients), here extended to the
        head broadcast: dA and dbias are summed over the repeated heads, as autodiff of the
        CPU tier's broadcast does
  - tops/ops/kda/gate.py:19-51       kda_gate_chunk_cumsum (natural log -> log2, chunk-local)
  - tops/cpu/ops/kda/fused_recurrent.py:14-18  _l2_normalize_last_dim:
        y = x / sqrt(sum x^2 + 1e-6)
"""

from __future__ import annotations

import numpy as np

from .common import f64

L2_EPS = 1e-6


def expand_headwise(A_log, dt_bias, H: int, K: int):
    """A [H] and bias [H, K] (or None) for H effective heads (tops/cpu/ops/kda/gate.py:22-58)."""
    A_log = f64(A_log)
    assert A_log.ndim == 1 and H % A_log.shape[0] == 0
    rep = H // A_log.shape[0]
    A = np.repeat(A_log, rep)
    if dt_bias is None:
        return A, None
    b = f64(dt_bias)
    assert b.ndim == 1 and b.shape[0] in (A_log.shape[0] * K, H * K)
    if b.shape[0] == H * K:
        return A, b.reshape(H, K)
    return A, np.repeat(b.reshape(-1, K), rep, axis=0)


def _softplus(x):
    return np.maximum(x, 0.0) + np.log1p(np.exp(-np.abs(x)))


def _sigmoid(x):
    return 0.5 * (1.0 + np.tanh(0.5 * x))


def kda_gate(g, A_log, dt_bias=None, lower_bound=None):
    """Activated gate, float64 [..., H, K]."""
    g = f64(g)
    H, K = g.shape[-2:]
    A, b = expand_headwise(A_log, dt_bias, H, K)
    x = g if b is None else g + b
    if lower_bound is None:
        return -np.exp(A)[:, None] * _softplus(x)
    return lower_bound * _sigmoid(np.exp(A)[:, None] * x)


def _fold(x_hk, n_base: int):
    """Sum [H, ...] over the head repeats back to [n_base, ...]."""
    H = x_hk.shape[0]
    return x_hk.reshape(n_base, H // n_base, *x_hk.shape[1:]).sum(1)


def kda_gate_bwd(g, A_log, dt_bias, dyg, lower_bound=None):
    """(dg [..., H, K], dA [len(A_log)], dbias [len(dt_bias)] or None)
    (tops/ops/kda/gate.py:54-119, head broadcast folded back)."""
    g, dyg = f64(g), f64(dyg)
    H, K = g.shape[-2:]
    A, b = expand_headwise(A_log, dt_bias, H, K)
    x = g if b is None else g + b
    eA = np.exp(A)[:, None]
    if lower_bound is None:
        y = -eA * _softplus(x)
        dg = -eA * dyg * _sigmoid(x)
        dA_el = dyg * y
    else:
        s = _sigmoid(eA * x)
        dg = dyg * lower_bound * s * (1.0 - s) * eA
        dA_el = dg * x
    axes = tuple(range(g.ndim - 2))
    dA_h = dA_el.sum(axis=axes).sum(-1)                      # [H]
    dA = _fold(dA_h, np.asarray(A_log).shape[0])
    dbias = None
    if dt_bias is not None:
        db_hk = dg.sum(axis=axes)                            # [H, K]
        nb = np.asarray(dt_bias).shape[0] // K
        dbias = _fold(db_hk, nb).reshape(-1)
    return dg, dA, dbias


def kda_gate_chunk_cumsum(g, chunk_size: int, cu_seqlens=None):
    """log2 chunk-local cumsum of natural-log gates (tops/ops/kda/gate.py:19-51)."""
    g = f64(g) / np.log(2.0)
    out = np.empty_like(g)
    B, T = g.shape[:2]
    seqs = [(b, 0, T) for b in range(B)] if cu_seqlens is None else \
        [(0, int(cu_seqlens[i]), int(cu_seqlens[i + 1])) for i in range(len(cu_seqlens) - 1)]
    for b, lo, hi in seqs:
        for c0 in range(lo, hi, chunk_size):
            c1 = min(c0 + chunk_size, hi)
            out[b, c0:c1] = np.cumsum(g[b, c0:c1], axis=0)
    return out


def l2norm(x):
    """y = x / sqrt(sum x^2 + 1e-6) over the last axis."""
    x = f64(x)
    return x / np.sqrt((x * x).sum(-1, keepdims=True) + L2_EPS)


def l2norm_bwd(x, dy):
    """dL/dx of y = l2norm(x): r (dy - y (y . dy)), r = 1 / sqrt(sum x^2 + eps)."""
    x, dy = f64(x), f64(dy)
    r = 1.0 / np.sqrt((x * x).sum(-1, keepdims=True) + L2_EPS)
    y = x * r
    return r * (dy - y * (y * dy).sum(-1, keepdims=True))
