"""KDA gate on MI355X: activation, chunk-local cumsum and backward.

Mirrors both gate modules of the reference:
  * tops/ops/kda/gate.py (the accelerator tier): `kda_gate_chunk_cumsum(g, chunk_size,
    cu_seqlens)` (natural-log gates -> log2 chunk-local cumsum, :19-51) and
    `kda_gate_bwd(g, A_log, dt_bias, dyg, lower_bound)` (:54-119);
  * tops/cpu/ops/kda/gate.py (the FLA-aligned surface): `naive_kda_gate`,
    `naive_kda_lowerbound_gate`, `kda_gate_fwd`, `fused_kda_gate` (:60-176) and the
    FLA form of `kda_gate_chunk_cumsum(g, A_log, chunk_size, scale, dt_bias, ...)` (:179-204).
`kda_gate_chunk_cumsum` takes either call form: a tensor in the second position (or an
`A_log` keyword) selects the FLA form.

    standard      y = -exp(A_log[h]) * softplus(g + dt_bias[h, k])
    lower bound   y = lower_bound * sigmoid(exp(A_log[h]) * (g + dt_bias[h, k]))

A_log [H'] with H' dividing the gate's head count (head h reads A_log[h / (H / H')]);
dt_bias [H' * K] or [H * K] (tops/cpu/ops/kda/gate.py:20-57).  The activation runs in
float32 on the HIP kernels of csrc/kda_gate.hip (tops_kda_gate_*); `fused_kda_gate` and the
two naive gates are differentiable (torch.autograd.Function over tops_kda_gate_bwd), with
dA_log and dt_bias gradients summed over the heads that share a parameter row.
Errors follow the reference: shape mismatches raise AssertionError.
"""
from __future__ import annotations

import math

import torch

from ... import _native as N
from ...utils import ChunkPlan

GATE_NONE = 0
GATE_SOFTPLUS = 1
GATE_LOWER_BOUND = 2

_RCP_LN2 = 1.0 / math.log(2.0)


def _require(cond, msg):
    if not cond:
        raise AssertionError(msg)


def _kernel_input(x: torch.Tensor) -> torch.Tensor:
    """Contiguous float32 / bfloat16 view of a gate tensor (other dtypes go to float32)."""
    if x.dtype not in (torch.float32, torch.bfloat16):
        x = x.to(torch.float32)
    return x.contiguous()


def _params(A_log, dt_bias, H: int, K: int):
    """float32 device copies of A_log / dt_bias with their head counts, checked as
    _expand_headwise_params (tops/cpu/ops/kda/gate.py:20-57) checks them."""
    _require(A_log is not None, "A_log is required for the KDA gate")
    _require(A_log.ndim == 1, f"A_log must be 1D, got shape {tuple(A_log.shape)}")
    ha = A_log.shape[0]
    _require(ha > 0 and H % ha == 0, f"Effective heads {H} must be divisible by A_log heads {ha}")
    a32 = A_log.detach().to(torch.float32).contiguous()
    if dt_bias is None:
        return a32, None, ha, 0
    _require(dt_bias.ndim == 1, f"dt_bias must be 1D, got shape {tuple(dt_bias.shape)}")
    n = dt_bias.shape[0]
    _require(n in (ha * K, H * K),
             f"dt_bias shape {tuple(dt_bias.shape)} incompatible with "
             f"(base={ha * K}, expanded={H * K})")
    return a32, dt_bias.detach().to(torch.float32).contiguous(), ha, n // K


def _mode(lower_bound) -> tuple[int, float]:
    return (GATE_SOFTPLUS, 0.0) if lower_bound is None else (GATE_LOWER_BOUND, float(lower_bound))


def _gate_fwd(g: torch.Tensor, A_log, dt_bias, lower_bound) -> torch.Tensor:
    _require(g.ndim >= 2, f"g must be [..., H, K], got shape {tuple(g.shape)}")
    N.require_cuda(g, A_log, dt_bias)
    H, K = g.shape[-2:]
    a32, b32, ha, hb = _params(A_log, dt_bias, H, K)
    gk = _kernel_input(g)
    y = torch.empty(g.shape, device=g.device, dtype=torch.float32)
    mode, lb = _mode(lower_bound)
    rows = g.numel() // (H * K) if H * K else 0
    N.call("tops_kda_gate_fwd", N.ptr(gk), N.dtype_code(gk.dtype), N.ptr(a32), N.ptr(b32),
           N.ptr(y), rows, H, K, ha, hb, mode, lb, N.stream())
    return y


def _gate_bwd(g: torch.Tensor, A_log, dt_bias, dyg: torch.Tensor, lower_bound):
    """(dg in g.dtype, dA in A_log.dtype, dbias in dt_bias.dtype or None)."""
    N.require_cuda(g, A_log, dt_bias, dyg)
    H, K = g.shape[-2:]
    _require(tuple(dyg.shape) == tuple(g.shape),
             f"dyg shape {tuple(dyg.shape)} != g shape {tuple(g.shape)}")
    a32, b32, ha, hb = _params(A_log, dt_bias, H, K)
    gk = _kernel_input(g)
    dy = dyg.contiguous().to(torch.float32)
    rows = g.numel() // (H * K)
    dg = torch.empty_like(gk)
    dA = torch.empty(ha, device=g.device, dtype=torch.float32)
    db = None if b32 is None else torch.empty(hb * K, device=g.device, dtype=torch.float32)
    n_ws = int(N.lib().tops_kda_gate_bwd_workspace(rows, H, K))
    if n_ws < 0:
        raise ValueError(f"tops_kda_gate_bwd_workspace({rows}, {H}, {K}) failed")
    ws = torch.empty(max(n_ws, 1), device=g.device, dtype=torch.float32)
    mode, lb = _mode(lower_bound)
    N.call("tops_kda_gate_bwd", N.ptr(gk), N.dtype_code(gk.dtype), N.ptr(a32), N.ptr(b32),
           N.ptr(dy), N.ptr(dg), N.ptr(dA), N.ptr(db), N.ptr(ws), n_ws, rows, H, K, ha, hb,
           mode, lb, N.stream())
    return (dg.to(g.dtype), dA.to(A_log.dtype),
            None if db is None else db.to(dt_bias.dtype))


class _KDAGate(torch.autograd.Function):
    @staticmethod
    def forward(ctx, g, A_log, dt_bias, lower_bound):
        y = _gate_fwd(g, A_log, dt_bias, lower_bound)
        ctx.save_for_backward(g, A_log, dt_bias)
        ctx.lower_bound = lower_bound
        return y

    @staticmethod
    def backward(ctx, dy):
        g, A_log, dt_bias = ctx.saved_tensors
        dg, dA, db = _gate_bwd(g, A_log, dt_bias, dy, ctx.lower_bound)
        return dg, dA, db, None


def kda_gate_fwd(g: torch.Tensor, A_log: torch.Tensor, dt_bias: torch.Tensor | None = None,
                 lower_bound: float | None = None,
                 output_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Activated gate [..., H, K] (tops/cpu/ops/kda/gate.py:97-115), differentiable in g,
    A_log and dt_bias."""
    return _KDAGate.apply(g, A_log, dt_bias, lower_bound).to(output_dtype)


def fused_kda_gate(g: torch.Tensor, A_log: torch.Tensor, dt_bias: torch.Tensor | None = None,
                   lower_bound: float | None = None,
                   output_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Public gate API (tops/cpu/ops/kda/gate.py:161-176)."""
    return kda_gate_fwd(g, A_log, dt_bias=dt_bias, lower_bound=lower_bound,
                        output_dtype=output_dtype)


def naive_kda_gate(g: torch.Tensor, A_log: torch.Tensor, dt_bias: torch.Tensor | None = None,
                   output_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """-exp(A_log) * softplus(g + dt_bias) (tops/cpu/ops/kda/gate.py:60-75)."""
    return kda_gate_fwd(g, A_log, dt_bias=dt_bias, output_dtype=output_dtype)


def naive_kda_lowerbound_gate(g: torch.Tensor, A_log: torch.Tensor,
                              dt_bias: torch.Tensor | None = None, lower_bound: float = -5.0,
                              output_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """lower_bound * sigmoid(exp(A_log) * (g + dt_bias)) (tops/cpu/ops/kda/gate.py:78-95)."""
    return kda_gate_fwd(g, A_log, dt_bias=dt_bias, lower_bound=lower_bound,
                        output_dtype=output_dtype)


def kda_gate_bwd(g: torch.Tensor, A_log: torch.Tensor, dt_bias: torch.Tensor | None = None,
                 dyg: torch.Tensor | None = None, lower_bound: float | None = None):
    """(dg, dA, dbias) of the gate (tops/ops/kda/gate.py:54-119): dg in g.dtype, dA in
    A_log.dtype [len(A_log)], dbias in dt_bias.dtype [len(dt_bias)] or None."""
    _require(dyg is not None, "dyg must be provided")
    with torch.no_grad():
        return _gate_bwd(g, A_log, dt_bias, dyg, lower_bound)


def _cumsum(g, A_log, dt_bias, lower_bound, mode, scale, chunk_size: int, cu_seqlens):
    _require(g.ndim == 4, f"g must be [B,T,H,K], got shape {tuple(g.shape)}")
    _require(int(chunk_size) > 0, f"chunk_size must be positive, got {chunk_size}")
    N.require_cuda(g)
    B, T, H, K = g.shape
    if cu_seqlens is not None:
        _require(B == 1, f"cu_seqlens requires B=1, got {B}")
    a32 = b32 = None
    ha = hb = 0
    lb = 0.0
    if mode != GATE_NONE:
        a32, b32, ha, hb = _params(A_log, dt_bias, H, K)
        mode, lb = _mode(lower_bound)
    gk = _kernel_input(g)
    out = torch.empty(g.shape, device=g.device, dtype=torch.float32)
    if g.numel() == 0:
        return out
    plan = ChunkPlan.get(B, T, cu_seqlens, g.device, int(chunk_size))
    with torch.no_grad():
        N.call("tops_kda_gate_chunk_cumsum", N.ptr(gk), N.dtype_code(gk.dtype), N.ptr(a32),
               N.ptr(b32), N.ptr(out), N.ptr(plan.cu_dev), N.ptr(plan.offsets_dev),
               N.ptr(plan.chunk_map_dev), plan.total, B, T, H, K, ha, hb, int(chunk_size),
               mode, lb, float(scale), N.stream())
    return out


def kda_gate_chunk_cumsum(g: torch.Tensor, *args, **kwargs) -> torch.Tensor:
    """Chunk-local cumsum of KDA gates, float32 [B,T,H,K].

    Accelerator form (tops/ops/kda/gate.py:19-51):
        kda_gate_chunk_cumsum(g, chunk_size, cu_seqlens=None)
      g holds activated natural-log gates; the result is in log2 space, so that
      exp2(out[t]) = prod over the chunk up to t of exp(g).
    FLA form (tops/cpu/ops/kda/gate.py:179-204):
        kda_gate_chunk_cumsum(g, A_log, chunk_size, scale=None, dt_bias=None,
                              cu_seqlens=None, output_dtype=float32, chunk_indices=None,
                              lower_bound=None, **kwargs)
      g holds raw gates; they are activated, summed chunk-locally and multiplied by
      `scale` (when given).
    """
    fla = "A_log" in kwargs or (args and isinstance(args[0], torch.Tensor))
    if not fla:
        names = ("chunk_size", "cu_seqlens")
        p = dict(zip(names, args))
        for n in names:
            if n in kwargs:
                p[n] = kwargs.pop(n)
        _require(not kwargs, f"unexpected arguments {sorted(kwargs)}")
        return _cumsum(g, None, None, None, GATE_NONE, _RCP_LN2, p["chunk_size"],
                       p.get("cu_seqlens"))
    names = ("A_log", "chunk_size", "scale", "dt_bias", "cu_seqlens", "output_dtype",
             "chunk_indices", "lower_bound")
    p = dict(zip(names, args))
    for n in names:
        if n in kwargs:
            p[n] = kwargs.pop(n)
    scale = p.get("scale")
    out = _cumsum(g, p["A_log"], p.get("dt_bias"), p.get("lower_bound"), GATE_SOFTPLUS,
                  1.0 if scale is None else scale, p["chunk_size"], p.get("cu_seqlens"))
    return out.to(p.get("output_dtype") or torch.float32)


__all__ = [
    "naive_kda_gate",
    "naive_kda_lowerbound_gate",
    "kda_gate_fwd",
    "kda_gate_bwd",
    "fused_kda_gate",
    "kda_gate_chunk_cumsum",
]
