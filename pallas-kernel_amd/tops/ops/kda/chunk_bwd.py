"""chunk_kda_bwd on MI355X (mirrors tops/ops/kda/chunk_bwd.py:655-832): the functional KDA
backward taking the chunk-local log2 gate cumsum g, as the reference's custom_vjp calls it.

The HIP backward (tops_kda_chunk_bwd) works on the per-token natural-log gate and
recomputes the forward intermediates itself, so the per-token gate is recovered from g
(differences inside each chunk, times ln 2) and Aqk / Akk are not read (the reference
recomputes them too unless disable_recompute).  The returned dg is the reference's: the
gradient w.r.t. the log2 gate, i.e. ln 2 times the natural-log gradient; with
use_gate_in_kernel it is chained through kda_gate_bwd to (dg, dA_log, dt_bias) as the
reference does.
"""
from __future__ import annotations

import math

import numpy as np
import torch

from ...utils import ChunkPlan, to_device
from ..common._stage import cu_host, require
from .chunk import _bwd, _check, _fwd

_LN2 = math.log(2.0)


def _chunk_starts(B: int, T: int, cu, C: int, device) -> torch.Tensor:
    """[T] bool (B rows share it) or [T] for a packed varlen batch: token opens a chunk."""
    t = np.arange(T)
    if cu is None:
        m = t % C == 0
    else:
        m = np.zeros(T, bool)
        for a, b in zip(cu[:-1], cu[1:]):
            m[a:b] = (t[a:b] - a) % C == 0
    return to_device(m, device, torch.bool)


def chunk_kda_bwd(q, k, v, beta, Aqk, Akk, scale, initial_state, do, dht, *, g=None, g_org=None,
                  cu_seqlens=None, chunk_indices=None, chunk_size: int = 64, safe_gate: bool = False,
                  lower_bound=None, use_gate_in_kernel: bool = False, A_log=None, dt_bias=None,
                  disable_recompute: bool = False, cp_context=None,
                  transpose_state_layout: bool = False, **kwargs):
    """Returns (dq, dk, dv, db, dg, dh0, dA_log, dbias); dh0 when initial_state is given,
    dA_log / dbias with use_gate_in_kernel (else None)."""
    del Aqk, Akk, chunk_indices, safe_gate, disable_recompute, cp_context, kwargs
    require(g is not None, "g (the chunk-local log2 gate cumsum) is required")
    C = int(chunk_size)
    require(C > 0 and C & (C - 1) == 0, "chunk_size must be a power of 2")
    B, T, H, K = q.shape
    cu = cu_host(cu_seqlens)
    if transpose_state_layout:
        initial_state = None if initial_state is None else initial_state.transpose(-1, -2)
        dht = None if dht is None else dht.transpose(-1, -2)
    starts = _chunk_starts(B, T, cu, C, q.device)[None, :, None, None]
    g32 = g.to(torch.float32)
    prev = torch.cat([torch.zeros_like(g32[:, :1]), g32[:, :-1]], dim=1)
    g_nat = torch.where(starts, g32, g32 - prev) * _LN2
    _check(q, k, v, g_nat, beta, initial_state, cu)
    if scale is None:
        scale = K ** -0.5
    q, k, v = (x.contiguous() for x in (q, k, v))
    b32 = beta.contiguous().to(torch.float32)
    h0 = None if initial_state is None else initial_state.contiguous().to(torch.float32)
    plan = ChunkPlan.get(B, T, cu, q.device)
    with torch.no_grad():
        _, _, saved = _fwd(q, k, v, g_nat.contiguous(), b32, h0, float(scale), False, plan,
                           keep=True)
        dq, dk, dv, db, dg, dh0 = _bwd(q, k, v, g_nat.contiguous(), b32,
                                       do.contiguous().to(q.dtype),
                                       None if dht is None else dht.contiguous().to(torch.float32),
                                       saved, float(scale), plan, want_dh0=h0 is not None)
    dg = dg * _LN2
    dA = dbias = None
    if use_gate_in_kernel:
        from .gate import kda_gate_bwd
        dg, dA, dbias = kda_gate_bwd(g_org, A_log, dt_bias, dyg=dg, lower_bound=lower_bound)
    if transpose_state_layout and dh0 is not None:
        dh0 = dh0.transpose(-1, -2)
    return dq, dk, dv, db, dg, dh0, dA, dbias


__all__ = ["chunk_kda_bwd"]
