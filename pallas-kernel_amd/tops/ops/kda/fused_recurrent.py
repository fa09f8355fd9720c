"""fused_recurrent_kda on MI355X (tops/ops/kda/fused_recurrent.py:18-105 and the FLA-aligned
surface of tops/cpu/ops/kda/fused_recurrent.py:71-565).

The reference runs the per-token delta rule as a scan:
    S' = S * exp(g_t);  S = S' + beta_t k_t (v_t - k_t^T S')^T;  o_t = S^T (scale q_t).
Here the same recurrence runs through the chunked KDA kernels (the chunk form is an exact
rewrite of the per-token recurrence, equal up to fp32 rounding), which keeps the state on
chip across a chunk instead of re-reading it per token; calls of at most a few tokens per
sequence that need no gradient (decode steps) run the per-token recurrence itself on the
register-state decode kernel, which reads and writes each state once.

FLA options (keyword-only here, so the accelerator tier's positional order
q, k, v, g, beta, scale, initial_state, output_final_state is kept):
  * use_gate_in_kernel: g holds raw gates, activated with A_log / dt_bias / lower_bound
    (tops_kda_gate_fwd);
  * use_qk_l2norm_in_kernel: q, k are L2-normalised in float32 (tops_l2norm_fwd) and the
    recurrence runs in float32;
  * grouped heads: q, k, g, beta may carry fewer heads than v (each is repeated to v's
    head count, tops/cpu/ops/kda/fused_recurrent.py:21-40);
  * cu_seqlens (B == 1): one recurrence per packed sequence, states [N, HV, K, V];
  * transpose_state_layout: states passed and returned as [N, HV, V, K].
The output has v's dtype (or `out`'s).  Everything is differentiable through torch
autograd, gates and normalisation included.
"""
from __future__ import annotations

import torch

from ... import _native as N
from ...utils import to_device
from ..gla.fused_recurrent import decode_sized
from .chunk import _prologue, chunk_kda
from .l2norm import l2norm


def _decode(q, k, v, g, beta, scale, h0, output_final_state, cu_seqlens, n):
    """Sequences of at most DECODE_MAX_TOKENS tokens that need no gradient (decode steps) on the
    register-state kernel (tops_kda_fused_recurrent_fwd_decode).  Returns (o, ht or None) or
    None where it does not apply."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad
                                       for t in (q, k, v, g, beta, h0)):
        return None
    if q.dtype not in (torch.float32, torch.bfloat16) or K > 128 or K % 4:
        return None
    if not decode_sized(T, cu_seqlens):
        return None
    q, k, v = (x.contiguous() for x in (q, k, v))
    f32 = lambda x: None if x is None else x.contiguous().to(torch.float32)  # noqa: E731
    o = torch.empty_like(v)
    ht = torch.empty(n, H, K, V, device=q.device, dtype=torch.float32) if output_final_state else None
    cu = None if cu_seqlens is None else to_device(cu_seqlens, q.device, torch.int32)
    N.call("tops_kda_fused_recurrent_fwd_decode", N.ptr(q), N.ptr(k), N.ptr(v), N.ptr(f32(g)),
           N.ptr(f32(beta)), N.ptr(f32(h0)), N.ptr(o), N.ptr(ht), N.ptr(cu), B, T, H, K, V, n,
           N.dtype_code(q.dtype), float(K ** -0.5 if scale is None else scale), N.stream())
    return o, ht


def _require(cond, msg):
    if not cond:
        raise AssertionError(msg)


def _repeat_heads(x: torch.Tensor, heads: int, name: str) -> torch.Tensor:
    h = x.shape[2]
    _require(heads % h == 0, f"{name} heads {h} must divide target heads {heads}")
    return x if h == heads else x.repeat_interleave(heads // h, dim=2)


def _run(q, k, v, g, beta, A_log, dt_bias, scale, initial_state, output_final_state,
         use_qk_l2norm_in_kernel, use_gate_in_kernel, lower_bound, cu_seqlens,
         transpose_state_layout):
    _require(q.ndim == 4, f"q must be 4D [B,T,H,K], got shape {tuple(q.shape)}")
    _require(k.ndim == 4 and k.shape[:2] == q.shape[:2] and k.shape[-1] == q.shape[-1],
             f"k shape {tuple(k.shape)} incompatible with q shape {tuple(q.shape)}")
    _require(v.ndim == 4 and v.shape[:2] == q.shape[:2],
             f"v shape {tuple(v.shape)} incompatible with q shape {tuple(q.shape)}")
    _require(g.ndim == 4 and g.shape[:2] == q.shape[:2] and g.shape[-1] == q.shape[-1],
             f"g shape {tuple(g.shape)} incompatible with q shape {tuple(q.shape)}")
    _require(beta.ndim == 3 and beta.shape[:2] == q.shape[:2],
             f"beta shape {tuple(beta.shape)} incompatible with q shape {tuple(q.shape)}")
    B, T, H, K = q.shape
    HV, V = v.shape[2], v.shape[3]
    if cu_seqlens is not None:
        _require(B == 1, f"cu_seqlens requires B=1, got {B}")
    n = len(cu_seqlens) - 1 if cu_seqlens is not None else B
    out_dtype = v.dtype
    if use_qk_l2norm_in_kernel:
        # normalising commutes with the head repeat: normalise the H heads once, in fp32,
        # so the repeat's backward sums fp32 gradients
        q, k = l2norm(q), l2norm(k)
        v = v.to(torch.float32)
    q, k, g = (_repeat_heads(x, HV, nm) for x, nm in ((q, "q"), (k, "k"), (g, "g")))
    beta = _repeat_heads(beta.unsqueeze(-1), HV, "beta").squeeze(-1)
    h0 = initial_state
    if h0 is not None:
        want = (n, HV, V, K) if transpose_state_layout else (n, HV, K, V)
        _require(tuple(h0.shape) == want, f"initial_state shape {tuple(h0.shape)} != {want}")
        if transpose_state_layout:
            h0 = h0.transpose(-1, -2)
    q, k, v, g = _prologue(q, k, v, g, A_log, dt_bias, use_gate_in_kernel, lower_bound, False)
    if q.dtype != v.dtype:        # e.g. bf16 q, k with fp32 v: run in float32
        q, k, v = (x.to(torch.float32) for x in (q, k, v))
    r = _decode(q, k, v, g, beta, scale, h0, output_final_state, cu_seqlens, n)
    o, ht = r if r is not None else chunk_kda(q, k, v, g, beta, scale=scale, initial_state=h0,
                                              output_final_state=output_final_state,
                                              cu_seqlens=cu_seqlens)
    if ht is not None and transpose_state_layout:
        ht = ht.transpose(-1, -2)
    return o.to(out_dtype), ht


def fused_recurrent_kda(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor,
                        beta: torch.Tensor, scale: float | None = None,
                        initial_state: torch.Tensor | None = None,
                        output_final_state: bool = False, *,
                        A_log: torch.Tensor | None = None, dt_bias: torch.Tensor | None = None,
                        use_qk_l2norm_in_kernel: bool = False, use_gate_in_kernel: bool = False,
                        lower_bound: float | None = None, cu_seqlens=None,
                        transpose_state_layout: bool = False, **kwargs):
    """q, k [B,T,H,K]; v [B,T,HV,V]; g [B,T,H,K] (natural-log gates, or raw gates with
    use_gate_in_kernel); beta [B,T,H]; initial_state [N,HV,K,V].  Returns (o [B,T,HV,V] in
    v.dtype, final_state [N,HV,K,V] float32 or None)."""
    return _run(q, k, v, g, beta, A_log, dt_bias, scale, initial_state, output_final_state,
                use_qk_l2norm_in_kernel, use_gate_in_kernel, lower_bound, cu_seqlens,
                transpose_state_layout)


def fused_recurrent_kda_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor,
                            beta: torch.Tensor, A_log: torch.Tensor | None = None,
                            dt_bias: torch.Tensor | None = None, scale: float | None = None,
                            initial_state: torch.Tensor | None = None,
                            output_final_state: bool = False,
                            use_qk_l2norm_in_kernel: bool = False,
                            use_gate_in_kernel: bool = False, lower_bound: float | None = None,
                            cu_seqlens=None, ssm_state_indices=None, num_accepted_tokens=None,
                            inplace_final_state: bool = True, out: torch.Tensor | None = None,
                            transpose_state_layout: bool = False, **kwargs):
    """FLA forward API (tops/cpu/ops/kda/fused_recurrent.py:71-209, 479-520).  With
    inplace_final_state (the default) an initial_state is required and the final state is
    returned in its dtype; as in the reference, the caller's initial_state is not modified.
    With `out`, the output is written into it and takes its dtype."""
    _require(ssm_state_indices is None, "ssm_state_indices is not supported")
    _require(num_accepted_tokens is None, "num_accepted_tokens is not supported")
    if inplace_final_state:
        _require(initial_state is not None,
                 "initial_state is required when inplace_final_state=True")
    o, ht = _run(q, k, v, g, beta, A_log, dt_bias, scale, initial_state,
                 output_final_state or inplace_final_state, use_qk_l2norm_in_kernel,
                 use_gate_in_kernel, lower_bound, cu_seqlens, transpose_state_layout)
    if inplace_final_state and ht is not None:
        ht = ht.to(initial_state.dtype)
    if out is not None:
        _require(tuple(out.shape) == tuple(o.shape),
                 f"out shape {tuple(out.shape)} != {tuple(o.shape)}")
        with torch.no_grad():
            out.copy_(o)
        o = out
    return o, ht


def fused_recurrent_kda_bwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor,
                            beta: torch.Tensor, do: torch.Tensor,
                            A_log: torch.Tensor | None = None,
                            dt_bias: torch.Tensor | None = None,
                            initial_state: torch.Tensor | None = None,
                            dht: torch.Tensor | None = None, scale: float | None = None,
                            use_qk_l2norm_in_kernel: bool = False,
                            use_gate_in_kernel: bool = False, lower_bound: float | None = None,
                            transpose_state_layout: bool = False, **kwargs):
    """FLA backward API (tops/cpu/ops/kda/fused_recurrent.py:212-475): (dq, dk, dv, dg, dbeta,
    dh0).  As in the reference, the gradients are those of the recurrence's own inputs:
    with use_qk_l2norm_in_kernel / use_gate_in_kernel, dq and dk are w.r.t. the normalised
    q, k and dg w.r.t. the activated gate (no chain through the prologue; autograd of
    fused_recurrent_kda gives the chained ones).  dq, dk, dv, dg, dbeta in the inputs'
    dtypes; dh0 float32 or None."""
    _require(q.ndim == 4 and k.shape == q.shape, f"k shape {tuple(k.shape)} != q shape {tuple(q.shape)}")
    _require(v.ndim == 4 and v.shape[:3] == q.shape[:3],
             f"v shape {tuple(v.shape)} incompatible with q shape {tuple(q.shape)}")
    _require(g.shape == q.shape, f"g shape {tuple(g.shape)} != q shape {tuple(q.shape)}")
    _require(beta.ndim == 3 and beta.shape == q.shape[:3],
             f"beta shape {tuple(beta.shape)} != {tuple(q.shape[:3])}")
    _require(do.shape == v.shape, f"do shape {tuple(do.shape)} != v shape {tuple(v.shape)}")
    with torch.no_grad():
        qn, kn, vn, gn = _prologue(q, k, v, g, A_log, dt_bias, use_gate_in_kernel, lower_bound,
                                   use_qk_l2norm_in_kernel)
        if qn.dtype != vn.dtype:
            qn, kn, vn = (x.to(torch.float32) for x in (qn, kn, vn))
    leaves = [x.detach().requires_grad_() for x in (qn, kn, vn, gn, beta)]
    h0 = None
    if initial_state is not None:
        h0 = initial_state.transpose(-1, -2) if transpose_state_layout else initial_state
        h0 = h0.detach().to(torch.float32).requires_grad_()
    with torch.enable_grad():
        o, ht = chunk_kda(*leaves, scale=scale, initial_state=h0,
                          output_final_state=dht is not None)
        outs, grads = [o], [do.to(o.dtype)]
        if dht is not None:
            d = dht.transpose(-1, -2) if transpose_state_layout else dht
            outs.append(ht)
            grads.append(d.to(torch.float32))
        inputs = leaves + ([h0] if h0 is not None else [])
        gr = torch.autograd.grad(outs, inputs, grads, allow_unused=True)
    dq, dk, dv, dg, dbeta = (torch.zeros_like(x) if d is None else d
                             for x, d in zip(leaves, gr[:5]))
    dh0 = None
    if h0 is not None:
        dh0 = gr[5] if gr[5] is not None else torch.zeros_like(h0)
        if transpose_state_layout:
            dh0 = dh0.transpose(-1, -2)
    return (dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype), dg.to(g.dtype),
            dbeta.to(beta.dtype), dh0)


__all__ = ["fused_recurrent_kda", "fused_recurrent_kda_fwd", "fused_recurrent_kda_bwd"]
