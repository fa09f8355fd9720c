"""Chunked KDA on MI355X: drop-in for tops.ops.kda.chunk (tops/ops/kda/chunk.py).

KDA is the gated delta rule with per-channel gates (natural-log g [B,T,H,K]) and a
per-token rate beta [B,T,H]:  S_t = diag(e^g_t) S_{t-1} + beta_t k_t (v_t - k_t^T S')^T,
o_t = S_t^T (scale q_t).  `chunk_kda` keeps the reference signature
(tops/ops/kda/chunk.py:193-217) and is differentiable: a torch.autograd.Function wires the
HIP backward, the counterpart of the reference's custom_vjp (chunk.py:219-255); dg is the
gradient w.r.t. the natural-log gates, as there.

Forward: tops_kda_chunk_fwd (chunk-parallel WY preparation + delta-rule state sweep).
Backward: tops_kda_chunk_bwd (reverse state-gradient sweep, WY backward, dq/dk/dg).
The forward saves w, T^T per chunk, v_new and the per-chunk states for the backward,
where the reference saves g_cumsum, Aqk and Akk^-1 and recomputes the rest
(tops/ops/kda/chunk_bwd.py:655-760).

q, k, v are float32 or bfloat16 (one dtype); gates, beta and states are computed in
float32.  Unlike the reference, T need not be a multiple of chunk_size (the last chunk is
masked), and `cu_seqlens` is honoured: each packed sequence runs its own recurrence.
`chunk_size` is accepted for signature compatibility; the kernels tile by 64, which gives
the same result up to fp32 rounding.
"""
from __future__ import annotations

import torch

from ... import _native as N
from ...utils import CHUNK, ChunkPlan
from .._chunk_core import check_qkv


def _check(q, k, v, g, beta, initial_state, cu_seqlens):
    check_qkv(q, k, v, initial_state, cu_seqlens)
    B, T, H, K = q.shape
    V = v.shape[-1]
    assert tuple(g.shape) == (B, T, H, K), f"g shape {tuple(g.shape)} != {(B, T, H, K)}"
    assert tuple(beta.shape) == (B, T, H), f"beta shape {tuple(beta.shape)} != {(B, T, H)}"
    if V > 128:
        raise NotImplementedError(f"tops-hip KDA kernels need V <= 128 (got V={V})")


def _fwd(q, k, v, g32, b32, h0, scale, output_final_state, plan: ChunkPlan, keep: bool):
    """Returns (o, ht, saved) with saved = (w, tt, v_new, h_ckpt) when keep."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    dev, f32 = q.device, torch.float32
    o = torch.empty_like(v)
    ht = torch.empty(plan.N, H, K, V, device=dev, dtype=f32) if output_final_state else None
    u = torch.empty(B, T, H, V, device=dev, dtype=f32)
    w = torch.empty(B, T, H, K, device=dev, dtype=f32)
    tt = torch.empty(plan.total, H, CHUNK, CHUNK, device=dev, dtype=f32) if keep else None
    vn = torch.empty(B, T, H, V, device=dev, dtype=f32) if keep else None
    hs = torch.empty(plan.total, H, K, V, device=dev, dtype=f32) if keep else None
    N.call("tops_kda_chunk_fwd", N.ptr(q), N.ptr(k), N.ptr(v), N.ptr(g32), N.ptr(b32), N.ptr(h0),
           N.ptr(o), N.ptr(ht), N.ptr(u), N.ptr(w), N.ptr(tt), N.ptr(vn), N.ptr(hs),
           N.ptr(plan.cu_dev), N.ptr(plan.offsets_dev), N.ptr(plan.chunk_map_dev), plan.total,
           B, T, H, K, V, plan.N, N.dtype_code(q.dtype), float(scale), N.stream())
    return o, ht, (w, tt, vn, hs)


def _bwd(q, k, v, g32, b32, do, dht, saved, scale, plan: ChunkPlan, want_dh0: bool):
    """Returns (dq, dk, dv, dbeta, dg, dh0); dbeta, dg, dh0 in float32."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    dev, f32 = q.device, torch.float32
    w, tt, vn, hs = saved
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    dbeta = torch.empty(B, T, H, device=dev, dtype=f32)
    dg = torch.empty(B, T, H, K, device=dev, dtype=f32)
    dh0 = torch.empty(plan.N, H, K, V, device=dev, dtype=f32) if want_dh0 else None
    dh_work = torch.empty_like(hs)
    dvn_work = torch.empty(plan.total, H, V, CHUNK, device=dev, dtype=f32)
    # bf16 keeps the WY parts of dk / dg on chip (one kernel); fp32 passes them through HBM
    split = q.dtype == torch.float32
    dk_work = torch.empty(B, T, H, K, device=dev, dtype=f32) if split else None
    dg_work = torch.empty(B, T, H, K, device=dev, dtype=f32) if split else None
    N.call("tops_kda_chunk_bwd", N.ptr(q), N.ptr(k), N.ptr(v), N.ptr(g32), N.ptr(b32), N.ptr(w),
           N.ptr(tt), N.ptr(vn), N.ptr(hs), N.ptr(do), N.ptr(dht), N.ptr(dh_work), N.ptr(dvn_work),
           N.ptr(dk_work), N.ptr(dg_work), N.ptr(dq), N.ptr(dk), N.ptr(dv), N.ptr(dbeta), N.ptr(dg),
           N.ptr(dh0), N.ptr(plan.cu_dev), N.ptr(plan.offsets_dev), N.ptr(plan.chunk_map_dev),
           plan.total, B, T, H, K, V, plan.N, N.dtype_code(q.dtype), float(scale), N.stream())
    return dq, dk, dv, dbeta, dg, dh0


class _ChunkKDA(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, g, beta, scale, h0, output_final_state, cu_seqlens):
        q, k, v = (x.contiguous() for x in (q, k, v))
        g32 = g.contiguous().to(torch.float32)
        b32 = beta.contiguous().to(torch.float32)
        h032 = None if h0 is None else h0.contiguous().to(torch.float32)
        plan = ChunkPlan.get(q.shape[0], q.shape[1], cu_seqlens, q.device)
        train = any(ctx.needs_input_grad[:5]) or (h0 is not None and ctx.needs_input_grad[6])
        o, ht, saved = _fwd(q, k, v, g32, b32, h032, scale, output_final_state, plan, keep=train)
        if train:
            ctx.save_for_backward(q, k, v, g32, b32, *saved)
            ctx.plan, ctx.scale = plan, scale
            ctx.dtypes = (g.dtype, beta.dtype, None if h0 is None else h0.dtype)
        return o, ht

    @staticmethod
    def backward(ctx, do, dht):
        q, k, v, g32, b32, w, tt, vn, hs = ctx.saved_tensors
        do = do.contiguous().to(q.dtype)
        dht = None if dht is None else dht.contiguous().to(torch.float32)
        g_dt, b_dt, h0_dt = ctx.dtypes
        dq, dk, dv, dbeta, dg, dh0 = _bwd(q, k, v, g32, b32, do, dht, (w, tt, vn, hs), ctx.scale,
                                          ctx.plan, want_dh0=h0_dt is not None)
        if dh0 is not None:
            dh0 = dh0.to(h0_dt)
        return dq, dk, dv, dg.to(g_dt), dbeta.to(b_dt), None, dh0, None, None


def _prologue(q, k, v, g, A_log, dt_bias, use_gate_in_kernel, lower_bound,
              use_qk_l2norm_in_kernel):
    """The FLA-side options of KDA applied ahead of the kernels: q / k L2 normalisation
    (float32 out, so v runs in float32 with them) and the in-kernel gate activation;
    both stay differentiable (dq, dk chain through the normalisation; dg, dA_log and
    dt_bias through the gate, as tops/cpu/ops/kda/chunk_bwd.py:617-668 does for the gate)."""
    if use_qk_l2norm_in_kernel:
        from .l2norm import l2norm
        q, k = l2norm(q), l2norm(k)
        v = v.to(torch.float32)
    if use_gate_in_kernel:
        from .gate import fused_kda_gate
        if A_log is None:
            raise AssertionError("A_log is required when use_gate_in_kernel=True")
        g = fused_kda_gate(g, A_log, dt_bias=dt_bias, lower_bound=lower_bound)
    return q, k, v, g


def chunk_kda(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor,
              beta: torch.Tensor, scale: float | None = None,
              initial_state: torch.Tensor | None = None, output_final_state: bool = False,
              cu_seqlens=None, chunk_size: int = 64, *, A_log: torch.Tensor | None = None,
              dt_bias: torch.Tensor | None = None, use_gate_in_kernel: bool = False,
              lower_bound: float | None = None, use_qk_l2norm_in_kernel: bool = False):
    """Chunked KDA, forward + backward (tops/ops/kda/chunk.py:193-217).

    q, k [B,T,H,K]; v [B,T,H,V]; g [B,T,H,K] natural-log gates; beta [B,T,H];
    initial_state [N,H,K,V].  Returns (o [B,T,H,V] in v.dtype, final_state [N,H,K,V] or
    None).  The keyword-only options are FLA's: with use_gate_in_kernel, g holds raw gates
    activated by A_log / dt_bias / lower_bound (tops/cpu/ops/kda/gate.py); with
    use_qk_l2norm_in_kernel, q and k are L2-normalised first."""
    out_dtype = v.dtype
    q, k, v, g = _prologue(q, k, v, g, A_log, dt_bias, use_gate_in_kernel, lower_bound,
                           use_qk_l2norm_in_kernel)
    _check(q, k, v, g, beta, initial_state, cu_seqlens)
    if scale is None:
        scale = q.shape[-1] ** -0.5
    o, ht = _ChunkKDA.apply(q, k, v, g, beta, float(scale), initial_state,
                            bool(output_final_state), cu_seqlens)
    return o.to(out_dtype), ht


def _g_cumsum_log2(g: torch.Tensor, cu_seqlens) -> torch.Tensor:
    """Chunk-local cumsum of g / ln 2 (the reference's kda_gate_chunk_cumsum output,
    tops/ops/kda/gate.py:19-51), on tops_kda_gate_chunk_cumsum."""
    from .gate import kda_gate_chunk_cumsum
    return kda_gate_chunk_cumsum(g, CHUNK, cu_seqlens)


def chunk_kda_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor,
                  beta: torch.Tensor, scale: float | None = None,
                  initial_state: torch.Tensor | None = None, output_final_state: bool = False,
                  cu_seqlens=None, chunk_size: int = 64):
    """Forward only (tops/ops/kda/chunk.py:25-190).  Returns (o, final_state, g_cumsum,
    Aqk, Akk_inv) like the reference: g_cumsum [B,T,H,K] is the chunk-local log2 cumsum and
    Akk_inv [B,T,H,64] the per-chunk (I + Akk)^-1 (fixed-length input; None for varlen,
    whose chunks do not tile the packed axis).  Aqk is not materialised by these kernels
    (the state sweep recomputes it in registers) and is returned as None."""
    _check(q, k, v, g, beta, initial_state, cu_seqlens)
    if scale is None:
        scale = q.shape[-1] ** -0.5
    q, k, v = (x.contiguous() for x in (q, k, v))
    g32 = g.contiguous().to(torch.float32)
    b32 = beta.contiguous().to(torch.float32)
    h0 = None if initial_state is None else initial_state.contiguous().to(torch.float32)
    plan = ChunkPlan.get(q.shape[0], q.shape[1], cu_seqlens, q.device)
    with torch.no_grad():
        o, ht, (w, tt, vn, hs) = _fwd(q, k, v, g32, b32, h0, scale, output_final_state, plan,
                                      keep=True)
        g_cumsum = _g_cumsum_log2(g32, cu_seqlens)
        akk = None
        if cu_seqlens is None:
            B, T, H, _ = q.shape
            nt = plan.total // B
            akk = tt.view(B, nt, H, CHUNK, CHUNK).permute(0, 1, 4, 2, 3).reshape(
                B, nt * CHUNK, H, CHUNK)[:, :T]
    return o, ht, g_cumsum, None, akk
