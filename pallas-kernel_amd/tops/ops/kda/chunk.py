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

import numpy as np
import torch

from ... import _native as N
from ...utils import CHUNK, ChunkPlan, cdiv, checkpoint_layout, inference_inputs
from .._chunk_core import States16, check_qkv, pack_states, unpack_states


def _check(q, k, v, g, beta, initial_state, cu_seqlens):
    check_qkv(q, k, v, initial_state, cu_seqlens)
    B, T, H, K = q.shape
    V = v.shape[-1]
    assert tuple(g.shape) == (B, T, H, K), f"g shape {tuple(g.shape)} != {(B, T, H, K)}"
    assert tuple(beta.shape) == (B, T, H), f"beta shape {tuple(beta.shape)} != {(B, T, H)}"
    if V > 128:
        raise NotImplementedError(f"tops-hip KDA kernels need V <= 128 (got V={V})")


def _c16(q) -> bool:
    """Whether the training path keeps fp16 state checkpoints (bf16 inputs; the checkpoint
    layout not "full32"): the states per chunk and dS as fp16 times a power-of-two factor per
    (chunk, head, 64 columns of V), half the bytes of fp32 ones."""
    return q.dtype == torch.bfloat16 and checkpoint_layout() != "full32"


def _fwd(q, k, v, g32, b32, h0, scale, output_final_state, plan: ChunkPlan, keep: bool):
    """Returns (o, ht, saved) with saved = (w, tt, v_new, h_ckpt) when keep; h_ckpt is a
    States16 for fp16 checkpoints."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    dev, f32 = q.device, torch.float32
    o = torch.empty_like(v)
    ht = torch.empty(plan.N, H, K, V, device=dev, dtype=f32) if output_final_state else None
    u = torch.empty(B, T, H, V, device=dev, dtype=f32)
    w = torch.empty(B, T, H, K, device=dev, dtype=f32)
    tt = torch.empty(plan.total, H, CHUNK, CHUNK, device=dev, dtype=f32) if keep else None
    vn = torch.empty(B, T, H, V, device=dev, dtype=f32) if keep else None
    tail = (N.ptr(plan.cu_dev), N.ptr(plan.offsets_dev), N.ptr(plan.chunk_map_dev), plan.total,
            B, T, H, K, V, plan.N, N.dtype_code(q.dtype), float(scale), N.stream())
    head = (N.ptr(q), N.ptr(k), N.ptr(v), N.ptr(g32), N.ptr(b32), N.ptr(h0), N.ptr(o), N.ptr(ht),
            N.ptr(u), N.ptr(w), N.ptr(tt), N.ptr(vn))
    if keep and _c16(q):
        hs = States16(torch.empty(plan.total, H, K, V, device=dev, dtype=torch.float16),
                      torch.empty(plan.total, H, cdiv(V, 64), device=dev, dtype=f32))
        N.call("tops_kda_chunk_fwd_c16", *head, N.ptr(hs.h), N.ptr(hs.scale), *tail)
    else:
        hs = torch.empty(plan.total, H, K, V, device=dev, dtype=f32) if keep else None
        N.call("tops_kda_chunk_fwd", *head, N.ptr(hs), *tail)
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
    dvn_work = torch.empty(plan.total, H, V, CHUNK, device=dev, dtype=f32)
    tail = (N.ptr(dh0), N.ptr(plan.cu_dev), N.ptr(plan.offsets_dev), N.ptr(plan.chunk_map_dev),
            plan.total, B, T, H, K, V, plan.N, N.dtype_code(q.dtype), float(scale), N.stream())
    if isinstance(hs, States16):
        dh_work = States16(torch.empty_like(hs.h), torch.empty_like(hs.scale))
        N.call("tops_kda_chunk_bwd_c16", N.ptr(q), N.ptr(k), N.ptr(v), N.ptr(g32), N.ptr(b32),
               N.ptr(w), N.ptr(tt), N.ptr(vn), N.ptr(hs.h), N.ptr(hs.scale), N.ptr(do), N.ptr(dht),
               N.ptr(dh_work.h), N.ptr(dh_work.scale), N.ptr(dvn_work), N.ptr(dq), N.ptr(dk),
               N.ptr(dv), N.ptr(dbeta), N.ptr(dg), *tail)
        return dq, dk, dv, dbeta, dg, dh0
    dh_work = torch.empty_like(hs)
    # bf16 keeps the WY parts of dk / dg on chip (one kernel); fp32 passes them through HBM
    split = q.dtype == torch.float32
    dk_work = torch.empty(B, T, H, K, device=dev, dtype=f32) if split else None
    dg_work = torch.empty(B, T, H, K, device=dev, dtype=f32) if split else None
    N.call("tops_kda_chunk_bwd", N.ptr(q), N.ptr(k), N.ptr(v), N.ptr(g32), N.ptr(b32), N.ptr(w),
           N.ptr(tt), N.ptr(vn), N.ptr(hs), N.ptr(do), N.ptr(dht), N.ptr(dh_work), N.ptr(dvn_work),
           N.ptr(dk_work), N.ptr(dg_work), N.ptr(dq), N.ptr(dk), N.ptr(dv), N.ptr(dbeta), N.ptr(dg),
           *tail)
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
            ctx.save_for_backward(q, k, v, g32, b32, *saved[:3], *pack_states(saved[3]))
            ctx.plan, ctx.scale = plan, scale
            ctx.dtypes = (g.dtype, beta.dtype, None if h0 is None else h0.dtype)
        return o, ht

    @staticmethod
    def backward(ctx, do, dht):
        q, k, v, g32, b32, w, tt, vn, hs, hsc = ctx.saved_tensors
        hs = unpack_states(hs, hsc)
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
    q, k, v, g, beta, initial_state = inference_inputs(q, k, v, g, beta, initial_state)
    o, ht = _ChunkKDA.apply(q, k, v, g, beta, float(scale), initial_state,
                            bool(output_final_state), cu_seqlens)
    return o.to(out_dtype), ht


def _padded_rows(cu: "np.ndarray", C: int):
    """Row map of the per-sequence chunk layout: each sequence of the packed axis padded to
    a multiple of C.  Returns (index of each padded row's token or -1 for padding, padded
    length, position of each token in the padded layout)."""
    lens = np.diff(cu)
    plens = -(-lens // C) * C
    pstart = np.concatenate([[0], np.cumsum(plens)]).astype(np.int64)
    src = np.full(int(pstart[-1]), -1, np.int64)
    dst = np.empty(int(cu[-1]), np.int64)
    for s in range(len(lens)):
        n = int(lens[s])
        src[pstart[s]:pstart[s] + n] = np.arange(cu[s], cu[s] + n)
        dst[cu[s]:cu[s] + n] = np.arange(pstart[s], pstart[s] + n)
    return src, int(pstart[-1]), dst


def _intra_matrices(q, k, v, g_cumsum, beta, scale, C, cu_seqlens):
    """Aqk and Akk_inv [B,T,H,C] in k.dtype, the flattened per-chunk matrices of the
    reference's chunk_kda_fwd (tops/ops/kda/chunk.py:173-190), from the intra-chunk stage
    kernel at chunk size C.  A ragged last chunk is zero-padded (padded rows and columns
    never reach a valid row: both matrices are lower triangular); with cu_seqlens each
    sequence is chunked on its own, as FLA's varlen layout does."""
    from .chunk_intra import kda_intra_chunk_fwd
    B, T, H, _ = q.shape
    xs = (q, k, v, g_cumsum, beta)
    if cu_seqlens is not None:
        from ...utils import _host_cu
        src, Tp, dst = _padded_rows(_host_cu(cu_seqlens), C)
        idx = torch.as_tensor(np.maximum(src, 0), device=q.device)
        keep = torch.as_tensor(src >= 0, device=q.device)
        padded = []
        for x in xs:
            y = x[:, idx]
            m = keep.view(1, -1, *([1] * (x.dim() - 2)))
            padded.append(torch.where(m, y, torch.zeros((), dtype=y.dtype, device=y.device)))
        rows = torch.as_tensor(dst, device=q.device)
    else:
        Tp = -(-T // C) * C
        padded = [torch.nn.functional.pad(x, (0, 0) * (x.dim() - 2) + (0, Tp - T)) for x in xs]
        rows = None
    qp, kp, vp, gp, bp = padded
    hf = lambda x: x.transpose(1, 2)          # noqa: E731  [B,T,H,D] -> [B,H,T,D]
    *_, aqk, akk = kda_intra_chunk_fwd(hf(qp), hf(kp), hf(gp), bp.transpose(1, 2), hf(vp),
                                       scale=scale, chunk_size=C)
    out = []
    for a in (aqk, akk):
        a = a.reshape(B, H, Tp, C).transpose(1, 2)
        out.append((a[:, rows] if rows is not None else a[:, :T]).contiguous())
    return out


def chunk_kda_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor,
                  beta: torch.Tensor, scale: float | None = None,
                  initial_state: torch.Tensor | None = None, output_final_state: bool = False,
                  cu_seqlens=None, chunk_size: int = 64):
    """Forward only (tops/ops/kda/chunk.py:25-190).  Returns (o, final_state, g_cumsum,
    Aqk, Akk_inv) as the reference: g_cumsum [B,T,H,K] is the chunk-local cumsum of g / ln 2
    at `chunk_size`; Aqk [B,T,H,C] (row t holds scale * sum_d q_td k_jd 2^(G_td - G_jd) for
    the tokens j of its chunk, j <= t) and Akk_inv [B,T,H,C] (the rows of (I + Akk)^-1,
    Akk_ij = beta_i sum_d k_id k_jd 2^(G_id - G_jd), j < i) are in k.dtype, per chunk of
    `chunk_size` (16, 32, 64 or 128).  o and final_state come from the fused kernels (64-row
    tiles; the same result up to fp32 rounding).  Unlike the reference, T need not be a
    multiple of chunk_size and cu_seqlens is honoured (each sequence chunked on its own)."""
    _check(q, k, v, g, beta, initial_state, cu_seqlens)
    C = int(chunk_size)
    if C not in (16, 32, 64, 128):
        raise NotImplementedError(f"tops-hip chunk_kda_fwd takes chunk_size 16, 32, 64 or 128, "
                                  f"got {C}")
    if scale is None:
        scale = q.shape[-1] ** -0.5
    q, k, v = (x.contiguous() for x in (q, k, v))
    g32 = g.contiguous().to(torch.float32)
    b32 = beta.contiguous().to(torch.float32)
    h0 = None if initial_state is None else initial_state.contiguous().to(torch.float32)
    plan = ChunkPlan.get(q.shape[0], q.shape[1], cu_seqlens, q.device)
    from .gate import kda_gate_chunk_cumsum
    with torch.no_grad():
        o, ht, _ = _fwd(q, k, v, g32, b32, h0, scale, output_final_state, plan, keep=False)
        g_cumsum = kda_gate_chunk_cumsum(g32, C, cu_seqlens)
        aqk, akk = _intra_matrices(q, k, v, g_cumsum, b32, float(scale), C, cu_seqlens)
    return o, ht, g_cumsum, aqk, akk
