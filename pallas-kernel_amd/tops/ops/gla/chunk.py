"""Chunked GLA on MI355X: drop-in for tops.ops.gla.chunk (tops/ops/gla/chunk.py).

`chunk_gla` keeps the reference signature (chunk.py:1207-1218) and is
differentiable: a torch.autograd.Function wires the fused HIP backward, the
MI355X counterpart of the custom_vjp the reference lacks for GLA.

Tensors are PyTorch-ROCm device tensors in the reference layout:
q, k [B,T,H,K]; v [B,T,H,V]; g [B,T,H,K] log-space gates; states [N,H,K,V].
q/k/v are float32 or bfloat16 (computed with fp32 accumulation; bf16 MFMA
operands split into hi+lo where a value is not bf16-exact), gates and states
float32.  `chunk_size` is accepted for signature compatibility: the kernels
always tile the sequence in chunks of 64, which gives the same result up to
fp32 rounding for any requested chunk size.

Gates: a per-token g runs the kernels' per-channel gate mode; g = None with a g_gamma
that is constant over (B, T) (a scalar, (H,), (1,1,H,1), (1,1,H,K) ...) runs their
constant-gate mode on g_gamma expanded to [H, K] (no [B,T,H,K] gate is built; no gate at
all is g_gamma = 0).  A g_gamma that varies over B or T is broadcast to a full gate, as the
reference broadcasts every g_gamma (chunk.py:1134-1138).
"""
from __future__ import annotations

import torch

from ...utils import ChunkPlan, cdiv, inference_inputs, to_device
from .._chunk_core import (GATE_K, GATE_GAMMA, GATE_GAMMA_K, PAIRED, check_qkv, paired_states,
                           pack_states, states_fp32, unpack_states, chunk_fwd as _core_fwd,
                           chunk_bwd as _core_bwd)


def _check(q, k, v, initial_state, cu_seqlens):
    check_qkv(q, k, v, initial_state, cu_seqlens, split_ok=True)


def _gate(q, g, g_gamma):
    """(mode, gate tensor) for the kernels: g [B,T,H,K] (GATE_K), or a constant [H,K]
    (GATE_GAMMA_K) that is a differentiable view of g_gamma."""
    B, T, H, K = q.shape
    if g is not None:
        assert tuple(g.shape) == (B, T, H, K), f"g shape {tuple(g.shape)} != {(B, T, H, K)}"
        return GATE_K, g
    if g_gamma is None:
        return GATE_GAMMA_K, torch.zeros(H, K, device=q.device, dtype=torch.float32)
    gg = torch.as_tensor(g_gamma, device=q.device)
    assert gg.dim() <= 4, f"g_gamma must broadcast to {(B, T, H, K)}, got {tuple(gg.shape)}"
    s4 = (1,) * (4 - gg.dim()) + tuple(gg.shape)
    g4 = gg.reshape(s4)
    if s4[0] == 1 and s4[1] == 1:
        return GATE_GAMMA_K, g4.expand(1, 1, H, K)[0, 0]
    return GATE_K, g4.to(torch.float32).expand(B, T, H, K)


class _ChunkGLA(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, gt, h0, mode, scale, output_final_state, cu_seqlens):
        q, k, v = (x.contiguous() for x in (q, k, v))
        g32 = gt.detach().contiguous().to(torch.float32)
        h032 = None if h0 is None else h0.contiguous().to(torch.float32)
        plan = ChunkPlan.get(q.shape[0], q.shape[1], cu_seqlens, q.device)
        train = any(ctx.needs_input_grad[:5])
        o, ht, hs = _core_fwd(q, k, v, (mode, g32), h032, scale, output_final_state, plan,
                              keep_states=PAIRED if train else False)
        if train:
            ctx.save_for_backward(q, k, v, g32, *pack_states(hs), h032)
            ctx.paired = paired_states(q, q.shape[-1], v.shape[-1])
            ctx.plan, ctx.scale, ctx.mode = plan, scale, mode
            ctx.g_dtype = gt.dtype
            ctx.h0_info = None if h0 is None else h0.dtype
        return o, ht

    @staticmethod
    def backward(ctx, do, dht):
        q, k, v, g32, hs, hsc, h032 = ctx.saved_tensors
        hs = unpack_states(hs, hsc)
        do = do.contiguous().to(q.dtype)
        dht = None if dht is None else dht.contiguous().to(torch.float32)
        want_dh0 = ctx.h0_info is not None
        want_dg = bool(ctx.needs_input_grad[3])
        dq, dk, dv, dg, dh0 = _core_bwd(q, k, v, (ctx.mode, g32), do, dht, hs, ctx.scale,
                                        ctx.plan, want_dh0, want_dg, h0=h032, paired=ctx.paired)
        if dh0 is not None:
            dh0 = dh0.to(ctx.h0_info)
        if dg is not None:
            if ctx.mode == GATE_GAMMA_K:
                dg = dg.sum(dim=(0, 1))            # the constant gate stands for every token
            dg = dg.to(ctx.g_dtype)
        return dq, dk, dv, dg, dh0, None, None, None, None


def chunk_gla(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor | None = None,
    g_gamma: torch.Tensor | None = None,
    scale: float | None = None,
    initial_state: torch.Tensor | None = None,
    output_final_state: bool = False,
    cu_seqlens=None,
    chunk_size: int = 16,
):
    """Chunked GLA (tops/ops/gla/chunk.py:1207-1271).

    Args follow the reference: g [B,T,H,K] per-step log gates, or g_gamma
    (broadcastable to [B,T,H,K], used only when g is None), else no decay;
    scale defaults to K^-0.5; initial_state [N,H,K,V]; cu_seqlens [N+1]
    (host or device ints, B must be 1).
    Returns (o [B,T,H,V] in q.dtype, final_state [N,H,K,V] fp32 or None).
    """
    assert chunk_size > 0, "chunk_size must be positive"
    K = q.shape[-1]
    mode, gt = _gate(q, g, g_gamma)
    if mode == GATE_GAMMA_K and not gt.requires_grad and (g_gamma is None or
                                                          torch.as_tensor(g_gamma).dim() == 0 or
                                                          torch.as_tensor(g_gamma).shape[-1] == 1):
        # no gate, or a constant shared by the K channels, and no gradient for it: the
        # one-decay-per-head mode (whose bf16 kernels keep q and k exact)
        mode, gt = GATE_GAMMA, gt[:, 0].contiguous()
    _check(q, k, v, initial_state, cu_seqlens)
    if scale is None:
        scale = K ** -0.5
    q, k, v, gt, initial_state = inference_inputs(q, k, v, gt, initial_state)
    o, ht = _ChunkGLA.apply(q, k, v, gt, initial_state, mode, float(scale),
                            bool(output_final_state), cu_seqlens)
    return o, (ht if output_final_state else None)


# ---------------------------------------------------------------------------------------
# Orchestrators with the reference's intermediate outputs
# ---------------------------------------------------------------------------------------

class _Padded:
    """The reference's padded layout (chunk.py:1140-1148, 768-824): T padded to a multiple of
    C, or (varlen) every sequence padded to a multiple of C.  `dest` maps each token row to
    its padded row; `cu` is the padded cu_seqlens (None for fixed length)."""

    def __init__(self, B, T, cu_seqlens, C, device):
        self.C = C
        if cu_seqlens is None:
            self.T = cdiv(T, C) * C
            self.dest = torch.arange(T, device=device)
            self.cu = None
        else:
            cu = [int(x) for x in (cu_seqlens.tolist() if isinstance(cu_seqlens, torch.Tensor)
                                   else cu_seqlens)]
            pcu = [0]
            for a, b in zip(cu[:-1], cu[1:]):
                pcu.append(pcu[-1] + cdiv(b - a, C) * C)
            self.T = pcu[-1]
            self.cu = pcu
            idx = [pcu[n] + i for n in range(len(cu) - 1) for i in range(cu[n + 1] - cu[n])]
            self.dest = to_device(idx, device, torch.int64)

    def pad(self, x):
        out = x.new_zeros((x.shape[0], self.T) + tuple(x.shape[2:]))
        out[:, self.dest] = x
        return out

    def unpad(self, x):
        return x[:, self.dest]


def _local_diff(g_cumsum, pad: _Padded):
    """The per-token gate of a chunk-local cumsum in the padded layout: g_t = G_t - G_{t-1}
    inside each chunk, G_0 at a chunk start (the inverse of chunk_local_cumsum)."""
    G = g_cumsum.to(torch.float32)
    B, Tp = G.shape[:2]
    prev = torch.zeros_like(G)
    prev[:, 1:] = G[:, :-1]
    first = (torch.arange(Tp, device=G.device) % pad.C) == 0
    prev[:, first] = 0
    return pad.unpad(G - prev)


def chunk_gla_fwd(q, k, v, g, g_gamma, g_cumsum, scale, initial_state, output_final_state,
                  cu_seqlens=None, chunk_size: int = 64):
    """Forward orchestrator (tops/ops/gla/chunk.py:1103-1199).  Returns (g_cumsum, A, h, ht, o)
    like the reference, in its padded layout (T padded to a multiple of chunk_size; varlen:
    every sequence padded):
      g_cumsum [B, Tp, H, K] fp32  the chunk-local gate cumsum (given, or computed: the
                                   analytic g_gamma * (i + 1) for a fixed-length g_gamma call,
                                   chunk.py:1155-1163)
      A        [B, Tp, H, C] fp32  the intra-chunk attention, full square (the consumer masks)
      h        [B, Tp / C, H, K, V] fp32  the state before every chunk
      ht       [N, H, K, V] fp32 or None;   o [B, T, H, V] in v.dtype (unpadded).
    A supplied g_cumsum (in that layout) stands for g: the per-token gate is its in-chunk
    difference.  o and ht come from the fused forward sweep; A, and h for chunk_size != 64,
    from the stage kernels (tops.ops.gla.stages)."""
    from .stages import chunk_gla_fwd_intra_gk, chunk_local_cumsum
    from ..common.chunk_h import _recurrence
    B, T, H, K = q.shape
    V = v.shape[-1]
    C = int(chunk_size)
    _check(q, k, v, initial_state, cu_seqlens)
    if scale is None:
        scale = K ** -0.5
    pad = _Padded(B, T, cu_seqlens, C, q.device)
    if g_cumsum is not None:
        assert tuple(g_cumsum.shape) == (B, pad.T, H, K), (
            f"g_cumsum must be {(B, pad.T, H, K)} (padded layout), got {tuple(g_cumsum.shape)}")
        mode, gt = GATE_K, _local_diff(g_cumsum, pad)
    else:
        mode, gt = _gate(q, g, g_gamma)
    plan = ChunkPlan.get(B, T, cu_seqlens, q.device)
    q, k, v = (x.contiguous() for x in (q, k, v))
    g32 = gt.detach().contiguous().to(torch.float32)
    h0 = None if initial_state is None else initial_state.contiguous().to(torch.float32)
    o, ht, hs = _core_fwd(q, k, v, (mode, g32), h0, scale, output_final_state, plan,
                          keep_states=C == 64)
    qp, kp = pad.pad(q), pad.pad(k)
    if g_cumsum is None:
        if mode == GATE_GAMMA_K and cu_seqlens is None:
            pos = (torch.arange(pad.T, device=q.device) % C + 1).to(torch.float32)
            g_cumsum = (g32[None, None] * pos[None, :, None, None]).expand(B, pad.T, H, K)
            g_cumsum = g_cumsum.contiguous()
        else:
            gfull = g32 if mode == GATE_K else g32.expand(B, T, H, K)
            g_cumsum = chunk_local_cumsum(pad.pad(gfull.contiguous()), C)
    g_cumsum = g_cumsum.to(torch.float32).contiguous()
    A = chunk_gla_fwd_intra_gk(qp, kp, g_cumsum, scale, chunk_size=C)
    if C == 64:
        h = states_fp32(hs).reshape(B if cu_seqlens is None else 1, -1, H, K, V)
    else:
        h, _ = _recurrence(kp, pad.pad(v), None, None, g_cumsum, h0, pad.cu, C, False, 1.0, 1,
                           torch.float32, False)
    return g_cumsum, A, h, ht, o


def chunk_gla_bwd(q, k, v, g, g_gamma, g_cumsum, scale, initial_state, h, A, do, dht,
                  cu_seqlens=None, chunk_size: int = 64):
    """Backward orchestrator (tops/ops/gla/chunk.py:832-997).

    Returns (dq, dk, dv, dg, dh0).  `h` may be the state checkpoints chunk_gla_fwd returns at
    chunk_size 64; otherwise they are recomputed.  A is not used (the kernels recompute it);
    g_cumsum (padded layout) stands for g when g and g_gamma are None.  A g_gamma caller gets
    dg sum-reduced to g_gamma's shape (chunk.py:987-995).  dh0 is returned when
    initial_state or dht is given (chunk.py:943)."""
    del A
    B, T, H, K = q.shape
    V = v.shape[-1]
    _check(q, k, v, initial_state, cu_seqlens)
    if g is None and g_gamma is None and g_cumsum is not None:
        g = _local_diff(g_cumsum, _Padded(B, T, cu_seqlens, int(chunk_size), q.device))
    mode, gt = _gate(q, g, g_gamma)
    plan = ChunkPlan.get(B, T, cu_seqlens, q.device)
    q, k, v = (x.contiguous() for x in (q, k, v))
    g32 = gt.detach().contiguous().to(torch.float32)
    h0 = None if initial_state is None else initial_state.contiguous().to(torch.float32)
    if h is None or int(chunk_size) != 64:
        _, _, hs = _core_fwd(q, k, v, (mode, g32), h0, scale, False, plan, keep_states=True)
    else:
        hs = h.reshape(plan.total, H, K, V).contiguous().to(torch.float32)
    want_dh0 = initial_state is not None or dht is not None
    dq, dk, dv, dg, dh0 = _core_bwd(q, k, v, (mode, g32), do.contiguous().to(q.dtype),
                                    None if dht is None else dht.contiguous().to(torch.float32),
                                    hs, scale, plan, want_dh0, True)
    if g is None and g_gamma is not None:
        gg = torch.as_tensor(g_gamma)
        if mode == GATE_GAMMA_K:
            dg = dg.sum(dim=(0, 1))
        dg = dg.sum_to_size(*gg.shape) if gg.dim() > 0 else dg.sum()
    return dq, dk, dv, dg, dh0


def chunk_gla_bwd_with_pl(q, k, v, g, g_gamma, g_cumsum, scale, initial_state, h, A, do, dht,
                          cu_seqlens=None, chunk_size: int = 64):
    """The reference's kernel-backed backward orchestrator (tops/ops/gla/chunk.py:1000-1095):
    the same contract as chunk_gla_bwd, including its asserts that T and the sequence
    boundaries are multiples of chunk_size (chunk.py:1032-1035).  Here both orchestrators run
    the same HIP backward."""
    C = int(chunk_size)
    assert q.shape[1] % C == 0, "T must be a multiple of chunk_size for chunk_gla_bwd_with_pl"
    if cu_seqlens is not None:
        cu = cu_seqlens.tolist() if isinstance(cu_seqlens, torch.Tensor) else list(cu_seqlens)
        assert all(int(x) % C == 0 for x in cu), (
            "cu_seqlens must be multiples of chunk_size for chunk_gla_bwd_with_pl")
    return chunk_gla_bwd(q, k, v, g, g_gamma, g_cumsum, scale, initial_state, h, A, do, dht,
                         cu_seqlens=cu_seqlens, chunk_size=chunk_size)
