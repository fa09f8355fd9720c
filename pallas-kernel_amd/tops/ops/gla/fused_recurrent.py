"""Fused recurrent GLA on MI355X: drop-in for tops.ops.gla.fused_recurrent
(tops/ops/gla/fused_recurrent.py) with the dtype contract of the reference's CPU tier
(tops/cpu/ops/gla/fused_recurrent.py:6-28, 362-422): o in q.dtype, ht fp32.

    h_t = h_{t-1} * exp(gk_t)[:, None] * exp(gv_t)[None, :] + k_t v_t^T
    o_t = h_t^T (scale * q_t)

`fused_recurrent_gla` is differentiable, covering gk, gv, reverse, initial_state and
cu_seqlens.  Two HIP implementations of the same recurrence are used:
  * without gv (the common case, and BASELINE config 2) the recurrence is computed
    chunkwise on MFMA by the chunk kernels (gla_sweep.hip, gla_dqkg.hip) -- the same
    sums, grouped by 64-token chunks.  reverse=True runs the same recurrence from the last
    token to the first (tops/cpu/ops/gla/fused_recurrent.py:116-160: one body, iterated
    backwards).  Without gradients that is the reverse chunk sweep itself
    (tops_chunk_reverse_fwd: the backward's state-gradient recurrence has the same form
    with q and k exchanged and the gate read one token later), reading the inputs in place;
    with gradients, or where the sweep would be split into sequence-parallel segments, it is
    the forward recurrence on every sequence's time-reversed inputs: the inputs are reversed
    per sequence, swept forward, and the output reversed back (the reversal is part of the
    autograd graph);
  * with gv and without gk (bf16, K, V <= 128), the forward runs chunkwise on the forward
    sweep with the gate applied per V column (tops_gla_chunk_fwd_gv); with gradients the
    backward is chunked too, on kernels of the same families (_GvChunk below);
  * otherwise with gv, the per-token kernels of gla_recurrent.hip (state in registers, one
    token at a time) run the forward, a replay + reverse backward and the gate-gradient
    suffix sums.
"""
from __future__ import annotations

import numpy as np
import torch

from ... import _native as N
from ...utils import ChunkPlan, inference_inputs, to_device


def _cu_dev(cu_seqlens, device):
    if cu_seqlens is None:
        return None
    return to_device(cu_seqlens, device, torch.int32).contiguous()


def _check(q, k, v, gk, gv, initial_state, cu_seqlens, wide_ok: bool = False):
    assert q.ndim == 4, f"q must be [B,T,H,K], got {tuple(q.shape)}"
    B, T, H, K = q.shape
    V = v.shape[-1]
    n = len(cu_seqlens) - 1 if cu_seqlens is not None else B
    assert tuple(k.shape) == (B, T, H, K), f"k shape {tuple(k.shape)} != expected {(B, T, H, K)}"
    assert v.ndim == 4 and tuple(v.shape[:3]) == (B, T, H), f"v shape {tuple(v.shape)} incompatible with q"
    assert gk is None or tuple(gk.shape) == (B, T, H, K), f"gk shape {tuple(gk.shape)} != expected {(B, T, H, K)}"
    assert gv is None or tuple(gv.shape) == (B, T, H, V), f"gv shape {tuple(gv.shape)} != expected {(B, T, H, V)}"
    assert initial_state is None or tuple(initial_state.shape) == (n, H, K, V), (
        f"initial_state shape {tuple(initial_state.shape)} != expected {(n, H, K, V)}")
    assert cu_seqlens is None or B == 1, f"cu_seqlens requires B=1, got B={B}"
    assert q.dtype == k.dtype == v.dtype, "q, k, v must share a dtype"
    if (K > 128 and not wide_ok) or K % 4:
        raise NotImplementedError(f"tops-hip fused recurrent kernels need K <= 128, K % 4 == 0 (got K={K})")
    N.require_cuda(q, k, v, gk, gv, initial_state)
    return B, T, H, K, V, n


def _k_slices(K: int):
    """Equal K slices of at most 128, multiples of 4 (None when K does not split so)."""
    n = -(-K // 128)
    return None if K % n or (K // n) % 4 else [slice(i * (K // n), (i + 1) * (K // n))
                                              for i in range(n)]


def _sliced(q, k, v, gk, gv, scale, initial_state, output_final_state, reverse, cu_seqlens):
    """fused_recurrent_gla for K > 128 or fp16 inputs, in fp32: every state entry has its own
    recurrence, so the output is the sum of the K slices' outputs and the final state their
    concatenation; autograd runs through the same slicing."""
    K = q.shape[-1]
    ks = _k_slices(K) if K > 128 else [slice(0, K)]
    if ks is None:
        raise NotImplementedError(f"tops-hip fused recurrent kernels need K <= 128 or K in equal "
                                  f"slices of at most 128, multiples of 4 (got K={K})")
    f32 = torch.float32
    q, k, v, gk, gv, initial_state = inference_inputs(q, k, v, gk, gv, initial_state)
    qf, kf, vf = (x.to(f32) for x in (q, k, v))
    o, hts = None, []
    for sl in ks:
        h0s = None if initial_state is None else initial_state[:, :, sl]
        os_, hs_ = _FusedRecurrentGLA.apply(qf[..., sl], kf[..., sl], vf,
                                            None if gk is None else gk[..., sl], gv, h0s,
                                            float(scale), bool(output_final_state), bool(reverse),
                                            cu_seqlens)
        o = os_ if o is None else o + os_
        hts.append(hs_)
    ht = torch.cat(hts, dim=2) if output_final_state else None
    return o.to(q.dtype), ht


def _f32(x):
    return None if x is None else x.contiguous().to(torch.float32)


def _fwd(q, k, v, gk32, gv32, h032, scale, output_final_state, reverse, cu, n, want_o32):
    B, T, H, K = q.shape
    V = v.shape[-1]
    o = torch.empty_like(v)
    o32 = torch.empty(B, T, H, V, device=q.device, dtype=torch.float32) if want_o32 else None
    ht = torch.empty(n, H, K, V, device=q.device, dtype=torch.float32) if output_final_state else None
    N.call("tops_gla_fused_recurrent_fwd", N.ptr(q), N.ptr(k), N.ptr(v), N.ptr(gk32), N.ptr(gv32),
           N.ptr(h032), N.ptr(o), N.ptr(o32), N.ptr(ht), N.ptr(cu), B, T, H, K, V, n,
           N.dtype_code(q.dtype), float(scale), int(bool(reverse)), N.stream())
    return o, o32, ht


def _bwd(q, k, v, gk32, gv32, o32, do, dht32, h032, scale, reverse, cu, n):
    B, T, H, K = q.shape
    V = v.shape[-1]
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    dgk = torch.empty(B, T, H, K, device=q.device, dtype=torch.float32) if gk32 is not None else None
    dgv = torch.empty(B, T, H, V, device=q.device, dtype=torch.float32) if gv32 is not None else None
    dh0 = torch.empty(n, H, K, V, device=q.device, dtype=torch.float32) if h032 is not None else None
    ws_bytes = N.lib().tops_gla_fused_recurrent_bwd_workspace(B, T, H, K, V, n,
                                                              int(gv32 is not None))
    ws = torch.empty((ws_bytes + 3) // 4, device=q.device, dtype=torch.float32)
    N.call("tops_gla_fused_recurrent_bwd", N.ptr(q), N.ptr(k), N.ptr(v), N.ptr(gk32), N.ptr(gv32),
           N.ptr(o32), N.ptr(do), N.ptr(dht32), N.ptr(h032), N.ptr(dq), N.ptr(dk), N.ptr(dv),
           N.ptr(dgk), N.ptr(dgv), N.ptr(dh0), N.ptr(ws), N.ptr(cu), B, T, H, K, V, n,
           N.dtype_code(q.dtype), float(scale), int(bool(reverse)), N.stream())
    return dq, dk, dv, dgk, dgv, dh0


class _FusedRecurrentGLA(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, gk, gv, h0, scale, output_final_state, reverse, cu_seqlens):
        q, k, v = (x.contiguous() for x in (q, k, v))
        gk32, gv32, h032 = _f32(gk), _f32(gv), _f32(h0)
        cu = _cu_dev(cu_seqlens, q.device)
        n = len(cu_seqlens) - 1 if cu_seqlens is not None else q.shape[0]
        train = any(ctx.needs_input_grad[:6])
        o, o32, ht = _fwd(q, k, v, gk32, gv32, h032, scale, output_final_state, reverse, cu, n,
                          want_o32=train and gv is not None)
        if train:
            ctx.save_for_backward(q, k, v, gk32, gv32, h032, o32)
            ctx.meta = (scale, reverse, cu, n)
            ctx.dtypes = tuple(None if x is None else x.dtype for x in (gk, gv, h0))
        return o, ht

    @staticmethod
    def backward(ctx, do, dht):
        q, k, v, gk32, gv32, h032, o32 = ctx.saved_tensors
        scale, reverse, cu, n = ctx.meta
        dq, dk, dv, dgk, dgv, dh0 = _bwd(q, k, v, gk32, gv32, o32, do.contiguous().to(q.dtype),
                                         _f32(dht), h032, scale, reverse, cu, n)
        gdt, vdt, hdt = ctx.dtypes
        dgk = None if dgk is None else dgk.to(gdt)
        dgv = None if dgv is None else dgv.to(vdt)
        dh0 = None if dh0 is None else dh0.to(hdt)
        return dq, dk, dv, dgk, dgv, dh0, None, None, None, None


def _chunked(gv, reverse, K, V):
    """Whether the chunk (MFMA) kernels compute this call (reverse=True through a per-sequence
    time reversal)."""
    del reverse
    return gv is None and K % 8 == 0 and V % 8 == 0 and V <= 128


def time_reversal(T: int, cu_seqlens, device):
    """Index that reverses every sequence in time: [T] for fixed length (applied per batch
    row), the packed varlen layout otherwise.  Its own inverse."""
    if cu_seqlens is None:
        return torch.arange(T - 1, -1, -1, device=device)
    cu = [int(x) for x in (cu_seqlens.tolist() if isinstance(cu_seqlens, torch.Tensor) else cu_seqlens)]
    idx = [cu[n] + cu[n + 1] - 1 - t for n in range(len(cu) - 1) for t in range(cu[n], cu[n + 1])]
    return to_device(np.asarray(idx, np.int64), device, torch.int64)


_REV_GATE_CODE = {"k": 0, "s": 1, "gamma": 2}


def reverse_chunk_native(q, k, v, mode, g, initial_state, scale, output_final_state, cu_seqlens):
    """The reverse-time recurrence on the reverse chunk sweep (tops_chunk_reverse_fwd), for
    calls that need no gradient.  mode: "k" (g [B,T,H,K]), "s" (g [B,T,H]) or "gamma"
    (g [H], a constant log-gate per head).  Returns (o, ht or None), or None where it does
    not apply: gradients wanted, dtypes or shapes the kernel does not take, or a call whose
    sequences the chunk kernels would split into sequence-parallel segments (the time-reversal
    route keeps that split)."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad
                                       for t in (q, k, v, g, initial_state)):
        return None
    if q.dtype not in (torch.float32, torch.bfloat16) or K > 128 or K % 8 or V % 8:
        return None
    plan = ChunkPlan(B, T, cu_seqlens, q.device)
    if plan.segments(H, V) is not None:
        return None
    q, k, v = (x.contiguous() for x in (q, k, v))
    gt = g.contiguous().to(torch.float32)
    o = torch.empty_like(v)
    ht = torch.empty(plan.N, H, K, V, device=q.device, dtype=torch.float32) \
        if output_final_state else None
    N.call("tops_chunk_reverse_fwd", N.ptr(q), N.ptr(k), N.ptr(v), N.ptr(gt), _REV_GATE_CODE[mode],
           N.ptr(_f32(initial_state)), N.ptr(o), N.ptr(ht), N.ptr(plan.cu_dev), B, T, H, K, V,
           plan.N, N.dtype_code(q.dtype), float(scale), N.stream())
    return o, ht


def gv_chunk_native(q, k, v, gv, initial_state, scale, output_final_state, cu_seqlens):
    """The value-gated forward (gv, no gk) on the chunk sweep (tops_gla_chunk_fwd_gv), for
    calls that need no gradient.  Returns (o, ht or None), or None where it does not apply:
    gradients wanted, inputs other than bf16, K > 128 or K, V not multiples of 8, or a call
    whose sequences the chunk kernels would split into sequence-parallel segments."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad
                                       for t in (q, k, v, gv, initial_state)):
        return None
    if q.dtype != torch.bfloat16 or K > 128 or K % 8 or V % 8:
        return None
    plan = ChunkPlan(B, T, cu_seqlens, q.device)
    if plan.segments(H, V) is not None:
        return None
    q, k, v = (x.contiguous() for x in (q, k, v))
    o = torch.empty_like(v)
    ht = torch.empty(plan.N, H, K, V, device=q.device, dtype=torch.float32) \
        if output_final_state else None
    N.call("tops_gla_chunk_fwd_gv", N.ptr(q), N.ptr(k), N.ptr(v), N.ptr(_f32(gv)),
           N.ptr(_f32(initial_state)), N.ptr(o), N.ptr(ht), N.ptr(plan.cu_dev), B, T, H, K, V,
           plan.N, N.dtype_code(q.dtype), float(scale), N.stream())
    return o, ht


def _gv_chunk_train_ok(q, v, gk, gv, reverse, cu_seqlens):
    """Whether a gv-only call with gradients runs on the chunk kernels (_GvChunk): bf16, K and
    V <= 128 and multiples of 8.  Its value-gate and reverse sweeps take whole sequences (no
    sequence-parallel split); for a few long sequences that leaves CUs idle, still far ahead
    of the per-token kernels."""
    if gv is None or gk is not None or reverse or q.dtype != torch.bfloat16:
        return False
    K = q.shape[-1]
    V = v.shape[-1]
    return K <= 128 and V <= 128 and K % 8 == 0 and V % 8 == 0


class _GvChunk(torch.autograd.Function):
    """fused_recurrent_gla with gv and without gk, forward and backward on chunk kernels
    (gradients of tops/ops/gla/fused_recurrent.py:496-619).  With S_t = S_(t-1) diag(a_t) +
    k_t v_t^T (a_t = exp(gv_t)), o_t = scale S_t^T q_t and dS_t the gradient reaching S_t:
      * dq_t = scale S_t dO_t.  S^T follows the key-gated recurrence S^T_t = diag(a_t) S^T_(t-1)
        + v_t k_t^T, so dq is the key-gated chunk forward with queries dO, keys v, values k,
        gate gv and initial state h0^T;
      * dk_t = dS_t v_t, dS^T_t = diag(a_(t+1)) dS^T_(t+1) + scale dO_t q_t^T: the state-gradient
        sweep of the key-gated chunk backward (tops_gla_chunk_rev_dv) with queries dO, keys v,
        output-gradient q and dht^T, whose dv is dk;
      * dv_t = dS_t^T k_t and dh0 = dS_1 diag(a_1): the value-gated state-gradient sweep
        (tops_gla_chunk_bwd_dv_gv32, dv in fp32);
      * dgv_t = sum over t' >= t of (o_t' dO_t' - v_t' dv_t') + sum_k (dht * ht)[k, :], the
        per-column identity of the gated recurrence (o in fp32 from the forward), by
        tops_gv_gate_grad."""

    @staticmethod
    def forward(ctx, q, k, v, gv, h0, scale, cu_seqlens):
        B, T, H, K = q.shape
        V = v.shape[-1]
        plan = ChunkPlan(B, T, cu_seqlens, q.device)
        q, k, v = (x.contiguous() for x in (q, k, v))
        gv32, h032 = _f32(gv), _f32(h0)
        o32 = torch.empty(B, T, H, V, device=q.device, dtype=torch.float32)
        o = torch.empty(B, T, H, V, device=q.device, dtype=q.dtype)
        ht = torch.empty(plan.N, H, K, V, device=q.device, dtype=torch.float32)
        N.call("tops_gla_chunk_fwd_gv32", N.ptr(q), N.ptr(k), N.ptr(v), N.ptr(gv32), N.ptr(h032),
               N.ptr(o32), N.ptr(o), N.ptr(ht), N.ptr(plan.cu_dev), B, T, H, K, V, plan.N,
               N.dtype_code(q.dtype), float(scale), N.stream())
        ctx.save_for_backward(q, k, v, gv32, h032, o32, ht)
        ctx.scale, ctx.cu = scale, cu_seqlens
        ctx.dtypes = (gv.dtype, None if h0 is None else h0.dtype)
        # an unused output hands backward None instead of zeros: no final-state term to form
        # when ht takes no part in the loss
        ctx.set_materialize_grads(False)
        return o, ht

    @staticmethod
    def backward(ctx, do, dht):
        from .chunk import chunk_gla
        q, k, v, gv, h0, o32, ht = ctx.saved_tensors
        scale, cu = ctx.scale, ctx.cu
        B, T, H, K = q.shape
        V = v.shape[-1]
        dev = q.device
        plan = ChunkPlan(B, T, cu, dev)
        if do is None:
            do = torch.zeros(B, T, H, V, device=dev, dtype=q.dtype)
        do = do.contiguous().to(q.dtype)
        dht32 = None if dht is None else dht.to(torch.float32).contiguous()
        # dq: the key-gated forward on the transposed state
        h0t = None if h0 is None else h0.transpose(-1, -2).contiguous()
        dq, _ = chunk_gla(do, v, k, gv, scale=scale, initial_state=h0t, output_final_state=False,
                          cu_seqlens=cu)
        # dk: the key-gated state-gradient sweep on the transposed state gradient (its dv)
        dk = torch.empty_like(q)
        dht_t = None if dht32 is None else dht32.transpose(-1, -2).contiguous()   # [N, H, V, K]
        N.call("tops_gla_chunk_rev_dv", N.ptr(do), N.ptr(v), N.ptr(gv), N.ptr(q), N.ptr(dht_t),
               N.ptr(dk), None, N.ptr(plan.cu_dev), B, T, H, V, K, plan.N,
               N.dtype_code(q.dtype), float(scale), N.stream())
        # dv (fp32) and dh0: the value-gated state-gradient sweep
        dv32 = torch.empty(B, T, H, V, device=dev, dtype=torch.float32)
        dh0 = None if h0 is None else torch.empty_like(h0)
        N.call("tops_gla_chunk_bwd_dv_gv32", N.ptr(q), N.ptr(k), N.ptr(do), N.ptr(gv), N.ptr(dht32),
               N.ptr(dv32), N.ptr(dh0), N.ptr(plan.cu_dev), B, T, H, K, V, plan.N,
               N.dtype_code(q.dtype), float(scale), N.stream())
        # dgv: suffix sums of o dO - v dv, plus the final state's term (tops_gv_gate_grad)
        c = None if dht32 is None else (dht32 * ht).sum(-2).contiguous()      # [N, H, V]
        # and the bf16 dv, rounded from dv32 on the same walk
        dgv = torch.empty(B, T, H, V, device=dev, dtype=torch.float32)
        dv = torch.empty(B, T, H, V, device=dev, dtype=v.dtype)
        N.call("tops_gv_gate_grad", N.ptr(o32), N.ptr(do), N.ptr(v), N.ptr(dv32), N.ptr(c),
               N.ptr(dgv), N.ptr(dv), N.ptr(plan.cu_dev), B, T, H, V, plan.N,
               N.dtype_code(q.dtype), N.stream())
        gdt, hdt = ctx.dtypes
        return (dq, dk, dv, dgv.to(gdt), None if dh0 is None else dh0.to(hdt),
                None, None)


DECODE_MAX_TOKENS = 4    # beyond this the chunk kernels are faster (measured at K = V = 128)


def longest_sequence(T, cu_seqlens):
    """Tokens in the longest sequence of a call (T for fixed length).  Reads cu_seqlens on
    the host (a device tensor is copied back, which synchronises its stream)."""
    if cu_seqlens is None:
        return T
    cu = cu_seqlens.tolist() if isinstance(cu_seqlens, torch.Tensor) else list(cu_seqlens)
    return max((cu[i + 1] - cu[i] for i in range(len(cu) - 1)), default=0)


def decode_sized(T, cu_seqlens) -> bool:
    """Whether a call is a batch of decode steps: sequences of at most DECODE_MAX_TOKENS
    tokens.  Boundaries in host memory (a list, an array, a CPU tensor) are read exactly.
    A device tensor is not read back, since that would synchronise the stream ahead of the
    launch on every step; its mean length T / N stands in for the longest.  The decode
    kernel is exact at any length (it walks a sequence token by token), so that estimate
    only decides which kernel is faster."""
    if isinstance(cu_seqlens, torch.Tensor) and cu_seqlens.device.type != "cpu":
        n = cu_seqlens.numel() - 1
        return n > 0 and T <= DECODE_MAX_TOKENS * n
    return longest_sequence(T, cu_seqlens) <= DECODE_MAX_TOKENS


def decode_native(q, k, v, gk, gv, initial_state, scale, output_final_state, reverse, cu_seqlens):
    """Sequences of at most DECODE_MAX_TOKENS tokens (decode steps against a state cache) on
    the register-state kernel (tops_gla_fused_recurrent_fwd_decode), for calls that need no
    gradient: it reads h0 and writes ht once, with no per-chunk staging.  Returns (o, ht or
    None), or None where it does not apply (gradients wanted, dtypes other than fp32 / bf16,
    K > 128 or K % 4, a longer sequence)."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad
                                       for t in (q, k, v, gk, gv, initial_state)):
        return None
    if q.dtype not in (torch.float32, torch.bfloat16) or K > 128 or K % 4:
        return None
    n = B if cu_seqlens is None else len(cu_seqlens) - 1
    if not decode_sized(T, cu_seqlens):
        return None
    q, k, v = (x.contiguous() for x in (q, k, v))
    o = torch.empty_like(v)
    ht = torch.empty(n, H, K, V, device=q.device, dtype=torch.float32) if output_final_state else None
    N.call("tops_gla_fused_recurrent_fwd_decode", N.ptr(q), N.ptr(k), N.ptr(v), N.ptr(_f32(gk)),
           N.ptr(_f32(gv)), N.ptr(_f32(initial_state)), N.ptr(o), None, N.ptr(ht),
           N.ptr(_cu_dev(cu_seqlens, q.device)), B, T, H, K, V, n, N.dtype_code(q.dtype),
           float(scale), int(bool(reverse)), N.stream())
    return o, ht


def _reversed_chunk(fn, q, k, v, g, cu_seqlens, **kw):
    """fn (a chunk op) on the time-reversed sequences; returns (o in original order, ht)."""
    rev = time_reversal(q.shape[1], cu_seqlens, q.device)
    flip = (lambda x: None if x is None else x.index_select(1, rev))
    o, ht = fn(flip(q), flip(k), flip(v), flip(g), cu_seqlens=cu_seqlens, **kw)
    return flip(o), ht


def fused_recurrent_gla(q, k, v, gk=None, gv=None, scale=None, initial_state=None,
                        output_final_state=False, reverse=False, cu_seqlens=None):
    """tops/ops/gla/fused_recurrent.py:439-482 (CPU dtype contract: o in q.dtype).
    Returns (o [B,T,H,V], ht [N,H,K,V] fp32 or None)."""
    B, T, H, K, V, n = _check(q, k, v, gk, gv, initial_state, cu_seqlens, wide_ok=True)
    wide = K > 128 or q.dtype not in (torch.float32, torch.bfloat16)
    if scale is None:
        scale = K ** -0.5
    r = decode_native(q, k, v, gk, gv, initial_state, scale, output_final_state, reverse, cu_seqlens)
    if r is not None:
        return r
    if reverse and gv is None:
        r = reverse_chunk_native(q, k, v, "k" if gk is not None else "gamma",
                                 gk if gk is not None else torch.zeros(H, device=q.device),
                                 initial_state, scale, output_final_state, cu_seqlens)
        if r is not None:
            return r
    if gv is not None and gk is None and not reverse:
        r = gv_chunk_native(q, k, v, gv, initial_state, scale, output_final_state, cu_seqlens)
        if r is not None:
            return r
        if _gv_chunk_train_ok(q, v, gk, gv, reverse, cu_seqlens):
            o, ht = _GvChunk.apply(q, k, v, gv, initial_state, float(scale), cu_seqlens)
            return o, (ht if output_final_state else None)
    if wide and not _chunked(gv, reverse, K, V):
        return _sliced(q, k, v, gk, gv, scale, initial_state, output_final_state, reverse,
                       cu_seqlens)
    if _chunked(gv, reverse, K, V):
        from .chunk import chunk_gla
        if reverse:
            return _reversed_chunk(
                lambda q_, k_, v_, g_, **kw: chunk_gla(q_, k_, v_, g_, **kw), q, k, v, gk,
                cu_seqlens, scale=scale, initial_state=initial_state,
                output_final_state=output_final_state)
        return chunk_gla(q, k, v, gk, scale=scale, initial_state=initial_state,
                         output_final_state=output_final_state, cu_seqlens=cu_seqlens)
    q, k, v, gk, gv, initial_state = inference_inputs(q, k, v, gk, gv, initial_state)
    o, ht = _FusedRecurrentGLA.apply(q, k, v, gk, gv, initial_state, float(scale),
                                     bool(output_final_state), bool(reverse), cu_seqlens)
    return o, (ht if output_final_state else None)


def fused_recurrent_gla_norm_gate(q, k, v, gk=None, gv=None, g=None, weight=None,
                                  eps: float = 1e-5, scale=None, initial_state=None,
                                  output_final_state=False, reverse=False, cu_seqlens=None):
    """The decode route of the reference's GLA layer as one op: fused_recurrent_gla followed by
    the layer's output norm over head_v_dim,
        y = o / sqrt(mean_v(o^2) + eps) * weight * silu(g)
    (FusedRMSNormGated, tops/modules/fused_norm_gate.py:6-37, applied at
    tops/layers/gla.py:330-336 after fused_recurrent_gla at :288-297; with g None, the layer's
    RMSNorm branch, tops/modules/layernorm.py:6-35).

    q, k, v, gk, gv, scale, initial_state, output_final_state, reverse, cu_seqlens: as
    fused_recurrent_gla.  g [B,T,H,V] (the output gate, per head) or None; weight [V] or None.
    Returns (y [B,T,H,V] in q.dtype, final state [N,H,K,V] fp32 or None).

    Decode steps (every sequence at most 4 tokens) that need no gradient, with V <= 128 and g
    in q's dtype, run as one kernel (tops_gla_fused_recurrent_fwd_decode_norm_gate): the norm
    is the epilogue of the recurrence, on o in fp32, and o itself never reaches HBM.  Other
    calls compose fused_recurrent_gla and the standalone norm kernel (differentiable)."""
    B, T, H, K, V, n = _check(q, k, v, gk, gv, initial_state, cu_seqlens, wide_ok=True)
    assert g is None or tuple(g.shape) == (B, T, H, V), \
        f"g shape {tuple(g.shape)} != expected {(B, T, H, V)}"
    assert weight is None or tuple(weight.shape) == (V,), \
        f"weight shape {tuple(weight.shape)} != expected {(V,)}"
    if scale is None:
        scale = K ** -0.5
    grads = torch.is_grad_enabled() and any(
        t is not None and t.requires_grad for t in (q, k, v, gk, gv, g, weight, initial_state))
    fused = (not grads and V <= 128 and K <= 128 and K % 4 == 0
             and q.dtype in (torch.float32, torch.bfloat16)
             and (g is None or g.dtype == q.dtype) and decode_sized(T, cu_seqlens))
    if not fused:
        from ...modules.layernorm import rms_norm_gated
        o, ht = fused_recurrent_gla(q, k, v, gk, gv, scale=scale, initial_state=initial_state,
                                    output_final_state=output_final_state, reverse=reverse,
                                    cu_seqlens=cu_seqlens)
        return rms_norm_gated(o, g, weight, eps), ht
    q, k, v = (x.contiguous() for x in (q, k, v))
    y = torch.empty_like(v)
    ht = torch.empty(n, H, K, V, device=q.device, dtype=torch.float32) if output_final_state else None
    N.call("tops_gla_fused_recurrent_fwd_decode_norm_gate", N.ptr(q), N.ptr(k), N.ptr(v),
           N.ptr(_f32(gk)), N.ptr(_f32(gv)), N.ptr(_f32(initial_state)),
           N.ptr(None if g is None else g.contiguous()), N.ptr(_f32(weight)), float(eps),
           N.ptr(y), N.ptr(ht), N.ptr(_cu_dev(cu_seqlens, q.device)), B, T, H, K, V, n,
           N.dtype_code(q.dtype), float(scale), int(bool(reverse)), N.stream())
    return y, ht


def fused_recurrent_gla_conv_norm_gate(x_q, x_k, x_v, conv_weights, conv_biases=None,
                                       conv_caches=None, conv_activation="silu", gk=None, g=None,
                                       weight=None, eps: float = 1e-5, scale=None,
                                       initial_state=None, output_final_state=False,
                                       cu_seqlens=None):
    """The reference GLA layer's decode route from its projections to the normalised output
    (tops/layers/gla.py:236-262, 288-297, 330-336), as one op:
        q, k, v = ShortConvolution(x_q), (x_k), (x_v)    (tops/modules/convolution.py:44-173)
        o, ht = fused_recurrent_gla(q, k, v, gk, initial_state, output_final_state)
        y = RMSNorm(o) * weight * silu(g)                 (tops/modules/fused_norm_gate.py:6-37)

    x_q, x_k [B,T,H,K] and x_v [B,T,H,V]: the q / k / v projections before their
    convolutions; conv_weights (w_q, w_k, w_v), each [D,1,W] or [D,W] (D = H*K, H*K, H*V);
    conv_biases (b_q, b_k, b_v) or None; conv_caches (c_q, c_k, c_v), each [N,D,W], or None;
    conv_activation "silu" / "swish" / None; gk [B,T,H,K] log gates; g [B,T,H,V] or None;
    weight [V] or None.  As in the layer, a call with one token per sequence (B*T == N) is a
    conv decode step (the caches roll by one token), any other call a prefill (the caches are
    not read, the new ones are the last W inputs).  Returns (y [B,T,H,V], final state
    [N,H,K,V] fp32 or None, (c_q, c_k, c_v) or None): y in the dtype the layer's route gives
    (the promotion of x and the conv weights).

    Without gradients, with every sequence at most 4 tokens, K <= 128, V <= 128 and no
    num_kv_groups repeat, it runs as one kernel (tops_gla_decode_conv_norm_gate): the
    convolutions are the decode kernel's token staging, the norm its epilogue; q, k, v and o
    never reach HBM.  Other calls compose short_conv / short_conv_step,
    fused_recurrent_gla and the norm kernel (differentiable)."""
    from ...modules.convolution import _act, short_conv, short_conv_step
    B, T, H, K = x_q.shape
    V = x_v.shape[-1]
    assert tuple(x_k.shape) == (B, T, H, K) and x_v.ndim == 4 and tuple(x_v.shape[:3]) == (B, T, H), \
        "x_q, x_k [B,T,H,K] and x_v [B,T,H,V] expected"
    n = B if cu_seqlens is None else len(cu_seqlens) - 1
    ws = [w.reshape(w.shape[0], -1) for w in conv_weights]
    W = ws[0].shape[1]
    dims = (H * K, H * K, H * V)
    for w, D in zip(ws, dims):
        assert tuple(w.shape) == (D, W), f"conv weight shape {tuple(w.shape)} != {(D, W)}"
    bs = tuple(conv_biases) if conv_biases is not None else (None, None, None)
    cs = tuple(conv_caches) if conv_caches is not None else (None, None, None)
    step = B * T == n
    ydt = torch.promote_types(x_q.dtype, ws[0].dtype)
    if ydt not in (torch.float32, torch.bfloat16):
        ydt = torch.float32
    grads = torch.is_grad_enabled() and any(
        t is not None and t.requires_grad
        for t in (x_q, x_k, x_v, gk, g, weight, initial_state, *conv_weights, *bs))
    fused = (not grads and V <= 128 and K <= 128 and K % 4 == 0 and 1 <= W <= 8
             and x_q.dtype in (torch.float32, torch.bfloat16)
             and x_q.dtype == x_k.dtype == x_v.dtype
             and (g is None or g.dtype == x_q.dtype) and decode_sized(T, cu_seqlens))
    if scale is None:
        scale = K ** -0.5
    if not fused:
        outs, new = [], []
        for x, w, b, c, D in zip((x_q, x_k, x_v), conv_weights, bs, cs, dims):
            x3 = x.reshape(B, T, D)
            if step:
                y3, c2 = short_conv_step(x3, w, b, conv_activation, c, output_final_state,
                                         cu_seqlens)
            else:
                y3, c2 = short_conv(x3, w, b, conv_activation, cu_seqlens, output_final_state)
            outs.append(y3.reshape(x.shape))
            new.append(c2)
        y, ht = fused_recurrent_gla_norm_gate(*outs, gk, None, g, weight, eps, scale=scale,
                                              initial_state=initial_state,
                                              output_final_state=output_final_state,
                                              cu_seqlens=cu_seqlens)
        return y, ht, (tuple(new) if any(c is not None for c in new) else None)
    xs = [x.contiguous() for x in (x_q, x_k, x_v)]
    dev = x_q.device
    w32 = [w.to(torch.float32).contiguous() for w in ws]
    b32 = [None if b is None else b.to(torch.float32).contiguous() for b in bs]
    # a decode step reads and rolls the caches; a prefill reads none and keeps the last W inputs
    keep = output_final_state or (step and cs[0] is not None)
    cin = [None if (c is None or not step) else c.to(torch.float32).contiguous() for c in cs]
    cout = [torch.empty(n, D, W, device=dev, dtype=torch.float32) if keep else None for D in dims]
    y = torch.empty(B, T, H, V, device=dev, dtype=ydt)
    ht = torch.empty(n, H, K, V, device=dev, dtype=torch.float32) if output_final_state else None
    N.call("tops_gla_decode_conv_norm_gate", *(N.ptr(x) for x in xs), *(N.ptr(w) for w in w32),
           *(N.ptr(b) for b in b32), *(N.ptr(c) for c in cin), *(N.ptr(c) for c in cout), W,
           _act(conv_activation), N.ptr(_f32(gk)), N.ptr(_f32(initial_state)),
           N.ptr(None if g is None else g.contiguous()), N.ptr(_f32(weight)), float(eps), N.ptr(y),
           int(ydt == torch.float32 and x_q.dtype != torch.float32), N.ptr(ht),
           N.ptr(_cu_dev(cu_seqlens, dev)), B, T, H, K, V, n, N.dtype_code(x_q.dtype),
           float(scale), N.stream())
    new = None
    if keep:
        # cache dtypes as the module gives them: a step keeps the cache's, a prefill x's
        new = tuple(co.to(c.dtype if (step and c is not None) else (torch.float32 if step else x.dtype))
                    for co, c, x in zip(cout, cs, (x_q, x_k, x_v)))
    return y, ht, new


def fused_recurrent_gla_fwd(q, k, v, gk=None, gv=None, scale=None, initial_state=None,
                            output_final_state=False, reverse=False, cu_seqlens=None):
    """tops/ops/gla/fused_recurrent.py:380-431.  Returns (o, ht), o in q.dtype."""
    B, T, H, K, V, n = _check(q, k, v, gk, gv, initial_state, cu_seqlens)
    if scale is None:
        scale = K ** -0.5
    r = decode_native(q, k, v, gk, gv, initial_state, scale, output_final_state, reverse, cu_seqlens)
    if r is not None:
        return r
    if _chunked(gv, reverse, K, V) and not reverse:
        from .chunk import chunk_gla
        return chunk_gla(q, k, v, gk, scale=scale, initial_state=initial_state,
                         output_final_state=output_final_state, cu_seqlens=cu_seqlens)
    if reverse and gv is None:
        r = reverse_chunk_native(q, k, v, "k" if gk is not None else "gamma",
                                 gk if gk is not None else torch.zeros(H, device=q.device),
                                 initial_state, scale, output_final_state, cu_seqlens)
        if r is not None:
            return r
    if gv is not None and gk is None and not reverse:
        r = gv_chunk_native(q, k, v, gv, initial_state, scale, output_final_state, cu_seqlens)
        if r is not None:
            return r
    o, _, ht = _fwd(q.contiguous(), k.contiguous(), v.contiguous(), _f32(gk), _f32(gv),
                    _f32(initial_state), scale, output_final_state, reverse,
                    _cu_dev(cu_seqlens, q.device), n, want_o32=False)
    return o, ht


def fused_recurrent_gla_bwd(q, k, v, gk=None, gv=None, o=None, do=None, dht=None, scale=None,
                            initial_state=None, reverse=False, cu_seqlens=None):
    """tops/ops/gla/fused_recurrent.py:881-958.  Returns (dq, dk, dv, dgk, dgv, dh0):
    dq/dk/dv in the input dtype, dgk/dgv fp32 (None without the gate), dh0 fp32 (None
    without initial_state).  `o` (the forward output) is required when gv is given."""
    B, T, H, K, V, n = _check(q, k, v, gk, gv, initial_state, cu_seqlens)
    assert do is not None and tuple(do.shape) == (B, T, H, V)
    assert dht is None or tuple(dht.shape) == (n, H, K, V)
    assert gv is None or o is not None, "o (forward output) is required when gv is used"
    if scale is None:
        scale = K ** -0.5
    if _chunked(gv, reverse, K, V) and not reverse:
        from .chunk import chunk_gla_bwd
        dq, dk, dv, dg, dh0 = chunk_gla_bwd(q, k, v, gk, None, None, scale, initial_state, None,
                                            None, do, dht, cu_seqlens=cu_seqlens)
        return dq, dk, dv, (dg if gk is not None else None), None, \
            (dh0 if initial_state is not None else None)
    return _bwd(q.contiguous(), k.contiguous(), v.contiguous(), _f32(gk), _f32(gv), _f32(o),
                do.contiguous().to(q.dtype), _f32(dht), _f32(initial_state), scale, reverse,
                _cu_dev(cu_seqlens, q.device), n)
