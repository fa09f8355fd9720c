"""The delta-rule inter-chunk state pass on MI355X (mirrors tops/ops/common/chunk_delta_h.py:
chunk_gated_delta_rule_fwd_h_ref :44-166 and chunk_gated_delta_rule_fwd_h :898-977), the
stage of the KDA forward that the fused path runs inside its DELTA sweeps.  Here it is its
own kernel (tops_delta_rule_fwd_h, csrc/kda_stages.hip): one workgroup per (sequence, head,
64-column V slice) walking the chunks with the state slice in LDS, fp32 arithmetic.

Per chunk (S the state before it): h = S; v_new = u - w S; S = S 2^(g_last + gk_last) +
k^T (v_new 2^(g_last - g)), with k already gated by the caller and the gates chunk-local
cumsums (log2 units, natural with use_exp2=False)."""
from __future__ import annotations

import math

import numpy as np
import torch

from ... import _native as N
from ...utils import to_device
from ._stage import act, cu_host, f32, require


def chunk_gated_delta_rule_fwd_h(k, w, u, g=None, gk=None, initial_state=None,
                                 output_final_state: bool = False, chunk_size: int = 64,
                                 save_new_value: bool = True, use_exp2: bool = True,
                                 cu_seqlens=None, chunk_indices=None):
    """k, w [B,T,H,K]; u [B,T,H,V]; g [B,T,H] and / or gk [B,T,H,K] (optional);
    initial_state [N,H,K,V].  Returns (h [B, NT, H, K, V] in k.dtype, v_new [B,T,H,V] float32
    or None, final_state [N,H,K,V] float32 or None).  Varlen (cu_seqlens, B == 1) chunks each
    sequence on its own, as the reference; chunk_indices is accepted and recomputed here."""
    del chunk_indices
    B, T, H, K = k.shape
    V = u.shape[-1]
    C = int(chunk_size)
    require(tuple(w.shape) == (B, T, H, K), f"w shape {tuple(w.shape)} != {(B, T, H, K)}")
    require(tuple(u.shape[:3]) == (B, T, H), f"u shape {tuple(u.shape)} incompatible with k")
    require(g is None or tuple(g.shape) == (B, T, H), "g must be [B, T, H]")
    require(gk is None or tuple(gk.shape) == (B, T, H, K), "gk must be [B, T, H, K]")
    require(K <= 256, "current kernel does not support head dimension larger than 256.")
    if K > 128 or not 0 < C <= 64:
        raise NotImplementedError("tops-hip delta-rule state pass needs K <= 128 and chunk_size <= 64")
    cu = cu_host(cu_seqlens)
    if cu is None:
        require(T % C == 0, "For non-varlen input, T must be divisible by chunk_size")
        Nseq, total, offs = B, B * (T // C), None
    else:
        require(B == 1, f"varlen mode requires B==1, got B={B}")
        lens = np.diff(np.asarray(cu, np.int64))
        nch = -(-lens // C)
        Nseq, total = len(cu) - 1, int(nch.sum())
        offs = torch.tensor(np.concatenate([[0], np.cumsum(nch)[:-1]]).astype(np.int32),
                            device=k.device)
    require(initial_state is None or tuple(initial_state.shape) == (Nseq, H, K, V),
            f"initial_state must be {(Nseq, H, K, V)}")
    (kk, ww, uu), code = act(k, w, u)
    f = 1.0 if use_exp2 else 1.0 / math.log(2.0)
    g32 = None if g is None else (f32(g) * f).contiguous()
    gk32 = None if gk is None else (f32(gk) * f).contiguous()
    h0 = f32(initial_state)
    dev = k.device
    h = torch.empty(total, H, K, V, device=dev, dtype=kk.dtype)
    v_new = torch.empty(B, T, H, V, device=dev, dtype=torch.float32) if save_new_value else None
    ht = torch.empty(Nseq, H, K, V, device=dev, dtype=torch.float32) if output_final_state else None
    cu_dev = None if cu is None else to_device(cu, dev, torch.int32)
    N.call("tops_delta_rule_fwd_h", N.ptr(kk), N.ptr(ww), N.ptr(uu), N.ptr(g32), N.ptr(gk32), code,
           N.ptr(h0), N.ptr(h), N.ptr(v_new), N.ptr(ht), N.ptr(cu_dev), N.ptr(offs),
           B, T, H, K, V, Nseq, C, N.stream())
    h = h.reshape(B, total // B, H, K, V)
    return (h if h.dtype == k.dtype else h.to(k.dtype)), v_new, ht


def chunk_gated_delta_rule_fwd_h_ref(k, w, v, g=None, gk=None, initial_state=None,
                                     output_final_state: bool = False, chunk_size: int = 64):
    """tops/ops/common/chunk_delta_h.py:44-166: the same pass with v for u, returning
    (h [B, NT, H, K, V], v_new [B, T, H, V], final_state or None), all float32."""
    h, v_new, ht = chunk_gated_delta_rule_fwd_h(k, w, v, g=g, gk=gk, initial_state=initial_state,
                                                output_final_state=output_final_state,
                                                chunk_size=chunk_size)
    return h.float(), v_new, ht


__all__ = ["chunk_gated_delta_rule_fwd_h", "chunk_gated_delta_rule_fwd_h_ref"]
