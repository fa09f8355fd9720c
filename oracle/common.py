"""Shared pieces of the float64 oracle (test infrastructure only).

Restates:
  * tops/utils.py:63-90            prepare_lens / prepare_chunk_indices
  * tops/cpu/ops/common/utils.py   cdiv, pad_to_multiple, read_chunk
  * tops/cpu/ops/common/chunk_o.py:18-112   chunk_local_cumsum, chunk_local_cumsum_segments
    (the latter also tops/ops/gla/chunk.py:55-107: varlen restarts, short last chunks)
  * tops/cpu/ops/common/chunk_h.py:31-226   chunk_fwd_h   (gk and scalar-g gates)
  * tops/cpu/ops/common/chunk_h.py:229-427  chunk_bwd_dh  (gk and scalar-g gates)

Arrays are NumPy float64 in the reference's [B, T, H, D] layout.
"""

from __future__ import annotations

import numpy as np

F64 = np.float64


def f64(x):
    return None if x is None else np.asarray(x, dtype=F64)


def cdiv(a: int, b: int) -> int:
    """tops/cpu/ops/common/utils.py:10-12."""
    return (a + b - 1) // b


def pad_time(x: np.ndarray, mult: int) -> np.ndarray:
    """Zero-pad axis 1 to a multiple of `mult` (tops/cpu/ops/common/utils.py:15-33)."""
    T = x.shape[1]
    Tp = cdiv(T, mult) * mult
    if Tp == T:
        return x
    pad = [(0, 0)] * x.ndim
    pad[1] = (0, Tp - T)
    return np.pad(x, pad)


def prepare_lens(cu_seqlens) -> np.ndarray:
    """tops/utils.py:63-68."""
    cu = np.asarray(cu_seqlens, dtype=np.int64)
    return cu[1:] - cu[:-1]


def prepare_chunk_indices(cu_seqlens, chunk_size: int) -> np.ndarray:
    """tops/utils.py:71-90: [total_NT, 2] int32 rows of (sequence id, chunk id within it)."""
    lens = prepare_lens(cu_seqlens)
    rows = []
    for n, L in enumerate(lens):
        for c in range(cdiv(int(L), chunk_size)):
            rows.append((n, c))
    return np.asarray(rows, dtype=np.int32).reshape(-1, 2)


def chunk_local_cumsum(g: np.ndarray, C: int, reverse: bool = False) -> np.ndarray:
    """Inclusive prefix sum of the gates inside each length-C chunk along axis 1.

    tops/cpu/ops/common/chunk_o.py:88-112 (non-varlen branch; T % C == 0).
    Works for [B,T,H] (scalar gates) and [B,T,H,K] (per-channel gates).
    """
    g = f64(g)
    B, T = g.shape[:2]
    assert T % C == 0
    x = g.reshape(B, T // C, C, *g.shape[2:])
    if reverse:
        x = np.flip(x, axis=2)
    x = np.cumsum(x, axis=2)
    if reverse:
        x = np.flip(x, axis=2)
    return np.ascontiguousarray(x.reshape(g.shape))


def chunk_local_cumsum_segments(g, C: int, reverse: bool = False, cu_seqlens=None,
                                head_first: bool = False, scale=None) -> np.ndarray:
    """Chunk-local cumsum where chunks restart at every sequence start and the last chunk of
    a sequence may be short; then * scale.

    tops/cpu/ops/common/chunk_o.py:22-112 (packed-layout branch) and the accelerator kernel
    tops/ops/gla/chunk.py:55-107 (valid-length masking).  g: [B,T,H,S] ([B,H,T,S] when
    head_first); cu_seqlens [N+1] with B == 1, else each batch row is one sequence.
    """
    g = f64(g)
    x = np.swapaxes(g, 1, 2) if head_first else g
    out = np.zeros_like(x)
    T = x.shape[1]
    bounds = [(0, T)] if cu_seqlens is None else list(zip(cu_seqlens[:-1], cu_seqlens[1:]))
    for b in range(x.shape[0]):
        for s0, s1 in bounds:
            for c0 in range(int(s0), int(s1), C):
                c1 = min(c0 + C, int(s1))
                blk = x[b, c0:c1]
                if reverse:
                    out[b, c0:c1] = np.flip(np.cumsum(np.flip(blk, 0), 0), 0)
                else:
                    out[b, c0:c1] = np.cumsum(blk, 0)
    if scale is not None:
        out = out * scale
    return np.ascontiguousarray(np.swapaxes(out, 1, 2) if head_first else out)


def chunk_fwd_h(k, v, *, gk=None, g=None, h0=None, C: int = 64):
    """Inter-chunk state recurrence, non-varlen (tops/cpu/ops/common/chunk_h.py:179-226).

    k: [B,T,H,K], v: [B,T,H,V], T % C == 0.  gk: [B,T,H,K] chunk-local cumsum
    (gates k, USE_GK); g: [B,T,H] chunk-local cumsum (gates v, USE_G).
    Returns h: [B,NT,H,K,V] (state *before* each chunk) and ht (state after the last).
    """
    k, v = f64(k), f64(v)
    B, T, H, K = k.shape
    V = v.shape[-1]
    NT = T // C
    kc = k.reshape(B, NT, C, H, K)
    vc = v.reshape(B, NT, C, H, V)
    h = np.zeros((B, H, K, V), F64) if h0 is None else f64(h0).copy()
    hs = np.empty((B, NT, H, K, V), F64)
    for i in range(NT):
        hs[:, i] = h
        bk, bv = kc[:, i], vc[:, i]
        if g is not None:
            gc = f64(g).reshape(B, NT, C, H)[:, i]          # [B,C,H]
            glast = gc[:, -1]                                # [B,H]
            h = h * np.exp(glast)[:, :, None, None]
            bv = bv * np.exp(glast[:, None, :] - gc)[..., None]
        if gk is not None:
            gc = f64(gk).reshape(B, NT, C, H, K)[:, i]       # [B,C,H,K]
            glast = gc[:, -1]                                # [B,H,K]
            h = h * np.exp(glast)[..., None]
            bk = bk * np.exp(glast[:, None] - gc)
        h = h + np.einsum("bchk,bchv->bhkv", bk, bv)
    return hs, h


def chunk_bwd_dh(q, do, *, gk=None, g=None, dht=None, scale: float = 1.0, C: int = 64):
    """Reverse state-gradient recurrence, non-varlen (tops/cpu/ops/common/chunk_h.py:387-427).

    dh[:, i] is the gradient w.r.t. the state *after* chunk i (entering chunk i+1);
    dh0 is the gradient w.r.t. the initial state.
    """
    q, do = f64(q), f64(do)
    B, T, H, K = q.shape
    V = do.shape[-1]
    NT = T // C
    qc = q.reshape(B, NT, C, H, K)
    doc = do.reshape(B, NT, C, H, V)
    dh = np.zeros((B, H, K, V), F64) if dht is None else f64(dht).copy()
    dhs = np.empty((B, NT, H, K, V), F64)
    for i in range(NT - 1, -1, -1):
        dhs[:, i] = dh
        bq = qc[:, i] * scale
        if gk is not None:
            gc = f64(gk).reshape(B, NT, C, H, K)[:, i]
            bq = bq * np.exp(gc)
            dh = dh * np.exp(gc[:, -1])[..., None]
        if g is not None:
            gc = f64(g).reshape(B, NT, C, H)[:, i]
            bq = bq * np.exp(gc)[..., None]
            dh = dh * np.exp(gc[:, -1])[:, :, None, None]
        dh = dh + np.einsum("bchk,bchv->bhkv", bq, doc[:, i])
    return dhs, dh


def split_varlen(x: np.ndarray, cu_seqlens) -> list:
    """Slices of a packed [1, T_total, ...] tensor, one [1, L_n, ...] per sequence."""
    cu = [int(c) for c in cu_seqlens]
    return [x[:, cu[n]:cu[n + 1]] for n in range(len(cu) - 1)]
