"""Seeded synthetic inputs (NumPy PCG64, machine-independent)."""
import numpy as np


def logsigmoid(x):
    return -np.logaddexp(0.0, -x)


def gla_inputs(B, T, H, K, V, seed, gate_div=16.0, h0=False, N=None, dtype=np.float32,
               grads=False):
    rng = np.random.Generator(np.random.PCG64(seed))
    q = rng.standard_normal((B, T, H, K)).astype(np.float32)
    k = rng.standard_normal((B, T, H, K)).astype(np.float32)
    v = rng.standard_normal((B, T, H, V)).astype(np.float32)
    g = (logsigmoid(rng.standard_normal((B, T, H, K))) / gate_div).astype(np.float32)
    d = dict(q=q, k=k, v=v, g=g)
    n0 = B if N is None else N
    d["h0"] = (0.1 * rng.standard_normal((n0, H, K, V))).astype(np.float32) if h0 else None
    if grads:
        d["do"] = rng.standard_normal((B, T, H, V)).astype(np.float32)
        d["dht"] = (0.1 * rng.standard_normal((n0, H, K, V))).astype(np.float32)
    return d


def bf16_round(x):
    """Round-to-nearest-even float32 -> bfloat16 values, returned as float32."""
    x = np.ascontiguousarray(x, np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def simple_gla_inputs(B, T, H, K, V, seed, gate_div=1.0, h0=False, N=None, grads=False):
    """Seeded simple-GLA inputs: q, k, v ~ N(0,1); g = logsigmoid(N(0,1))/gate_div [B,T,H];
    g_gamma = -|N(0,1)|/8 [H]."""
    rng = np.random.Generator(np.random.PCG64(seed))
    d = dict(q=rng.standard_normal((B, T, H, K)).astype(np.float32),
             k=rng.standard_normal((B, T, H, K)).astype(np.float32),
             v=rng.standard_normal((B, T, H, V)).astype(np.float32),
             g=(logsigmoid(rng.standard_normal((B, T, H))) / gate_div).astype(np.float32),
             g_gamma=(-np.abs(rng.standard_normal(H)) / 8).astype(np.float32))
    n0 = B if N is None else N
    d["h0"] = (0.1 * rng.standard_normal((n0, H, K, V))).astype(np.float32) if h0 else None
    if grads:
        d["do"] = rng.standard_normal((B, T, H, V)).astype(np.float32)
        d["dht"] = (0.1 * rng.standard_normal((n0, H, K, V))).astype(np.float32)
    return d


def varlen_cu(T_total, N, seed):
    """cu_seqlens [N+1] with seeded uniform-random cut points (generally not chunk-aligned)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    cuts = np.sort(rng.choice(np.arange(1, T_total), N - 1, replace=False))
    return [0] + [int(c) for c in cuts] + [T_total]


def kda_inputs(B, T, H, K, V, seed, gate_div=16.0, h0=False, grads=False, N=None):
    """BASELINE config-5 style KDA inputs: q, k ~ N(0,1) L2-normalised over K per (b,t,h)
    as x / sqrt(sum x^2 + 1e-6) (tops/cpu/ops/kda/fused_recurrent.py:14-18); v ~ N(0,1);
    beta = sigmoid(N(0,1)) [B,T,H]; g = logsigmoid(N(0,1)) / gate_div [B,T,H,K]."""
    rng = np.random.Generator(np.random.PCG64(seed))

    def l2n(x):
        return x / np.sqrt(np.sum(x * x, axis=-1, keepdims=True) + 1e-6)
    d = dict(q=l2n(rng.standard_normal((B, T, H, K))).astype(np.float32),
             k=l2n(rng.standard_normal((B, T, H, K))).astype(np.float32),
             v=rng.standard_normal((B, T, H, V)).astype(np.float32),
             beta=(1.0 / (1.0 + np.exp(-rng.standard_normal((B, T, H))))).astype(np.float32),
             g=(logsigmoid(rng.standard_normal((B, T, H, K))) / gate_div).astype(np.float32))
    n = B if N is None else N
    d["h0"] = (0.1 * rng.standard_normal((n, H, K, V))).astype(np.float32) if h0 else None
    if grads:
        d["do"] = rng.standard_normal((B, T, H, V)).astype(np.float32)
        d["dht"] = (0.1 * rng.standard_normal((n, H, K, V))).astype(np.float32)
    return d
