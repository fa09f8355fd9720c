"""Independent formulations used to pin the oracle (test helpers).

The "parallel form" writes the gated recurrence S_t = diag(exp(g_t)) S_{t-1} + k_t v_t^T,
o_t = scale * S_t^T q_t as an explicit quadratic sum with a materialised decay
mask built from the *global* (not chunk-local) cumulative gate sum:

  o_t = scale * sum_{s<=t} sum_k q_tk k_sk exp(Gc_tk - Gc_sk) v_s + scale * (q_t*exp(Gc_t)) @ h0
  h_T = exp(Gc_T)[:,None] * h0 + sum_s (k_s * exp(Gc_T - Gc_s)) v_s^T

It shares no code or chunking with the oracle, and torch float64 autograd
through it gives every gradient without any hand-derived backward formula.
"""
import numpy as np
import torch


def gla_parallel_torch(q, k, v, g, h0=None, scale=None, gv=None):
    """Batched torch float64 parallel form; g: [B,T,H,K] per-channel log gates,
    gv: optional [B,T,H,V] per-value log gates."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    if scale is None:
        scale = K ** -0.5
    Gc = torch.cumsum(g, dim=1)                                  # [B,T,H,K]
    # D[b,t,s,h,k] = exp(Gc_t - Gc_s) for s <= t
    diff = Gc[:, :, None] - Gc[:, None, :]                       # [B,T,S,H,K]
    mask = torch.tril(torch.ones(T, T, dtype=torch.bool))[None, :, :, None, None]
    D = torch.where(mask, torch.exp(torch.where(mask, diff, torch.zeros_like(diff))),
                    torch.zeros_like(diff))
    if gv is None:
        A = torch.einsum("bthk,bshk,btshk->btsh", q, k, D)
        o = scale * torch.einsum("btsh,bshv->bthv", A, v)
    else:
        Gv = torch.cumsum(gv, dim=1)
        dv_ = Gv[:, :, None] - Gv[:, None, :]
        Dv = torch.where(mask, torch.exp(torch.where(mask, dv_, torch.zeros_like(dv_))),
                         torch.zeros_like(dv_))
        A = torch.einsum("bthk,bshk,btshk->btsh", q, k, D)
        o = scale * torch.einsum("btsh,bshv,btshv->bthv", A, v, Dv)
    GT = Gc[:, -1]                                               # [B,H,K]
    kd = k * torch.exp(GT[:, None] - Gc)
    if gv is None:
        ht = torch.einsum("bshk,bshv->bhkv", kd, v)
    else:
        GvT = Gv[:, -1]
        ht = torch.einsum("bshk,bshv->bhkv", kd, v * torch.exp(GvT[:, None] - Gv))
    if h0 is not None:
        if gv is None:
            o = o + scale * torch.einsum("bthk,bhkv->bthv", q * torch.exp(Gc), h0)
            ht = ht + torch.exp(GT)[..., None] * h0
        else:
            o = o + scale * torch.einsum("bthk,bhkv,bthv->bthv", q * torch.exp(Gc), h0,
                                         torch.exp(Gv))
            ht = ht + torch.exp(GT)[..., None] * h0 * torch.exp(Gv[:, -1])[:, :, None, :]
    return o, ht


def gla_parallel_grads(q, k, v, g, h0, do, dht, scale=None, gv=None):
    """Gradients of sum(o*do) + sum(ht*dht) through the parallel form (torch fp64 autograd).

    Returns numpy dict with o, ht, dq, dk, dv, dg, dh0 (and dgv)."""
    t = {n: (None if x is None else torch.tensor(np.asarray(x, np.float64), requires_grad=True))
         for n, x in dict(q=q, k=k, v=v, g=g, h0=h0, gv=gv).items()}
    o, ht = gla_parallel_torch(t["q"], t["k"], t["v"], t["g"], t["h0"], scale, t["gv"])
    loss = (o * torch.tensor(np.asarray(do, np.float64))).sum()
    if dht is not None:
        loss = loss + (ht * torch.tensor(np.asarray(dht, np.float64))).sum()
    loss.backward()
    out = dict(o=o.detach().numpy(), ht=ht.detach().numpy())
    for n in ("q", "k", "v", "g", "h0", "gv"):
        if t[n] is not None:
            out["d" + n] = t[n].grad.numpy()
    return out


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = np.linalg.norm(b.ravel())
    return np.linalg.norm((a - b).ravel()) / (den if den > 0 else 1.0)


def kda_naive_torch(q, k, v, g, beta, h0=None, scale=None):
    """Per-token gated delta rule in torch (differentiable), written from the recurrence
    S' = S diag(exp g_t); S = S' + beta_t k_t (v_t - S'^T k_t)^T; o_t = S^T (scale q_t)."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    if scale is None:
        scale = K ** -0.5
    S = torch.zeros(B, H, K, V, dtype=q.dtype) if h0 is None else h0
    outs = []
    for t in range(T):
        S = S * torch.exp(g[:, t])[..., None]
        pred = torch.einsum("bhk,bhkv->bhv", k[:, t], S)
        S = S + torch.einsum("bhk,bhv->bhkv", beta[:, t][..., None] * k[:, t], v[:, t] - pred)
        outs.append(torch.einsum("bhk,bhkv->bhv", q[:, t] * scale, S))
    return torch.stack(outs, 1), S


def kda_grads(q, k, v, g, beta, h0, do, dht, scale=None):
    """o, ht and the gradients of sum(o*do) + sum(ht*dht) through kda_naive_torch (fp64)."""
    t = {n: torch.tensor(np.asarray(x, np.float64), requires_grad=True)
         for n, x in dict(q=q, k=k, v=v, g=g, beta=beta).items()}
    h0t = None if h0 is None else torch.tensor(np.asarray(h0, np.float64), requires_grad=True)
    o, ht = kda_naive_torch(t["q"], t["k"], t["v"], t["g"], t["beta"], h0t, scale)
    loss = (o * torch.tensor(np.asarray(do, np.float64))).sum()
    if dht is not None:
        loss = loss + (ht * torch.tensor(np.asarray(dht, np.float64))).sum()
    loss.backward()
    out = dict(o=o.detach().numpy(), ht=ht.detach().numpy())
    for n in ("q", "k", "v", "g", "beta"):
        out["d" + n] = t[n].grad.numpy()
    if h0t is not None:
        out["dh0"] = h0t.grad.numpy()
    return out
