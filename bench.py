"""Headline benchmark: chunk_gla forward + backward at B=8, T=4096, H=16, K=V=128, bf16.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]

One step = tops.ops.gla.chunk_gla forward (o, final state) plus its backward
(dq, dk, dv, dg, dh0) through torch autograd, on synthetic inputs already resident
in HBM (q, k, v, dO ~ N(0,1) bf16; g = logsigmoid(N(0,1))/16 fp32; h0, dht ~
N(0, 0.1^2) fp32).  Prints ONE JSON line with the throughput (tokens/s, tokens =
B*T per step), the roofline of the dominant kernel timed live with HIP events on
the stream the kernels run on, and a CPU baseline: torch-CPU float32 restatements of the
reference's algorithms (oracle/torch_cpu.py, pinned against the float64 oracle) timed on this
host's cores, forward and forward + backward, on each measured config's own inputs copied
from the GPU.  The same CPU runs are the parity reference at the full BASELINE shapes: the
line carries the relative L2 error of every output and gradient of the GPU step against them.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "pallas-kernel_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

B, T, H, K, V, C = 8, 4096, 16, 128, 128, 64
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
MFMA_BF16_PEAK_TFS = 2500.0    # MI355X dense bf16 MFMA
METRIC = "chunk_gla fwd+bwd tokens/s (B8,T4096,H16,D128 bf16); % MFMA/HBM peak"

# Algorithmic HBM bytes per launch of each kernel at this config (bf16 q/k/v/o/do and
# their gradients, fp32 gates, gate gradient and states; nothing intermediate counted).
_TH = B * T * H
_S = B * H * K * V * 4
# Rows are keyed by C-ABI entry point; the training step calls the fp16-checkpoint entries
# ("entry": the default checkpoint layout for bf16 inputs with per-channel gates), and
# set_checkpoint_layout("full32") the fp32-checkpoint ones: both are timed under one row.
KERNELS = {
    # q, k, v, g read; o written; h0 read; ht written
    "tops_gla_chunk_fwd": dict(kernel="gla_pipe_kernel<fwd>", entry="tops_gla_chunk_fwd_c16",
                               bytes=_TH * (2 * K + 2 * K + 2 * V + 4 * K + 2 * V) + 2 * _S),
    # q, k, g, dO read; dv written; dht read; dh0 written
    "tops_gla_chunk_bwd_dh": dict(kernel="gla_pipe_kernel<rev>", entry="tops_gla_chunk_bwd_dh_c16",
                                  bytes=_TH * (2 * K + 2 * K + 4 * K + 2 * V + 2 * V) + 2 * _S),
    # q, k, v, g, dO read; dq, dk, dg written
    "tops_gla_chunk_bwd_dqkg": dict(kernel="gla_dqkg_kernel", entry="tops_gla_chunk_bwd_dqkg_c16",
                                    bytes=_TH * (2 * K + 2 * K + 2 * V + 4 * K + 2 * V
                                                 + 2 * K + 2 * K + 4 * K)),
}
# Whole-path minimum (each tensor read once per pass, written once): 2 323 644 416 B and
# 294 912 flop per token-head (fwd 4KV+2CK+2CV, bwd twice that).
PATH_BYTES = 2_323_644_416
PATH_FLOPS = _TH * (3 * (4 * K * V + 2 * C * K + 2 * C * V))


def make_inputs(device, seed=1003):
    import torch
    gen = torch.Generator(device=device).manual_seed(seed)

    def n(*shape, std=1.0):
        return torch.randn(*shape, generator=gen, device=device, dtype=torch.float32) * std

    bf = torch.bfloat16
    q = n(B, T, H, K).to(bf).requires_grad_()
    k = n(B, T, H, K).to(bf).requires_grad_()
    v = n(B, T, H, V).to(bf).requires_grad_()
    g = (torch.nn.functional.logsigmoid(n(B, T, H, K)) / 16).requires_grad_()
    h0 = n(B, H, K, V, std=0.1).requires_grad_()
    do = n(B, T, H, V).to(bf)
    dht = n(B, H, K, V, std=0.1)
    return q, k, v, g, h0, do, dht


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _host(t):
    return None if t is None else t.detach().float().cpu()


def _rel(a, b):
    """Relative L2 error ||a - b|| / ||b|| in float64."""
    import torch
    a, b = a.double(), b.double()
    return float(torch.linalg.norm(a - b) / torch.linalg.norm(b))


class CpuLeg:
    """The CPU baseline and full-shape parity leg.  Each measured config registers its inputs
    (copied from the GPU after its timing), its GPU outputs and the torch-CPU restatement of
    its reference function; run() then times the restatement, forward alone and forward +
    backward, on every CPU thread this process is granted (OMP_NUM_THREADS, else
    os.cpu_count()), one warm-up and the median of `repeats`, and compares the GPU outputs
    with the forward + backward result.  Reported only; the tolerance is north_star's
    (bf16 paths 2e-3, fp32 1e-4, relative L2)."""

    def __init__(self, repeats=3, warmup=1):
        self.repeats, self.warmup, self.cases = repeats, warmup, []

    def add(self, name, tokens, gpu_ms, fwd, fwd_bwd, gpu_out, tol):
        self.cases.append(dict(name=name, tokens=tokens, gpu_ms=gpu_ms, fwd=fwd,
                               fwd_bwd=fwd_bwd, gpu_out=gpu_out, tol=tol))

    def _median(self, fn):
        times, out = [], None
        for i in range(self.warmup + self.repeats):
            t0 = time.perf_counter()
            out = fn()
            if i >= self.warmup:
                times.append(time.perf_counter() - t0)
        return statistics.median(times), out

    def run(self):
        import torch
        threads = int(os.environ.get("OMP_NUM_THREADS") or 0) or (os.cpu_count() or 1)
        prev = torch.get_num_threads()
        torch.set_num_threads(threads)
        res = {}
        try:
            for c in self.cases:
                row = {}
                t_f, ref = self._median(c["fwd"])
                row["fwd_s"] = round(t_f, 4)
                row["fwd_tokens_s"] = round(c["tokens"] / t_f, 1)
                if c["fwd_bwd"] is not None:
                    t_fb, ref = self._median(c["fwd_bwd"])
                    row["fwd_bwd_s"] = round(t_fb, 4)
                    row["fwd_bwd_tokens_s"] = round(c["tokens"] / t_fb, 1)
                gms = c["gpu_ms"]
                for key, ms in gms.items():
                    cpu_s = row.get(key + "_s")
                    if cpu_s:
                        row[f"gpu_speedup_{key}"] = round(cpu_s / (ms * 1e-3), 1)
                errs = {n: _rel(g, ref[n]) for n, g in c["gpu_out"].items()
                        if g is not None and ref.get(n) is not None}
                row["parity"] = {"rel_err": {n: float(f"{e:.3e}") for n, e in errs.items()},
                                 "tolerance": c["tol"],
                                 "pass": all(e <= c["tol"] for e in errs.values())}
                res[c["name"]] = row
        finally:
            torch.set_num_threads(prev)
        return res, threads


def cpu_summary(res, threads):
    head = res.get("3", {})
    return {"value": head.get("fwd_bwd_tokens_s"), "unit": "tokens/s", "cores": threads,
            "kind": "port", "cpu_count": os.cpu_count(), "cpu_model": _cpu_model(),
            "seconds_per_step": head.get("fwd_bwd_s"),
            "sample": f"torch-CPU float32 restatements of tops/cpu (oracle/torch_cpu.py, pinned "
                      f"to the float64 oracle) on each config's own GPU inputs: the full step of "
                      f"each config, forward and forward + backward, {threads} threads, 1 warm-up "
                      f"+ median of 3; value = config 3 fwd+bwd",
            "configs": {k: {x: y for x, y in v.items() if x != "parity"} for k, v in res.items()}}


def _time(fn, iters, warmup=2, settle_s=0.2):
    """Mean wall time of iters calls, after untimed calls that settle the GPU clock (at least
    warmup of them, and at least settle_s of wall time: the clock ramps up over the first
    ~30 ms of busy work after an idle period, and calls of ~0.15 ms with host waits between
    them keep it lower for longer)."""
    import torch
    fn()                       # the first call may load code objects and allocate
    torch.cuda.synchronize()
    n, t_s = 1, time.perf_counter()
    while n < warmup or time.perf_counter() - t_s < settle_s:
        fn()
        n += 1
        if n % 16 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(iters):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / iters


def secondary(dev, iters=10, configs=(2, 4, 5), leg=None):
    """The other BASELINE configs that fit one GPU, measured the same way (inputs resident,
    synchronise around the timed iterations): config 1 (chunk_gla forward, fp32), config 2
    (fused_recurrent_gla forward), config 4 (simple GLA, varlen, forward + backward) and
    config 5 (KDA, forward + backward); each registers its inputs and outputs with the CPU
    leg when one is given."""
    import torch
    out = []
    gen = torch.Generator(device=dev).manual_seed(1002)
    if 1 in configs:
        out.append(_config1(dev, iters, leg))
    if 2 in configs:
        out.append(_config2(dev, gen, iters, leg))
    if 4 in configs:
        out.append(_config4(dev, gen, iters, leg))
    if 5 in configs:
        out.append(_config5(dev, gen, iters, leg))
    if 6 in configs:
        out.append(_neighbours(dev, gen, iters))
    if 7 in configs:
        out.append(_decode(dev, gen, iters))
    return out


def _decode(dev, gen, iters):
    """Decode steps (one token per sequence against a state cache), the route the reference's
    layer takes for q_len <= 64: fused_recurrent_gla (B256 H16 K=V=128, gk) and
    fused_recurrent_kda (B64 H32 K=V=128), bf16 inputs, fp32 states.  Each decode kernel is
    timed per launch with HIP events on its stream; its bytes are the state read and written
    (2 K V 4 per sequence and head) plus the token's inputs and output."""
    import torch
    from tops import _native as NT
    from tops.modules import rms_norm_gated
    from tops.ops.gla import fused_recurrent_gla, fused_recurrent_gla_norm_gate
    from tops.ops.kda import fused_recurrent_kda
    bf = torch.bfloat16
    D = 128
    cases = []
    Bg, Hg = 256, 16
    q1, k1, v1 = (torch.randn(Bg, 1, Hg, D, device=dev, generator=gen).to(bf) for _ in range(3))
    g1 = torch.nn.functional.logsigmoid(torch.randn(Bg, 1, Hg, D, device=dev, generator=gen)) / 16
    s1 = torch.randn(Bg, Hg, D, D, device=dev, generator=gen) * 0.1
    cases.append(("tops_gla_fused_recurrent_fwd_decode", "fused_recurrent_gla B256 T1 H16 K=V=128 gk",
                  Bg * Hg * (2 * D * D * 4 + 3 * D * 2 + D * 4 + D * 2),
                  lambda: fused_recurrent_gla(q1, k1, v1, g1, initial_state=s1, output_final_state=True)))
    # the layer's decode route with its output norm fused into the same kernel:
    # y = RMSNorm(o) * w * silu(g) over V; bytes as above plus the gate read (o is never stored)
    og1 = torch.randn(Bg, 1, Hg, D, device=dev, generator=gen).to(bf)
    nw1 = torch.ones(D, device=dev)
    cases.append(("tops_gla_fused_recurrent_fwd_decode_norm_gate",
                  "fused_recurrent_gla + FusedRMSNormGated B256 T1 H16 K=V=128 gk",
                  Bg * Hg * (2 * D * D * 4 + 3 * D * 2 + D * 4 + D * 2 + D * 2),
                  lambda: fused_recurrent_gla_norm_gate(q1, k1, v1, g1, None, og1, nw1,
                                                        initial_state=s1, output_final_state=True)))
    Bk, Hk = 64, 32
    q2, k2 = (torch.nn.functional.normalize(torch.randn(Bk, 1, Hk, D, device=dev, generator=gen), dim=-1).to(bf)
              for _ in range(2))
    v2 = torch.randn(Bk, 1, Hk, D, device=dev, generator=gen).to(bf)
    g2 = torch.nn.functional.logsigmoid(torch.randn(Bk, 1, Hk, D, device=dev, generator=gen)) / 16
    b2 = torch.sigmoid(torch.randn(Bk, 1, Hk, device=dev, generator=gen))
    s2 = torch.randn(Bk, Hk, D, D, device=dev, generator=gen) * 0.1
    cases.append(("tops_kda_fused_recurrent_fwd_decode", "fused_recurrent_kda B64 T1 H32 K=V=128",
                  Bk * Hk * (2 * D * D * 4 + 3 * D * 2 + D * 4 + 4 + D * 2),
                  lambda: fused_recurrent_kda(q2, k2, v2, g2, b2, None, s2, True)))
    rows = []
    # a plain device copy of the GLA state cache (read + write of the same bytes) on the same
    # stream, timed the same way: the practical bound the decode kernels are measured against
    src = torch.empty_like(s1).normal_(generator=gen)
    dst = torch.empty_like(src)
    cev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(iters)]
    dst.copy_(src)
    for e0, e1 in cev:
        e0.record()
        dst.copy_(src)
        e1.record()
    torch.cuda.synchronize()
    cms = sum(e0.elapsed_time(e1) for e0, e1 in cev) / iters
    cbytes = 2 * src.numel() * 4
    copy_ref = {"what": "dst.copy_(src), fp32 [256, 16, 128, 128]", "bytes": cbytes, "avg_ms": round(cms, 4),
                "hbm_gbs": round(cbytes / (cms * 1e-3) / 1e9, 1)}
    del src, dst
    with torch.no_grad():
        for _, _, _, f in cases:
            f()
        torch.cuda.synchronize()
        NT.enable_timing(True)
        for _ in range(iters):
            for _, _, _, f in cases:
                f()
        torch.cuda.synchronize()
        ev = NT.timing_events()
        NT.enable_timing(False)
    for name, shape, nbytes, _ in cases:
        ms = [e0.elapsed_time(e1) for e0, e1 in ev.get(name, [])]
        if not ms:
            continue
        avg = sum(ms) / len(ms)
        gbs = nbytes / (avg * 1e-3) / 1e9
        rows.append({"entry": name, "shape": shape, "avg_ms": round(avg, 4), "launches": len(ms),
                     "algo_bytes": nbytes, "hbm_gbs": round(gbs, 1),
                     "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)})
    for r in rows:
        r["frac_of_copy"] = round(r["hbm_gbs"] / copy_ref["hbm_gbs"], 4)
    # the same norm unfused: the decode kernel writes o, the standalone norm kernel reads it
    with torch.no_grad():
        unf = _time(lambda: rms_norm_gated(fused_recurrent_gla(q1, k1, v1, g1, initial_state=s1,
                                                               output_final_state=True)[0],
                                           og1, nw1), iters)
        fus = _time(lambda: fused_recurrent_gla_norm_gate(q1, k1, v1, g1, None, og1, nw1,
                                                          initial_state=s1,
                                                          output_final_state=True), iters)
    norm_route = {"what": "decode step + output norm, B256 H16 K=V=128, wall time per call",
                  "fused_ms": round(fus * 1e3, 4), "unfused_ms": round(unf * 1e3, 4)}
    # the layer's whole decode route from the projections: three ShortConvolution steps (W 4,
    # SiLU, fp32 caches), the recurrence and the norm, unfused and as one kernel
    from tops.modules import short_conv_step
    from tops.ops.gla import fused_recurrent_gla_conv_norm_gate
    Dk = Hg * D
    xq, xk, xv = (torch.randn(Bg, 1, Dk, device=dev, generator=gen).to(bf) for _ in range(3))
    cws = [torch.randn(Dk, 4, device=dev, generator=gen) / 2 for _ in range(3)]
    ccs = [torch.randn(Bg, Dk, 4, device=dev, generator=gen) for _ in range(3)]

    def unfused_layer():
        qkv = [short_conv_step(x, w, None, "silu", c, True)[0].reshape(Bg, 1, Hg, D)
               for x, w, c in zip((xq, xk, xv), cws, ccs)]
        o, _ = fused_recurrent_gla(*qkv, g1, initial_state=s1, output_final_state=True)
        return rms_norm_gated(o, og1.float(), nw1)

    with torch.no_grad():
        unf_l = _time(unfused_layer, iters)
        fus_l = _time(lambda: fused_recurrent_gla_conv_norm_gate(
            *(x.reshape(Bg, 1, Hg, D) for x in (xq, xk, xv)), cws, None, ccs, "silu", g1, og1,
            nw1, initial_state=s1, output_final_state=True), iters)
    norm_route["layer_route"] = {
        "what": "ShortConvolution q/k/v steps + decode step + output norm, B256 H16 K=V=128 W4",
        "fused_ms": round(fus_l * 1e3, 4), "unfused_ms": round(unf_l * 1e3, 4)}
    # the same route at a small serving batch (B 8), where the launches dominate
    b8 = slice(0, 8)
    with torch.no_grad():
        unf8 = _time(lambda: rms_norm_gated(fused_recurrent_gla(
            *[short_conv_step(x[b8], w, None, "silu", c[b8], True)[0].reshape(8, 1, Hg, D)
              for x, w, c in zip((xq, xk, xv), cws, ccs)], g1[b8], initial_state=s1[b8],
            output_final_state=True)[0], og1[b8].float(), nw1), iters)
        fus8 = _time(lambda: fused_recurrent_gla_conv_norm_gate(
            *(x[b8].reshape(8, 1, Hg, D) for x in (xq, xk, xv)), cws, None,
            [c[b8] for c in ccs], "silu", g1[b8], og1[b8], nw1, initial_state=s1[b8],
            output_final_state=True), iters)
    norm_route["layer_route_b8"] = {"what": "the same at B8 (launch-bound)",
                                    "fused_ms": round(fus8 * 1e3, 4),
                                    "unfused_ms": round(unf8 * 1e3, 4)}
    return {"config": "decode steps (state-cache bound)", "kernels": rows, "copy_ref": copy_ref,
            "norm_route": norm_route}


def _neighbours(dev, gen, iters):
    """The kernels either side of the op, each timed per launch with HIP events on the stream
    it runs on, against its algorithmic HBM bytes: the KDA gate (forward, backward, log2
    chunk cumsum) and the q / k L2 norm at config 5's shape, FusedRMSNormGated on the GLA
    output and ShortConvolution (W = 4) on a projection at config 3's layer shape."""
    import torch
    from tops import _native as NT
    from tops.modules import rms_norm_gated, short_conv
    from tops.ops.kda import fused_kda_gate, kda_gate_chunk_cumsum, l2norm
    f32, bf = torch.float32, torch.bfloat16
    B5, T5, H5, D = 4, 8192, 32, 128
    n5 = B5 * T5 * H5 * D
    g = torch.randn(B5, T5, H5, D, device=dev, generator=gen).requires_grad_()
    A = torch.log(torch.rand(H5, device=dev, generator=gen) * 3 + 1).requires_grad_()
    bias = torch.randn(H5 * D, device=dev, generator=gen).requires_grad_()
    dyg = torch.randn(B5, T5, H5, D, device=dev, generator=gen)
    gl = torch.nn.functional.logsigmoid(torch.randn(B5, T5, H5, D, device=dev, generator=gen))
    q = torch.randn(B5, T5, H5, D, device=dev, generator=gen).to(bf).requires_grad_()
    dq = torch.randn(B5, T5, H5, D, device=dev, generator=gen)
    n3 = B * T * H * V
    o = torch.randn(B, T, H, V, device=dev, generator=gen).to(bf).requires_grad_()
    og = torch.randn(B, T, H, V, device=dev, generator=gen).to(bf).requires_grad_()
    w = torch.ones(V, device=dev, requires_grad=True)
    do = torch.randn(B, T, H, V, device=dev, generator=gen).to(bf)
    Dh = H * K
    x = torch.randn(B, T, Dh, device=dev, generator=gen).to(bf).requires_grad_()
    cw = (torch.randn(Dh, 1, 4, device=dev, generator=gen) / 2).requires_grad_()
    cb = torch.randn(Dh, device=dev, generator=gen).requires_grad_()
    dy = torch.randn(B, T, Dh, device=dev, generator=gen)
    nc = B * T * Dh
    algo = {  # entry point -> (algorithmic bytes per launch, shape)
        "tops_kda_gate_fwd": (n5 * 8, "g f32 [4,8192,32,128] -> y f32"),
        "tops_kda_gate_bwd": (n5 * 12, "g, dyg f32 -> dg f32 (+ dA, dbias)"),
        "tops_kda_gate_chunk_cumsum": (n5 * 8, "g f32 -> log2 chunk cumsum f32"),
        "tops_l2norm_fwd": (n5 * 6, "q bf16 [4,8192,32,128] -> f32"),
        "tops_l2norm_bwd": (n5 * 8, "q bf16, dy f32 -> dq bf16"),
        "tops_rmsnorm_gated_fwd": (n3 * 6, "o, g bf16 [8,4096,16,128] -> bf16"),
        "tops_rmsnorm_gated_bwd": (n3 * 10, "o, g, dy bf16 -> do, dg bf16 (+ dw)"),
        "tops_short_conv_fwd": (nc * 6, "x bf16 [8,4096,2048], W=4 -> y f32"),
        "tops_short_conv_bwd": (nc * 8, "x bf16, dy f32 -> dx bf16 (+ dw, db)"),
    }

    def run():
        y = fused_kda_gate(g, A, dt_bias=bias)
        torch.autograd.grad(y, (g, A, bias), dyg)
        kda_gate_chunk_cumsum(gl, 64)
        torch.autograd.grad(l2norm(q), q, dq)
        torch.autograd.grad(rms_norm_gated(o, og, w), (o, og, w), do)
        yc, _ = short_conv(x, cw, cb, "silu")
        torch.autograd.grad(yc, (x, cw, cb), dy)
    run()
    torch.cuda.synchronize()
    NT.enable_timing(True)
    for _ in range(iters):
        run()
    torch.cuda.synchronize()
    ev = NT.timing_events()
    NT.enable_timing(False)
    rows = []
    for name, (nbytes, shape) in algo.items():
        ms = [e0.elapsed_time(e1) for e0, e1 in ev.get(name, [])]
        if not ms:
            continue
        avg = sum(ms) / len(ms)
        gbs = nbytes / (avg * 1e-3) / 1e9
        rows.append({"entry": name, "shape": shape, "avg_ms": round(avg, 4), "launches": len(ms),
                     "algo_bytes": nbytes, "hbm_gbs": round(gbs, 1),
                     "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)})
    return {"config": "layer-side and KDA gate kernels (HBM-bound streams)", "kernels": rows}


def _config1(dev, iters, leg):
    """config 1: chunk_gla forward, fp32, B2 T512 H4 K=V=64; q, k, v ~ N(0,1), then q scaled
    by K^-1/2 (and the default scale K^-1/2 applied on top); g = logsigmoid(N(0,1))/16; no
    initial state; o + final state."""
    import torch
    from oracle import torch_cpu as TC
    from tops.ops.gla import chunk_gla
    B1, T1, H1, D1 = 2, 512, 4, 64
    gen = torch.Generator(device=dev).manual_seed(1001)
    q, k, v = (torch.randn(B1, T1, H1, D1, device=dev, generator=gen) for _ in range(3))
    q = q * D1 ** -0.5
    g = torch.nn.functional.logsigmoid(torch.randn(B1, T1, H1, D1, device=dev, generator=gen)) / 16
    with torch.no_grad():
        sec = _time(lambda: chunk_gla(q, k, v, g, output_final_state=True), iters)
        o, ht = chunk_gla(q, k, v, g, output_final_state=True)
    torch.cuda.synchronize()
    if leg is not None:
        hq, hk, hv, hg = (_host(x) for x in (q, k, v, g))
        leg.add("1", B1 * T1, {"fwd": sec * 1e3},
                lambda: dict(zip(("o", "ht"), TC.chunk_gla_fwd_bwd(hq, hk, hv, hg, None, None, None,
                                                                   D1 ** -0.5, backward=False))),
                None, {"o": _host(o), "ht": _host(ht)}, 1e-4)
    return {"config": "BASELINE config 1: chunk_gla fwd B2 T512 H4 K=V=64 fp32",
            "tokens_per_s": round(B1 * T1 / sec, 1), "ms": round(sec * 1e3, 4)}


def _config2(dev, gen, iters, leg):
    """config 2: B16 T2048 H8 K=V=128, bf16 q/k/v, fp32 gk and h0; o + final state."""
    import torch
    from oracle import torch_cpu as TC
    from tops.ops.gla import fused_recurrent_gla
    bf = torch.bfloat16
    B2, T2, H2, D2 = 16, 2048, 8, 128
    q, k, v = (torch.randn(B2, T2, H2, D2, device=dev, generator=gen).to(bf) for _ in range(3))
    gk = torch.nn.functional.logsigmoid(torch.randn(B2, T2, H2, D2, device=dev, generator=gen)) / 16
    h0 = torch.randn(B2, H2, D2, D2, device=dev, generator=gen) * 0.1
    with torch.no_grad():
        sec = _time(lambda: fused_recurrent_gla(q, k, v, gk, initial_state=h0,
                                                output_final_state=True), iters)
        # the same shape walked in reverse (the reverse chunk sweep with the gate read one
        # token later), and with a per-column gv gate instead of gk (the forward sweep with the
        # gate on the value side): same algorithmic bytes
        sec_rev = _time(lambda: fused_recurrent_gla(q, k, v, gk, initial_state=h0,
                                                    output_final_state=True, reverse=True), iters)
        sec_gv = _time(lambda: fused_recurrent_gla(q, k, v, None, gv=gk, initial_state=h0,
                                                   output_final_state=True), iters)
        o, ht = fused_recurrent_gla(q, k, v, gk, initial_state=h0, output_final_state=True)
    # training with the gv gate (forward + backward on the chunk kernels; gk-only training is
    # chunk_gla's step, the headline)
    qg, kg, vg = (x.detach().clone().requires_grad_() for x in (q, k, v))
    gvg, h0g = gk.detach().clone().requires_grad_(), h0.detach().clone().requires_grad_()
    dog = torch.randn(B2, T2, H2, D2, device=dev, generator=gen).to(bf)

    def gv_train():
        og, _ = fused_recurrent_gla(qg, kg, vg, None, gv=gvg, initial_state=h0g,
                                    output_final_state=True)
        return torch.autograd.grad(og, (qg, kg, vg, gvg, h0g), dog)
    sec_gvt = _time(gv_train, iters)
    del qg, kg, vg, gvg, h0g, dog
    torch.cuda.synchronize()
    if leg is not None:
        hq, hk, hv, hg, hh0 = (_host(x) for x in (q, k, v, gk, h0))
        leg.add("2", B2 * T2, {"fwd": sec * 1e3},
                lambda: dict(zip(("o", "ht"), TC.chunk_gla_fwd_bwd(hq, hk, hv, hg, hh0, None, None,
                                                                   D2 ** -0.5, backward=False))),
                None, {"o": _host(o), "ht": _host(ht)}, 2e-3)
    algo = 419_430_400

    def frac(s):
        return round(algo / s / 1e9 / HBM_PEAK_GBS, 4)
    return {"config": "BASELINE config 2: fused_recurrent_gla fwd B16 T2048 H8 K=V=128 bf16",
            "tokens_per_s": round(B2 * T2 / sec, 1), "ms": round(sec * 1e3, 4),
            "algo_bytes": algo, "hbm_gbs": round(algo / sec / 1e9, 1), "hbm_frac": frac(sec),
            "reverse": {"ms": round(sec_rev * 1e3, 4), "hbm_frac": frac(sec_rev)},
            "gv": {"ms": round(sec_gv * 1e3, 4), "hbm_frac": frac(sec_gv)},
            "gv_train_ms": round(sec_gvt * 1e3, 4)}


def _config4(dev, gen, iters, leg):
    """config 4: simple GLA, T_total 16384 in 8 seeded varlen sequences, H32 K=V=128, bf16."""
    import numpy as np
    import torch
    from oracle import torch_cpu as TC
    from tops.ops.simple_gla import chunk_simple_gla
    bf = torch.bfloat16
    T4, H4, D2 = 16384, 32, 128
    rng = np.random.Generator(np.random.PCG64(1004))
    cu = [0] + sorted(int(c) for c in rng.choice(np.arange(1, T4), 7, replace=False)) + [T4]
    q, k, v = (torch.randn(1, T4, H4, D2, device=dev, generator=gen).to(bf).requires_grad_()
               for _ in range(3))
    g = torch.nn.functional.logsigmoid(torch.randn(1, T4, H4, device=dev, generator=gen)).requires_grad_()
    do = torch.randn(1, T4, H4, D2, device=dev, generator=gen).to(bf)

    def step4():
        o, _ = chunk_simple_gla(q, k, v, None, g=g, cu_seqlens=cu)
        return (o,) + torch.autograd.grad(o, (q, k, v, g), do)
    sec = _time(step4, iters)
    with torch.no_grad():
        sec_f = _time(lambda: chunk_simple_gla(q, k, v, None, g=g, cu_seqlens=cu), iters)
    res = step4()
    torch.cuda.synchronize()
    if leg is not None:
        hq, hk, hv, hg, hdo = (_host(x) for x in (q, k, v, g, do))
        names = ("o", "ht", "dq", "dk", "dv", "dg", "dh0")
        sc = D2 ** -0.5
        leg.add("4", T4, {"fwd": sec_f * 1e3, "fwd_bwd": sec * 1e3},
                lambda: dict(zip(names[:2], TC.chunk_simple_gla_fwd_bwd(
                    hq, hk, hv, hg, sc, cu_seqlens=cu, backward=False))),
                lambda: dict(zip(names, TC.chunk_simple_gla_fwd_bwd(hq, hk, hv, hg, sc, do=hdo,
                                                                    cu_seqlens=cu))),
                dict(zip(("o", "dq", "dk", "dv", "dg"), (_host(x) for x in res))), 2e-3)
    return {"config": "BASELINE config 4: chunk_simple_gla fwd+bwd, varlen T16384 (8 seqs) "
                      "H32 K=V=128 bf16, per-token g",
            "tokens_per_s": round(T4 / sec, 1), "ms": round(sec * 1e3, 4),
            "fwd_ms": round(sec_f * 1e3, 4),
            "hbm_floor_ms": round(1.483e9 / (HBM_PEAK_GBS * 1e9) * 1e3, 4)}


def _config5(dev, gen, iters, leg):
    """config 5: KDA B4 T8192 H32 K=V=128; q, k L2-normalised, bf16 q/k/v, fp32 g, beta."""
    import torch
    from oracle import torch_cpu as TC
    from tops.ops.kda import chunk_kda
    bf = torch.bfloat16
    B5, T5, H5, D2 = 4, 8192, 32, 128

    def l2n(x):
        return x / torch.sqrt((x * x).sum(-1, keepdim=True) + 1e-6)
    q, k = (l2n(torch.randn(B5, T5, H5, D2, device=dev, generator=gen)).to(bf).requires_grad_()
            for _ in range(2))
    v = torch.randn(B5, T5, H5, D2, device=dev, generator=gen).to(bf).requires_grad_()
    beta = torch.sigmoid(torch.randn(B5, T5, H5, device=dev, generator=gen)).requires_grad_()
    g = (torch.nn.functional.logsigmoid(torch.randn(B5, T5, H5, D2, device=dev, generator=gen))
         / 16).requires_grad_()
    do = torch.randn(B5, T5, H5, D2, device=dev, generator=gen).to(bf)

    def step5():
        o, ht = chunk_kda(q, k, v, g, beta, output_final_state=True)
        return (o, ht) + torch.autograd.grad(o, (q, k, v, g, beta), do)
    sec = _time(step5, iters)
    with torch.no_grad():
        sec_f = _time(lambda: chunk_kda(q, k, v, g, beta, output_final_state=True), iters)
    res = step5()
    torch.cuda.synchronize()
    if leg is not None:
        hq, hk, hv, hg, hb, hdo = (_host(x) for x in (q, k, v, g, beta, do))
        names = ("o", "ht", "dq", "dk", "dv", "dbeta", "dg", "dh0")
        sc = D2 ** -0.5
        leg.add("5", B5 * T5, {"fwd": sec_f * 1e3, "fwd_bwd": sec * 1e3},
                lambda: dict(zip(names[:2], TC.chunk_kda_fwd_bwd(hq, hk, hv, hg, hb, sc,
                                                                 backward=False))),
                lambda: dict(zip(names, TC.chunk_kda_fwd_bwd(hq, hk, hv, hg, hb, sc, do=hdo))),
                dict(zip(("o", "ht", "dq", "dk", "dv", "dg", "dbeta"), (_host(x) for x in res))),
                2e-3)
    # input/output floor: fwd reads q, k, v (bf16), g (fp32), writes o; bwd reads q, k, v, g, dO,
    # writes dq, dk, dv (bf16), dg (fp32); beta / dbeta
    n5 = B5 * T5 * H5 * D2
    io5 = n5 * (2 * 3 + 4 + 2) + n5 * (2 * 4 + 4 + 2 * 3 + 4) + B5 * T5 * H5 * 4 * 3
    return {"config": "BASELINE config 5: chunk_kda fwd+bwd B4 T8192 H32 K=V=128 bf16",
            "tokens_per_s": round(B5 * T5 / sec, 1), "ms": round(sec * 1e3, 4),
            "fwd_ms": round(sec_f * 1e3, 4),
            "io_bytes": io5, "hbm_floor_ms": round(io5 / (HBM_PEAK_GBS * 1e9) * 1e3, 4)}


def traffic_from_profiles(kernel):
    """HBM bytes per launch measured with rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE
    (calibrated against a copy kernel), if the committed summary holds the kernel."""
    path = os.path.join(ROOT, "profiles", "traffic_chunk_gla_config3.json")
    try:
        with open(path) as f:
            return json.load(f)["kernels"][kernel]["hbm_bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-secondary", action="store_true", help="skip the config 1 / 2 / 4 / 5 lines")
    ap.add_argument("--configs", default="1,2,4,5,6,7",
                    help="secondary configs to measure (1, 2, 4, 5: BASELINE configs; 6: the "
                         "gate / norm / conv kernels, 7: decode steps)")
    ap.add_argument("--only-secondary", action="store_true",
                    help="measure only the secondary configs (for profiling them alone)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="after the timed steps, copy a 1 GiB fp32 buffer 3 times: the known-size "
                         "kernel that calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE")
    a = ap.parse_args()
    configs = tuple(int(x) for x in a.configs.split(",") if x)
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the GLA hot path shards over (batch, head) "
              "with no communication, so a multi-GPU figure adds nothing here; run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)

    import torch
    from tops import _native as NT
    from tops.ops.gla import chunk_gla
    dev = torch.device("cuda:0")
    NT.lib()
    if a.only_secondary:
        print(json.dumps({"secondary": secondary(dev, iters=a.steps, configs=configs)}), flush=True)
        return
    q, k, v, g, h0, do, dht = make_inputs(dev)
    ins = (q, k, v, g, h0)

    def step():
        o, ht = chunk_gla(q, k, v, g, initial_state=h0, output_final_state=True)
        return torch.autograd.grad((o, ht), ins, (do, dht))

    # The GPU's clock ramps up over the first ~30 ms of work after an idle period (per-step
    # times at this shape fall from ~1.5 ms to their steady value over ~25 steps, and do so
    # again after 2 s of idle).  Untimed steps until 60 ms of wall time have passed settle it
    # before the W warmup steps, so that the K timed steps measure the steady rate of a
    # training loop; the number of settling steps is reported in the line.
    step()                     # the first call also loads code objects and allocates
    torch.cuda.synchronize()
    settle = 1
    t_s = time.perf_counter()
    while time.perf_counter() - t_s < 0.06:
        for _ in range(5):
            step()
        settle += 5
        torch.cuda.synchronize()
    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize()
    NT.enable_timing(True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(a.steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ev = NT.timing_events()
    NT.enable_timing(False)
    if a.copy_calibration:
        src = torch.zeros(1 << 28, device=dev, dtype=torch.float32)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    elapsed = t1 - t0
    ms_step = elapsed * 1e3 / a.steps
    value = B * T * a.steps / elapsed

    kern = {}
    for name, info in KERNELS.items():
        ms = [e0.elapsed_time(e1) for e0, e1 in ev.get(name, []) + ev.get(info["entry"], [])]
        if not ms:
            continue
        avg = sum(ms) / len(ms)
        kern[name] = dict(kernel=info["kernel"], avg_ms=round(avg, 4), launches=len(ms),
                          algo_bytes=info["bytes"],
                          achieved_gbs=round(info["bytes"] / (avg * 1e-3) / 1e9, 1))
    dom = max(kern, key=lambda n: kern[n]["avg_ms"])
    dk = kern[dom]
    roofline = {"bound": "hbm", "achieved": dk["achieved_gbs"], "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(dk["achieved_gbs"] / HBM_PEAK_GBS, 4),
                "traffic": traffic_from_profiles(dk["kernel"]), "kernel": dk["kernel"],
                "avg_ms": dk["avg_ms"], "algo_bytes_per_launch": dk["algo_bytes"]}
    t_floor = PATH_BYTES / (HBM_PEAK_GBS * 1e9)
    path = {"algo_bytes": PATH_BYTES, "algo_flops": PATH_FLOPS,
            "hbm_floor_ms": round(t_floor * 1e3, 4),
            "frac_of_roofline": round(t_floor / (ms_step * 1e-3), 4),
            "mfma_frac": round(PATH_FLOPS / (ms_step * 1e-3) / (MFMA_BF16_PEAK_TFS * 1e12), 4)}
    leg = None if a.no_cpu else CpuLeg()
    # the forward alone, and one more step whose outputs go to the parity check (untimed)
    with torch.no_grad():
        sec_f = _time(lambda: chunk_gla(q, k, v, g, initial_state=h0, output_final_state=True), 10)
        o3, ht3 = chunk_gla(q, k, v, g, initial_state=h0, output_final_state=True)
    grads3 = step()
    torch.cuda.synchronize()
    if leg is not None:
        from oracle import torch_cpu as TC
        hq, hk, hv, hg, hh0, hdo, hdht = (_host(x) for x in (q, k, v, g, h0, do, dht))
        names = ("o", "ht", "dq", "dk", "dv", "dg", "dh0")
        leg.add("3", B * T, {"fwd": sec_f * 1e3, "fwd_bwd": ms_step},
                lambda: dict(zip(names[:2], TC.chunk_gla_fwd_bwd(hq, hk, hv, hg, hh0, None, None,
                                                                 K ** -0.5, C, backward=False))),
                lambda: dict(zip(names, TC.chunk_gla_fwd_bwd(hq, hk, hv, hg, hh0, hdo, hdht,
                                                             K ** -0.5, C))),
                dict(zip(names, (_host(x) for x in (o3, ht3) + tuple(grads3)))), 2e-3)
    del o3, ht3, grads3
    sec_rows = None if a.no_secondary else secondary(dev, configs=configs, leg=leg)
    cpu, parity = None, None
    if leg is not None:
        res, threads = leg.run()
        cpu = cpu_summary(res, threads)
        parity = {"reference": "torch-CPU float32 restatement of tops/cpu on the GPU run's own "
                               "inputs (oracle/torch_cpu.py, pinned to the float64 oracle at 1e-5)",
                  "metric": "relative L2 error per output, ||gpu - ref|| / ||ref||",
                  "configs": {name: row["parity"] for name, row in res.items()}}
    out = {"metric": METRIC, "value": round(value, 1), "unit": "tokens/s", "n_gpus": 1,
           "steps": a.steps, "warmup": a.warmup, "settle_steps": settle,
           "ms_per_step": round(ms_step, 4),
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
           "data": "synthetic",
           "config": {"workload": "chunk_gla fwd+bwd (BASELINE config 3)", "B": B, "T": T,
                      "H": H, "K": K, "V": V, "chunk": C, "h0": True, "dht": True},
           "fwd_ms": round(sec_f * 1e3, 4),
           "roofline": roofline, "path_roofline": path, "kernels": kern,
           "parity": parity, "secondary": sec_rows, "cpu_baseline": cpu}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
