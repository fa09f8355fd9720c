"""Per-phase clock breakdown of the pipelined chunk sweep (gla_pipe_kernel) at a chunk_gla
shape, from the instrumented library (built by ``python pallas-kernel_amd/build.py
--phase-clocks``; the regular library compiles no clocks).

    python pallas-kernel_amd/phase_clocks.py [--B 8 --T 4096 --H 16 --K 128 --V 128]

Runs the forward training sweep (fp16 checkpoints), the reverse training sweep (dh, fp16
checkpoints) and the inference forward (no checkpoints) on synthetic bf16 inputs (q, k, v /
dO ~ N(0, 1), g = logsigmoid(N(0, 1)) / 16), and prints, per sweep, the shader-clock cycles
per chunk that each wave spends in the six intervals of the chunk loop (mean over the waves
of all workgroups; waves 0-1 also compute the two D tiles past the eighth), the clock rate
seen by the waves (s_memtime over s_memrealtime) and the kernel's own time (HIP events).
A wave's time between two barriers is its own work in that phase; its wait at the barrier
is the rest of the slowest wave's work.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os

import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "tops", "_lib", "libtops_pipe_clocks.so")
PHASES = ["B1 wait", "plane writes + gate scan", "B2 wait",
          "matrix phase (H^T, checkpoint, D tiles, state update, staging)", "B3 wait",
          "output products"]
NW = 8


def _lib():
    if not os.path.exists(LIB):
        raise RuntimeError(f"{LIB} is missing: python pallas-kernel_amd/build.py --phase-clocks")
    lib = ctypes.CDLL(LIB)
    f = lib.tops_pipe_phase_clocks
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_void_p] * 8 + [ctypes.c_int] * 6 + [ctypes.c_float, ctypes.c_void_p]
    return f


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr() if t is not None else 0)


def run(B, T, H, K, V, reps=5, seed=0):
    fn = _lib()
    dev = torch.device("cuda:0")
    gen = torch.Generator(device="cpu").manual_seed(seed)
    q = torch.randn(B, T, H, K, generator=gen).to(dev, torch.bfloat16)
    k = torch.randn(B, T, H, K, generator=gen).to(dev, torch.bfloat16)
    v = torch.randn(B, T, H, V, generator=gen).to(dev, torch.bfloat16)
    do = torch.randn(B, T, H, V, generator=gen).to(dev, torch.bfloat16)
    g = (F.logsigmoid(torch.randn(B, T, H, K, generator=gen)) / 16).to(dev)
    out = torch.empty(B, T, H, V, device=dev, dtype=torch.bfloat16)
    NT = (T + 63) // 64
    NV = (V + 63) // 64
    ck = torch.empty(B * NT, H, K, V, device=dev, dtype=torch.float16)
    cs = torch.empty(B * NT, H, NV, device=dev, dtype=torch.float32)
    grid = B * H * NV
    clocks = torch.zeros(grid, NW, 8, device=dev, dtype=torch.int64)
    stream = torch.cuda.current_stream(dev)
    scale = K ** -0.5
    res = {}
    for name, y, rev, train in (("forward (training, fp16 checkpoints)", v, 0, True),
                                ("reverse dh (training, fp16 checkpoints)", do, 1, True),
                                ("forward (inference)", v, 0, False)):
        def launch():
            rc = fn(_ptr(q), _ptr(k), _ptr(g), _ptr(y), _ptr(out), _ptr(ck if train else None),
                    _ptr(cs if train else None), _ptr(clocks), B, T, H, K, V, rev,
                    ctypes.c_float(scale), ctypes.c_void_p(stream.cuda_stream))
            if rc != 0:
                raise RuntimeError(f"tops_pipe_phase_clocks returned {rc}")
        launch()
        torch.cuda.synchronize()
        acc = torch.zeros(grid, NW, 8, dtype=torch.float64)
        ms = []
        for _ in range(reps):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            launch()
            e1.record(stream)
            torch.cuda.synchronize()
            ms.append(e0.elapsed_time(e1))
            acc += clocks.cpu().double()
        acc /= reps
        per_chunk = acc[..., :6] / NT                       # [grid, wave, phase]
        mhz = float(acc[..., 6].sum() / acc[..., 7].sum()) * 100.0
        allw = per_chunk.mean(dim=(0, 1))
        w01 = per_chunk[:, :2].mean(dim=(0, 1))
        w27 = per_chunk[:, 2:].mean(dim=(0, 1))
        loop_us = float(acc[..., 6].mean()) / mhz
        perw = per_chunk.mean(dim=0)                       # [wave, phase]
        res[name] = dict(
            phases={p: dict(all=float(allw[i]), waves01=float(w01[i]), waves27=float(w27[i]),
                            per_wave=[round(float(perw[w, i])) for w in range(NW)])
                    for i, p in enumerate(PHASES)},
            cycles_per_chunk=float(allw.sum()), clock_mhz=mhz,
            us_per_chunk=float(allw.sum()) / mhz, loop_us=loop_us,
            kernel_ms_min=min(ms), kernel_ms=sorted(ms)[len(ms) // 2], chunks=NT, workgroups=grid)
    return res


def markdown(res, shape):
    lines = []
    for name, r in res.items():
        lines.append(f"### {name}\n")
        lines.append(f"{shape}; {r['workgroups']} workgroups x 8 waves, {r['chunks']} chunks each; "
                     f"kernel {r['kernel_ms']:.4f} ms (HIP events, median; min {r['kernel_ms_min']:.4f}); "
                     f"waves' clock {r['clock_mhz']:.0f} MHz; chunk loop {r['loop_us']:.1f} us per "
                     f"wave, {r['us_per_chunk']:.3f} us per chunk\n")
        lines.append("| interval | cycles / chunk (all waves) | waves 0-1 | waves 2-7 | share |")
        lines.append("|---|---|---|---|---|")
        tot = r["cycles_per_chunk"]
        for p, d in r["phases"].items():
            lines.append(f"| {p} | {d['all']:.0f} | {d['waves01']:.0f} | {d['waves27']:.0f} | "
                         f"{100 * d['all'] / tot:.1f}% |")
        lines.append(f"| total | {tot:.0f} | | | |\n")
        lines.append("| interval | " + " | ".join(f"wave {w}" for w in range(NW)) + " |")
        lines.append("|---|" + "---|" * NW)
        for p, d in r["phases"].items():
            lines.append(f"| {p} | " + " | ".join(str(x) for x in d["per_wave"]) + " |")
        lines.append("")
    return "\n".join(lines)


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    for a, d in (("B", 8), ("T", 4096), ("H", 16), ("K", 128), ("V", 128)):
        ap.add_argument(f"--{a}", type=int, default=d)
    ap.add_argument("--json", action="store_true")
    a = ap.parse_args()
    r = run(a.B, a.T, a.H, a.K, a.V)
    shape = f"B={a.B} T={a.T} H={a.H} K={a.K} V={a.V} bf16"
    print(json.dumps(r) if a.json else markdown(r, shape))
