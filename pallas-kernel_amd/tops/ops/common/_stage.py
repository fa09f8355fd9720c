"""Host helpers shared by the stage functions: dtype plumbing around the HIP stage kernels
(which read float32 or bfloat16 q / k / v / do and float32 gates, states and gradients)."""
from __future__ import annotations

import functools

import torch

from ... import _native as N

KERNEL_DTYPES = (torch.float32, torch.bfloat16)


def require(cond, msg: str) -> None:
    if not cond:
        raise AssertionError(msg)


def promoted(*ts) -> torch.dtype:
    """The dtype JAX / torch promotion gives the reference's result for these inputs."""
    return functools.reduce(torch.promote_types, [t.dtype for t in ts if t is not None])


def act(*ts):
    """q / k / v / do in one kernel dtype (their promoted dtype when float32 / bfloat16,
    else float32), contiguous.  Returns (tensors, dtype code)."""
    dt = promoted(*ts)
    kdt = dt if dt in KERNEL_DTYPES else torch.float32
    N.require_cuda(*ts)
    return [t.to(kdt).contiguous() for t in ts], N.dtype_code(kdt)


def f32(t):
    """float32 contiguous copy (or the tensor itself when it already is), None passes."""
    if t is None:
        return None
    N.require_cuda(t)
    return t.to(torch.float32).contiguous()


def finish(out: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    return out if out.dtype == dtype else out.to(dtype)


def chunk_size_ok(C: int) -> None:
    require(C in (16, 32, 64, 128), f"chunk_size must be 16, 32, 64 or 128 on this backend, got {C}")


def cu_host(cu):
    """cu_seqlens as a host int list (None passes)."""
    if cu is None:
        return None
    if isinstance(cu, torch.Tensor):
        return [int(x) for x in cu.detach().cpu().tolist()]
    return [int(x) for x in cu]
