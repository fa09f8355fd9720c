"""GPU test helpers: move seeded numpy inputs to the device, compare with the oracle."""
import numpy as np
import torch

from _closed_forms import rel  # noqa: F401
from _inputs import bf16_round


def to_dev(x, dtype, device):
    if x is None:
        return None
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(device=device, dtype=dtype)


def seen(x, dtype):
    """The values the kernel actually sees (bf16-rounded for bf16 inputs), as float64."""
    if x is None:
        return None
    x = np.asarray(x, np.float32)
    return (bf16_round(x) if dtype == torch.bfloat16 else x).astype(np.float64)


def host(t):
    return None if t is None else t.detach().float().cpu().numpy().astype(np.float64)


def tol(dtype):
    """fp32 rel-err <= 1e-4, bf16 paths <= 2e-3."""
    return 1e-4 if dtype == torch.float32 else 2e-3


def out_bound(ref, dtype, stored):
    """Bound on rel-err against the unrounded float64 oracle for an output stored in `stored`
    dtype: the north-star 2e-3 for bf16 (1e-4 for fp32).  Rounding a bf16 result alone costs
    about 1.5e-3 of relative L2 error on average, and on a tensor of a few dozen elements
    (T = 1, small heads) that sample can itself exceed 2e-3; there the bound is the error of
    the correctly rounded oracle plus 2.5e-4, i.e. the kernel may add no more than that to the
    rounding any bf16 result must carry."""
    lim = tol(dtype)
    if stored != torch.bfloat16 or ref is None:
        return lim
    floor = rel(seen(ref, torch.bfloat16), ref)
    return max(lim, floor + 2.5e-4)
