"""Host-side helpers mirroring tops/utils.py (varlen chunk maps, ceil-div)."""
from __future__ import annotations

from collections import OrderedDict

import numpy as np
import torch

from . import _native as N

CHUNK = 64  # tile length of every chunked kernel


def cdiv(x: int, y: int) -> int:
    """tops/utils.py:19-26."""
    return (x + y - 1) // y


def inference_inputs(*ts):
    """The op's tensor arguments as its autograd Function should see them: detached when grad
    mode is off (torch.no_grad / inference_mode), since a Function's forward sees
    needs_input_grad = True for inputs that require grad even then, and would keep the
    backward's state checkpoints for a backward that cannot run."""
    if torch.is_grad_enabled():
        return ts
    return tuple(t.detach() if isinstance(t, torch.Tensor) else t for t in ts)


def _host_cu(cu_seqlens) -> np.ndarray:
    if isinstance(cu_seqlens, torch.Tensor):
        cu_seqlens = cu_seqlens.detach().cpu().numpy()
    return np.ascontiguousarray(np.asarray(cu_seqlens, dtype=np.int32))


def prepare_lens(cu_seqlens) -> np.ndarray:
    """tops/utils.py:63-68."""
    cu = _host_cu(cu_seqlens)
    return cu[1:] - cu[:-1]


def prepare_chunk_indices(cu_seqlens, chunk_size: int) -> np.ndarray:
    """[total_NT, 2] int32 (sequence id, chunk id): tops/utils.py:71-90, built by the
    native host routine tops_prepare_chunk_indices."""
    cu = _host_cu(cu_seqlens)
    n = len(cu) - 1
    cap = int(cu[-1]) // chunk_size + n
    offs = np.empty(n + 1, np.int32)
    idx = np.empty((max(cap, 1), 2), np.int32)
    total = N._fn("tops_prepare_chunk_indices")(cu.ctypes.data, n, chunk_size, offs.ctypes.data,
                                               idx.ctypes.data, cap)
    if total < 0:
        raise ValueError(N.lib().tops_last_error().decode())
    return idx[:total].copy()


def _upload(a: np.ndarray, device) -> torch.Tensor:
    """One int32 host array to the device; staged through pinned memory so the copy is
    queued on the current stream instead of draining it."""
    return to_device(a, device, torch.int32)


_NP = {torch.int32: np.int32, torch.int64: np.int64, torch.bool: np.bool_, torch.float32: np.float32}


def to_device(a, device, dtype=torch.int32) -> torch.Tensor:
    """A small host array (list, numpy array or CPU tensor) on `device`, staged through pinned
    memory and queued on the current stream behind the work already there.  A copy from
    pageable memory instead was seen to land in a block the caching allocator had just
    recycled before a queued kernel had finished reading it (a temporary freed on the host
    while its reader was still queued); device tensors are only converted."""
    if isinstance(a, torch.Tensor):
        if a.device.type != "cpu":
            return a.to(device=device, dtype=dtype)
        t = a.to(dtype).contiguous()
    else:
        t = torch.from_numpy(np.ascontiguousarray(np.asarray(a), _NP[dtype]))
    if torch.device(device).type == "cuda":
        return t.pin_memory().to(device, non_blocking=True)
    return t.to(device)


def _split_views(t: torch.Tensor, sizes):
    out, o = [], 0
    for n in sizes:
        out.append(t[o:o + n])
        o += n
    return out


_PLANS: "OrderedDict" = OrderedDict()
_PLANS_MAX = 32


class ChunkPlan:
    """Chunk bookkeeping of one call: sequences, global chunk offsets, device maps (one
    device array, uploaded once)."""

    @classmethod
    def get(cls, B: int, T: int, cu_seqlens, device, C: int = CHUNK) -> "ChunkPlan":
        """The plan for these sizes / sequence boundaries, reused across calls (the maps
        depend only on the boundaries)."""
        cu = None if cu_seqlens is None else _host_cu(cu_seqlens)
        key = (B, T, C, str(torch.device(device)), None if cu is None else cu.tobytes())
        plan = _PLANS.get(key)
        if plan is None:
            plan = cls(B, T, cu, device, C)
            _PLANS[key] = plan
            if len(_PLANS) > _PLANS_MAX:
                _PLANS.popitem(last=False)
        else:
            _PLANS.move_to_end(key)
        return plan

    def __init__(self, B: int, T: int, cu_seqlens, device, C: int = CHUNK):
        self.C = C
        self.varlen = cu_seqlens is not None
        if self.varlen:
            cu = _host_cu(cu_seqlens)
            self.N = len(cu) - 1
            idx = prepare_chunk_indices(cu, C)
            self.total = idx.shape[0]
            offs = np.zeros(self.N + 1, np.int32)
            np.cumsum(np.bincount(idx[:, 0], minlength=self.N), out=offs[1:])
            dev = _upload(np.concatenate([cu, offs, idx[:, 0]]), device)
            self.cu_dev, self.offsets_dev, self.chunk_map_dev = _split_views(
                dev, (self.N + 1, self.N + 1, self.total))
        else:
            self.N = B
            self.total = B * cdiv(T, C)
            self.cu_dev = self.offsets_dev = self.chunk_map_dev = None
            cu = np.arange(B + 1, dtype=np.int32) * T
        self.cu_host = cu
        self.device = device
        self._seg = {}

    def segments(self, H: int, V: int):
        """The sequence-parallel split of this call for H heads and V columns (a SegPlan),
        or None when every sequence sweeps whole."""
        key = (H, V, _SPLIT["mode"])
        if key not in self._seg:
            self._seg[key] = SegPlan.build(self, H, V)
        return self._seg[key]


# Sequence-parallel sweeps.  A sweep runs one workgroup per (sequence, head, 64-column
# V tile) and walks that sequence's chunks in order, so a call whose sequences are few or
# unequal leaves CUs idle while its longest sequence finishes.  Such sequences are cut
# at chunk boundaries into segments that sweep concurrently (tops_chunk_state_pass /
# tops_chunk_state_combine in include/tops_hip.h).
_SPLIT = {"mode": None}   # None: automatic; 0: never split; k > 0: segments of k chunks
MIN_SEG_CHUNKS = 8        # shortest segment worth its state pass
MIN_PIECE_CHUNKS = 4      # shortest state-pass piece
SPLIT_SLACK = 1.25        # split a sequence only when it is this much above the target


def set_sequence_split(mode=None) -> None:
    """None: split long sequences when the CUs would otherwise idle (default); 0: never;
    an integer k > 0: cut every sequence into ceil(chunks / k) near-equal segments."""
    if mode is not None and (not isinstance(mode, int) or mode < 0):
        raise ValueError("set_sequence_split takes None or an integer >= 0")
    _SPLIT["mode"] = mode


# Residual states of the GLA / simple-GLA training path.  "full": the forward keeps the
# state before every chunk and the backward's reverse sweep writes dh for every chunk
# (2 x chunks x H x K x V).  For bf16 inputs with per-channel gates (chunk_gla, K, V <= 128)
# these are fp16 times a power-of-two factor per (chunk, head, 64 columns of V); other
# calls keep fp32.  "full32": fp32 everywhere.  "paired" (bf16 inputs): one fp32 buffer of
# chunks x H x K x V holding h before the even chunks and dh after the odd ones; the dq / dk
# / dg kernel rebuilds the rest from each chunk's pair partner.  Half the memory and
# checkpoint bytes of "full32", but the rebuild needs both chunks of a pair on one CU.
_CKPT = {"layout": "full"}


def set_checkpoint_layout(layout: str = "full") -> None:
    """"full" (default), "full32" or "paired": see the comment above."""
    if layout not in ("full", "full32", "paired"):
        raise ValueError("set_checkpoint_layout takes 'full', 'full32' or 'paired'")
    _CKPT["layout"] = layout


def checkpoint_layout() -> str:
    return _CKPT["layout"]


def _device_cus(device) -> int:
    return int(torch.cuda.get_device_properties(device).multi_processor_count)


class SegPlan:
    """Segments of the sequences of one ChunkPlan, in token order, and the state-pass pieces
    of both sweep directions (host arrays and their device copies):
      cu_dev [Nv+1]        segment boundaries (a varlen layout over the same tokens)
      offsets_dev [Nv+1]   first global chunk of each segment (the plan's chunk numbering)
      seg_first_dev [N+1]  segments of real sequence n: [seg_first[n], seg_first[n+1])
      last_dev, first_dev  [N] last / first segment of every real sequence
      fwd / rev            a Pieces: the rows each state-pass workgroup sweeps, grouped per
                           sequence in sweep order, and the segment each piece hands into
    A piece is a segment that hands a state on (all but the last of a sequence forward, all
    but the first in reverse), cut into ``sub``-chunk parts when the pass alone would leave
    the device idle."""

    class Pieces:
        def __init__(self, start, end, first, dst):
            self.n = len(start)
            self.start, self.end = np.array(start, np.int32), np.array(end, np.int32)
            self.first, self.dst = np.array(first, np.int32), np.array(dst, np.int32)

    @staticmethod
    def split_counts(chunks: np.ndarray, slots: int, mode) -> np.ndarray:
        """Segments per sequence.  Automatic: aim at total/slots chunks per segment (at least
        MIN_SEG_CHUNKS) and split only sequences above SPLIT_SLACK times that."""
        if mode == 0:
            return np.ones_like(chunks)
        if mode is not None:
            return np.maximum(1, -(-chunks // mode))
        target = max(-(-int(chunks.sum()) // max(slots, 1)), MIN_SEG_CHUNKS)
        m = -(-chunks // target)
        return np.where(chunks > SPLIT_SLACK * target, m, 1)

    @staticmethod
    def piece_chunks(state_chunks: int, wgs_per_piece: int, cus: int) -> int:
        """Piece length (chunks) so that the state pass is about one round of workgroups on
        `cus` CUs (one state-pass workgroup per CU), at least MIN_PIECE_CHUNKS."""
        return max(-(-state_chunks * wgs_per_piece // max(cus, 1)), MIN_PIECE_CHUNKS)

    @classmethod
    def build(cls, plan: "ChunkPlan", H: int, V: int):
        cu = plan.cu_host.astype(np.int64)
        lens = cu[1:] - cu[:-1]
        C = plan.C
        chunks = -(-lens // C)
        mode = _SPLIT["mode"]
        if mode == 0:
            return None
        per = max(H * cdiv(V, 64), 1)
        cus = _device_cus(plan.device)
        slots = cus // per if mode is None else 1
        m = cls.split_counts(chunks, slots, mode)
        if int(m.max()) <= 1:
            return None
        return cls(cu, chunks, m, C, plan.device, per=per, cus=cus)

    @staticmethod
    def _cut(lo_chunk: int, n_chunks: int, sub: int):
        """[lo, hi) chunk ranges of near-equal parts of at most about `sub` chunks."""
        k = max(1, -(-n_chunks // sub))
        base, rem = divmod(n_chunks, k)
        out, c = [], lo_chunk
        for i in range(k):
            sz = base + (1 if i < rem else 0)
            out.append((c, c + sz))
            c += sz
        return out

    def __init__(self, cu, chunks, m, C, device, per=None, cus=None):
        coff = np.concatenate([[0], np.cumsum(chunks)])
        starts, offs, seg_first = [], [], [0]
        seq_bounds = []                       # per sequence: segment boundaries in chunks
        for n in range(len(chunks)):
            base, rem = divmod(int(chunks[n]), int(m[n]))
            sizes = [base + (1 if j < rem else 0) for j in range(int(m[n]))]
            cb = [0]
            for sz in sizes:
                cb.append(cb[-1] + sz)
            seq_bounds.append(cb)
            for j in range(len(sizes)):
                starts.append(int(cu[n]) + C * cb[j])
                offs.append(int(coff[n]) + cb[j])
            seg_first.append(seg_first[-1] + len(sizes))
        # piece length: one round of state-pass workgroups (pieces = segments when unknown)
        state_chunks = sum(cb[-1] - (cb[-1] - cb[-2]) for cb in seq_bounds if len(cb) > 2)
        sub = self.piece_chunks(state_chunks, per, cus) if per and cus else None

        def row(n, c):                        # token row of chunk boundary c of sequence n
            return min(int(cu[n]) + C * c, int(cu[n + 1]))

        fwd = ([], [], [0], [])
        rev = ([], [], [0], [])
        for n, cb in enumerate(seq_bounds):
            j0, ms = seg_first[n], len(cb) - 1
            # forward: segments 0..ms-2, token order; the piece ending at boundary j + 1
            # hands into segment j + 1
            for j in range(ms - 1):
                parts = self._cut(cb[j], cb[j + 1] - cb[j], sub or (cb[j + 1] - cb[j]))
                for i, (a, b) in enumerate(parts):
                    fwd[0].append(row(n, a))
                    fwd[1].append(row(n, b))
                    fwd[3].append(j0 + j + 1 if i == len(parts) - 1 else -1)
            fwd[2].append(len(fwd[0]))
            # reverse: segments ms-1..1, from the end of the sequence; the piece starting at
            # boundary j hands into segment j - 1
            for j in range(ms - 1, 0, -1):
                parts = self._cut(cb[j], cb[j + 1] - cb[j], sub or (cb[j + 1] - cb[j]))
                for i, (a, b) in enumerate(reversed(parts)):
                    rev[0].append(row(n, a))
                    rev[1].append(row(n, b))
                    rev[3].append(j0 + j - 1 if i == len(parts) - 1 else -1)
            rev[2].append(len(rev[0]))
        self.sub = sub
        self.fwd = self.Pieces(*fwd)
        self.rev = self.Pieces(*rev)
        self.Nv = len(starts)
        cu_v = np.array(starts + [int(cu[-1])], np.int32)
        offs_v = np.array(offs + [int(coff[-1])], np.int32)
        sf = np.array(seg_first, np.int32)
        self.seg_first = sf
        self.cu_host = cu_v
        parts = [cu_v, offs_v, sf, sf[:-1], sf[1:] - 1]
        for pc in (self.fwd, self.rev):
            parts += [pc.start, pc.end, pc.first, pc.dst]
        views = _split_views(_upload(np.concatenate(parts), device), [len(x) for x in parts])
        (self.cu_dev, self.offsets_dev, self.seg_first_dev, self.first_dev, self.last_dev) = views[:5]
        for pc, v in ((self.fwd, views[5:9]), (self.rev, views[9:13])):
            pc.start_dev, pc.end_dev, pc.first_dev, pc.dst_dev = v


# ---- small helpers of tops/utils.py:7-140, on torch tensors (and NumPy arrays) ----

def next_power_of_2(n: int) -> int:
    """Smallest power of 2 >= n (tops/utils.py:7-17)."""
    return 1 if n <= 1 else 1 << (int(n) - 1).bit_length()


def align_up(x: int, align: int) -> int:
    """x rounded up to a multiple of align (tops/utils.py:29-31)."""
    return cdiv(x, align) * align


def pad_to_multiple(x, multiple, axis, val):
    """Pad x at the end of each `axis` to a multiple of `multiple` with `val`
    (tops/utils.py:34-60); ints or equal-length lists."""
    multiple = [multiple] if isinstance(multiple, int) else list(multiple)
    axis = [axis] if isinstance(axis, int) else list(axis)
    assert len(multiple) == len(axis), (
        f"Length of multiple {len(multiple)} must match length of axis {len(axis)}")
    widths = [(0, 0)] * x.ndim
    for ax, mu in zip(axis, multiple):
        rem = x.shape[ax] % mu
        if rem:
            widths[ax] = (0, mu - rem)
    if isinstance(x, np.ndarray):
        return np.pad(x, widths, constant_values=val)
    if not isinstance(x, torch.Tensor):
        raise NotImplementedError(f"pad_to_multiple is not implemented for type {type(x)}")
    flat = [p for w in reversed(widths) for p in w]
    return torch.nn.functional.pad(x, flat, value=val)


def assert_shape(x, expected_shape, name="tensor"):
    """Assert that x (or every tensor of a list / tuple) has expected_shape
    (tops/utils.py:111-124)."""
    exp = tuple(expected_shape)
    if isinstance(x, (list, tuple)):
        named = isinstance(name, (list, tuple)) and len(name) == len(x)
        for i, t in enumerate(x):
            n = name[i] if named else f"{name}_{i}"
            assert tuple(t.shape) == exp, f"[{n}] Expected shape {exp}, got {tuple(t.shape)}"
    else:
        assert tuple(x.shape) == exp, f"[{name}] Expected shape {exp}, got {tuple(x.shape)}"


def assert_shape_or_none(x, expected_shape, name="tensor"):
    """assert_shape skipping None entries (tops/utils.py:92-109)."""
    if x is None:
        return
    if isinstance(x, (list, tuple)):
        named = isinstance(name, (list, tuple)) and len(name) == len(x)
        keep = [(name[i] if named else f"{name}_{i}", t) for i, t in enumerate(x) if t is not None]
        for n, t in keep:
            assert_shape(t, expected_shape, n)
    else:
        assert_shape(x, expected_shape, name)


def export_public(current_globals) -> list:
    """Public names a module defines itself (no leading underscore, not imported, not a
    module) (tops/utils.py:126-140)."""
    import types
    mod = current_globals.get("__name__")
    out = []
    for n, obj in current_globals.items():
        if n.startswith("_") or isinstance(obj, types.ModuleType):
            continue
        if hasattr(obj, "__module__") and obj.__module__ != mod:
            continue
        out.append(n)
    return out
