"""CPU replay of the address arithmetic of the buffer-resource kernels (test infrastructure).

Every global access of gla_sweep_kernel (all instances: GLA / simple-GLA gate modes, the KDA
delta rule, the state-only pass), gla_dqkg_kernel (bf16 / fp32, fp32 v), kda_prep_kernel,
kda_wy_kernel / kda_bwd_fused_kernel and fr_decode_kernel is re-evaluated here per workgroup, chunk and thread, with the kernels' own
thread mappings, masks and (voffset, soffset, width) decomposition.  An access whose voffset
is kOOB is dropped by the hardware and skipped; every other access must lie entirely inside
its tensor.  The launches are derived from the host code's own plans (ChunkPlan / SegPlan of
tops.utils), so the segment path and varlen packing are covered as the ops run them.

The model restates the offset expressions of the .hip sources line by line; it cannot prove
that the kernels compute the same numbers, but it catches a wrong mask, a load wider than its
element run (the 16-byte read of a 4-byte per-token gate), or a range that starts before a
tensor (an empty sequence walked in reverse).
"""
from __future__ import annotations

import numpy as np

KOOB = 0x80000000
C = 64


class OOBError(AssertionError):
    pass


class Checker:
    """Collects accesses; raises on the first one outside its tensor."""

    def __init__(self, sizes: dict):
        self.sizes = sizes          # tensor name -> bytes
        self.count = 0

    def acc(self, name, base, voff, soff, width, what):
        base, voff, soff = (np.asarray(x, np.int64) for x in (base, voff, soff))
        base, voff, soff = np.broadcast_arrays(base, voff, soff)
        live = voff < KOOB
        if not live.any():
            return
        start = (base + voff + soff)[live]
        end = start + width
        nb = self.sizes[name]
        bad = (start < 0) | (end > nb)
        self.count += int(live.sum())
        if bad.any():
            i = int(np.argmax(bad))
            raise OOBError(f"{what}: {name} bytes [{start[i]}, {end[i]}) outside [0, {nb})")

    def rows_rsrc(self, name, e0, nrows, width, es):
        """make_rsrc_rows(t, e0, nrows, width): the range must end inside the tensor."""
        e0 = np.asarray(e0, np.int64)
        base = e0 * width * es
        n = (nrows - e0) * width * es
        n = np.minimum(n, 0x7fffffff)
        if np.any(base + n > self.sizes[name]) or np.any(base < 0):
            raise OOBError(f"resource over {name} runs past the tensor")


def _tid(nth):
    t = np.arange(nth, dtype=np.int64)
    return t, t & 63, t >> 6


def _kp(K):
    return 32 if K <= 32 else (64 if K <= 64 else 128)


# --------------------------------------------------------------------------- gla_sweep_kernel
def sweep(ck: Checker, p: dict, es: int, rev: bool, delta: bool = False, st: bool = False,
          gate_width_bytes: int = 4, unguarded_prefetch: bool = False, gshift: bool = False,
          planted_shift: bool = False, gv: bool = False):
    """gla_sweep_kernel<TIn, KP, REV, DELTA, ST> (csrc/gla_sweep.hip).  p holds the SweepParams
    fields: B, T, H, K, V, N, cu (host array or None), seg_end, offsets, gate_mode and which of
    s0 / s_fin / ckpt / y32 / dec_fin / u / w are bound (tensor names in ck.sizes).  gshift:
    the reverse sweep reads the gate one token later (tops_chunk_reverse_fwd); planted_shift
    moves the gate rows one token earlier in the sequence's first chunk too (the mistake the
    first-chunk case exists for).  gv: the value-gate forward (tops_gla_chunk_fwd_gv): g is
    [B,T,H,V], read as two columns per Y row, and the K-side gate reads nothing."""
    B, T, H, K, V, N = (p[x] for x in ("B", "T", "H", "K", "V", "N"))
    KP = _kp(K)
    NTH, BV = 512, 64
    NV = -(-V // 64)
    NQ = KP // 4
    NSEG = NTH // NQ
    RPT = C // NSEG
    CQL, SGL = 8, 4
    NCQH = NQ // CQL
    NHT = (KP // 16) * (BV // 16) // 8
    YR = 4
    fwd_delta, rev_delta = delta and not rev, delta and rev
    gm = p.get("gate_mode", 0)
    rowK, rowV = H * K, H * V
    nrows = B * T * H
    cu, seg_end, offs = p.get("cu"), p.get("seg_end"), p.get("offsets")

    tid, lane, wave = _tid(NTH)
    l16, lg = lane & 15, lane >> 4
    R, nh = wave >> 1, wave & 1
    msb = (wave * NHT) // (BV // 16)
    hw = tid >> 5
    sgl = (lane & 31) // CQL
    sgh = hw // NCQH
    cq = (lane & 31) % CQL + CQL * (hw % NCQH)
    seg = sgl + SGL * sgh
    c0, r0 = 4 * cq, seg * RPT
    colok = c0 < K
    yc = (lane & 7) + 8 * (hw & 3)
    yseg = ((lane >> 3) & 3) + 4 * (hw >> 2)
    hh = np.arange(H, dtype=np.int64)[:, None, None]             # [H, 1, 1]
    vt = np.arange(NV, dtype=np.int64)[None, :, None]            # [1, NV, 1]
    yv = vt * BV + 2 * yc
    offQ = np.where(colok, (r0 * rowK + c0) * es, KOOB)
    offG = np.where(colok, (r0 * rowK + c0) * 4, KOOB)
    offY = np.where(yv < V, ((yseg * YR) * rowV + yv) * es, KOOB)
    offYg = np.where(yv < V, ((yseg * YR) * rowV + yv) * 4, KOOB)
    if gm == 0:
        offGm, gstride, gw, gname_w = offG, rowK * 4, 16, K
    elif gm == 1:
        offGm, gstride, gw, gname_w = r0 * H * 4, H * 4, gate_width_bytes, 1
    else:
        offGm, gstride, gw, gname_w = np.full_like(r0, KOOB), 0, 0, 1

    if cu is not None:
        for j in range(min(N, 512)):      # the LPT ranking reads cu[j], seq_end(j)
            assert j + 1 < len(cu) or seg_end is not None
    for n in range(N):
        if cu is not None:
            row0 = int(cu[n])
            L = (int(seg_end[n]) if seg_end is not None else int(cu[n + 1])) - row0
            cbase = int(offs[n]) if offs is not None else 0
        else:
            row0, L, cbase = n * T, T, n * (-(-T // C))
        NTs = -(-L // C)
        gsh = gshift and rev and not delta and not st
        if gsh and L > 0:
            # the decay of h0 by the last token's gate (plain loads, kr < K checked)
            el = (row0 + L - 1) * H + hh
            for r in range(4):
                kr = 16 * msb + 4 * lg + r
                if gm == 0:
                    ck.acc(p["g"], 0, np.where(kr < K, (el * K + kr) * 4, KOOB), 0, 4, "sweep g last")
                elif gm == 1:
                    ck.acc(p["g"], 0, el * 4 + 0 * kr, 0, 4, "sweep g last")
                elif gm == 2:
                    ck.acc(p["g"], 0, hh * 4 + 0 * kr, 0, 4, "sweep g_gamma")
                else:
                    ck.acc(p["g"], 0, np.where(kr < K, (hh * K + kr) * 4, KOOB), 0, 4, "sweep g_gamma")
        # the first chunk is prefetched only when there is one (unguarded_prefetch plants the
        # unconditional prefetch, which for an empty sequence walked in reverse is chunk -1)
        walk = [NTs - 1 - it if rev else it for it in range(NTs)]
        if unguarded_prefetch and NTs == 0:
            walk = [-1 if rev else 0]
        # state in / out: [N, H, K, V] fp32 (plain pointers, kr < K and vv < V checked)
        for i in range(NHT):
            nn = (wave * NHT + i) % (BV // 16)
            vv = vt * BV + 16 * nn + l16
            for r in range(4):
                kr = 16 * msb + 4 * lg + r
                ok = (kr < K) & (vv < V)
                idx = np.where(ok, (((n * H + hh) * K + kr) * V + vv) * 4, KOOB)
                for nm in ("s0", "s_fin"):
                    if p.get(nm):
                        ck.acc(p[nm], 0, idx, 0, 4, f"sweep {nm}")
        if st and p.get("dec_fin"):
            for r in range(4):
                kr = 16 * msb + 4 * lg + r
                sel = (vt == 0) & (((wave * NHT) % (BV // 16)) == 0) & (l16 == 0) & (kr < K)
                ck.acc(p["dec_fin"], 0, np.where(sel, ((n * H + hh) * K + kr) * 4, KOOB), 0, 4,
                       "sweep dec_fin")
        for c in walk:
            t0 = c * C
            nval = min(C, L - t0)
            e0 = (row0 + t0) * H + hh
            for nm, w_ in (("q", K), ("k", K)):
                ck.rows_rsrc(p[nm], e0, nrows, w_, es)
            # load_chunk: q, k, g
            for i in range(RPT):
                ok = r0 + i < nval
                for nm in ("q", "k"):
                    ck.acc(p[nm], e0 * K * es, np.where(ok, offQ, KOOB), i * rowK * es, 4 * es,
                           f"sweep load {nm} chunk {c}")
                if gsh:
                    gadj = 1 if (t0 == 0 and not planted_shift) else 0
                    eg = e0 - H if (t0 > 0 or planted_shift) else e0
                    if gm in (0, 1):
                        ck.rows_rsrc(p["g"], eg, nrows, gname_w, 4)
                    rd = ok & (r0 + i >= gadj) & (offGm < KOOB)
                    ck.acc(p["g"], eg * gname_w * 4,
                           np.where(rd, offGm + (i - gadj) * gstride, KOOB), 0, gw,
                           f"sweep load shifted g (mode {gm}) chunk {c}")
                elif gw and not gv:
                    ck.acc(p["g"], e0 * gname_w * 4, np.where(ok, offGm, KOOB), i * gstride, gw,
                           f"sweep load g (mode {gm}) chunk {c}")
            if not fwd_delta:
                for i in range(YR):
                    ok = yseg * YR + i < nval
                    ck.acc(p["y"], e0 * V * es, np.where(ok, offY, KOOB), i * rowV * es, 2 * es,
                           f"sweep load y chunk {c}")
            if gv:
                ck.rows_rsrc(p["g"], e0, nrows, V, 4)
                for i in range(YR):
                    ok = yseg * YR + i < nval
                    ck.acc(p["g"], e0 * V * 4, np.where(ok, offYg, KOOB), i * rowV * 4, 8,
                           f"sweep load gv chunk {c}")
            if fwd_delta:
                trow = 16 * R + l16
                for kc in range(KP // 32):
                    k0 = 32 * kc + 8 * lg
                    o = np.where((trow < nval) & (k0 < K), (trow * rowK + k0) * 4, KOOB)
                    ck.acc(p["w"], e0 * K * 4, o, 0, 32, "sweep load w (delta fwd)")
                for j in range(2):
                    vv = vt * BV + 16 * (2 * nh + j) + l16
                    for r in range(4):
                        tok = 16 * R + 4 * lg + r
                        o = np.where((tok < nval) & (vv < V), (tok * rowV + vv) * 4, KOOB)
                        ck.acc(p["u"], e0 * V * 4, o, 0, 4, "sweep load u")
                        if p.get("y32"):
                            ck.acc(p["y32"], e0 * V * 4, o, 0, 4, "sweep store v_new")
            if rev_delta:
                for i in range(RPT):
                    ck.acc(p["w"], e0 * K * 4, np.where(r0 + i < nval, offG, KOOB), i * rowK * 4,
                           16, "sweep load w (delta rev)")
            if st:
                continue
            if p.get("ckpt"):
                cbase_b = ((cbase + c) * H + hh) * K * V * 4
                for i in range(NHT):
                    nn = (wave * NHT + i) % (BV // 16)
                    kr = 16 * msb + 4 * lg
                    vv = vt * BV + 16 * nn + l16
                    vo = np.where(vv < V, (kr * V + vv) * 4, KOOB)
                    for r in range(4):
                        ck.acc(p["ckpt"], cbase_b, np.where(kr + r < K, vo, KOOB), r * V * 4, 4,
                               "sweep store checkpoint")
            if rev_delta:
                base = ((cbase + c) * H + hh) * V * C * 4
                for j in range(2):
                    vv = vt * BV + 16 * (2 * nh + j) + l16
                    ck.acc(p["y32"], base, np.where(vv < V, (vv * C + 16 * R + 4 * lg) * 4, KOOB),
                           0, 16, "sweep store dv_new^T")
            else:
                tok = 16 * R + l16
                oo = np.where(tok < nval, (tok * rowV + vt * BV + 4 * lg) * es, KOOB)
                for j in range(2):
                    nn = 2 * nh + j
                    v0 = vt * BV + 16 * nn + 4 * lg
                    ck.acc(p["out"], e0 * V * es, np.where(v0 < V, oo, KOOB), 16 * nn * es, 4 * es,
                           "sweep store out")


# --------------------------------------------------------------------------- gla_dqkg_kernel
def _chunks(p):
    """(n, c, row0, L) of every global chunk gc, as the chunk-parallel kernels derive them."""
    out = []
    if p.get("cu") is not None:
        cu, offs, cmap = p["cu"], p["offsets"], p["chunk_map"]
        for gc in range(p["total"]):
            n = int(cmap[gc])
            out.append((gc, n, gc - int(offs[n]), int(cu[n]), int(cu[n + 1]) - int(cu[n])))
    else:
        nt = -(-p["T"] // C)
        for gc in range(p["total"]):
            n = gc // nt
            out.append((gc, n, gc % nt, n * p["T"], p["T"]))
    return out


def dqkg(ck: Checker, p: dict, es: int, esv: int, pair: bool = False, planted_link: bool = False):
    """gla_dqkg_kernel<TIn, TV, KP, VP> (csrc/gla_dqkg.hip).  pair: the PAIR instance
    (interleaved checkpoints in p["hs"]: a workgroup takes global chunks 2i, 2i + 1, each
    with the 256-thread mapping of the unpaired kernel; the state rows are read as two 4-float
    runs, from the chunk's slot and the partner's, or from p["h0"] / p["dht"] of the
    sequence when the partner lies in another one)."""
    H, K, V = p["H"], p["K"], p["V"]
    KP, VP = _kp(K), _kp(V)
    KH, NPS, VC = 32, KP // 32, VP // 32
    EP, EPV = 16 // es, 16 // esv
    NPC, NPCV = VP // EP, VP // EPV
    NPT, NPTV = C * NPC // 256, C * NPCV // 256
    gm = p.get("gate_mode", 0)
    rowK, rowV = H * K, H * V
    nrows = p["B"] * p["T"] * H
    tid, lane, wave = _tid(256)
    l16, lg = lane & 15, lane >> 4
    kb, rh = wave & 1, wave >> 1
    ch, sg = tid & 31, tid >> 5
    scalar_gate_inst = es == esv
    hh = np.arange(H, dtype=np.int64)[:, None]
    chunks = _chunks(p)
    KVB = K * V * 4
    for gc, n, c, row0, L in chunks:
        # the state sources of this chunk: (tensor, base byte offset) for h and dh, or None
        if pair:
            c0 = gc - (gc & 1)
            linked = c0 + 1 < p["total"] and chunks[c0][1] == chunks[c0 + 1][1]
            linked = linked or planted_link     # (a planted mistake: partner always read)
            own = ("hs", (gc * H + hh) * KVB)
            if linked:
                other = ("hs", ((gc + 1 if gc % 2 == 0 else gc - 1) * H + hh) * KVB)
            else:
                nm = p.get("dht") if gc % 2 == 0 else p.get("h0")
                other = (nm, (n * H + hh) * KVB) if nm else None
            states = [own, other]
            runs = [(16 * j, 0) for j in range(2)]          # v0 = 32 vc + 16 j + 4 lg, 16 bytes
        else:
            states = [(p["hs"], (gc * H + hh) * KVB), (p["dhs"], (gc * H + hh) * KVB)]
            runs = [(0, 0), (0, 16)]                        # v0 = 32 vc + 8 lg, 2 x 16 bytes
        t0 = c * C
        nval = min(C, L - t0)
        e0 = (row0 + t0) * H + hh
        ck.rows_rsrc(p["q"], e0, nrows, K, es)
        for i in range(NPTV):
            pc = tid + 256 * i
            row, col = pc // NPCV, (pc % NPCV) * EPV
            ck.acc(p["v"], e0 * V * esv, np.where((row < nval) & (col < V), (row * rowV + col) * esv, KOOB),
                   0, 16, "dqkg load v")
        for i in range(NPT):
            pc = tid + 256 * i
            row, col = pc // NPC, (pc % NPC) * EP
            ck.acc(p["do"], e0 * V * es, np.where((row < nval) & (col < V), (row * rowV + col) * es, KOOB),
                   0, 16, "dqkg load dO")
        for ps in range(NPS):
            kc = ps * KH + ch
            for i in range(8):
                r = 8 * sg + i
                v_ = (kc < K) & (r < nval)
                off = r * rowK + kc
                for nm in ("q", "k"):
                    if es == 4:
                        ck.acc(p[nm], e0 * K * 4, np.where(v_, off * 4, KOOB), 0, 4, "dqkg pass load")
                    else:
                        ck.acc(p[nm], e0 * K * 2, np.where(v_, (off & ~1) * 2, KOOB), 0, 4, "dqkg pass load")
                if gm in (0, 1):      # the constant gates (2: [H], 3: [H, K]) load nothing
                    gstr, gcol, gwid = (rowK * 4, kc * 4, K) if gm == 0 else (H * 4, 0, 1)
                    ck.acc(p["g"], e0 * gwid * 4, np.where(v_, r * gstr + gcol, KOOB), 0, 4,
                           "dqkg load g")
            cb = ps * KH
            kk = cb + 16 * kb + l16
            for vc in range(VC):
                for dv0, soff in runs:
                    v0 = 32 * vc + (4 if pair else 8) * lg + dv0
                    o = np.where((kk < K) & (v0 < V), (kk * V + v0) * 4, KOOB)
                    for st in states:
                        if st is not None:
                            ck.acc(st[0], st[1], o, soff, 16, f"dqkg load state {st[0]}")
            kc4 = cb + 16 * kb + 4 * lg
            for a in range(2):
                tok = 16 * (2 * rh + a) + l16
                ok = (kc4 < K) & (tok < nval)
                off = tok * rowK + kc4
                if not scalar_gate_inst:
                    for nm in ("dk_add", "dg_add"):
                        if p.get(nm):
                            ck.acc(p[nm], e0 * K * 4, np.where(ok, off * 4, KOOB), 0, 16, f"dqkg load {nm}")
                for nm in ("q", "k"):
                    if es == 4:
                        ck.acc(p[nm], e0 * K * 4, np.where(ok, off * 4, KOOB), 0, 16, "dqkg epilogue load")
                for nm in ("dq", "dk"):
                    ck.acc(p[nm], e0 * K * es, np.where(ok, off * es, KOOB), 0, 4 * es, f"dqkg store {nm}")
                if gm in (0, 3) and p.get("dg"):
                    ck.acc(p["dg"], e0 * K * 4, np.where(ok, off * 4, KOOB), 0, 16, "dqkg store dg")
        if gm == 1 and p.get("dg"):
            ck.acc(p["dg"], e0 * 4, np.where(tid < nval, tid * H * 4, KOOB), 0, 4, "dqkg store dg (scalar)")


# --------------------------------------------------------------------------- KDA kernels
def kda_prep(ck: Checker, p: dict, es: int):
    """kda_prep_kernel<TIn, KP, VP> (csrc/kda_prep.hip)."""
    H, K, V = p["H"], p["K"], p["V"]
    KP, VP = _kp(K), _kp(V)
    NQ, NQV = KP // 4, VP // 4
    RPT, RPTV = C // (256 // NQ), C // (256 // NQV)
    KH2, VH2 = min(KP, 64), min(VP, 64)
    NKP, NVP = KP // KH2, VP // VH2
    rowK, rowV = H * K, H * V
    tid, lane, wave = _tid(256)
    l16, lg = lane & 15, lane >> 4
    hw = tid >> 5
    CQL = min(NQ, 8); SGL = 32 // CQL; NCQH = NQ // CQL
    cq = (lane & 31) % CQL + CQL * (hw % NCQH)
    seg = (lane & 31) // CQL + SGL * (hw // NCQH)
    c0, r0 = 4 * cq, seg * RPT
    offK = np.where(c0 < K, (r0 * rowK + c0) * es, KOOB)
    offG = np.where(c0 < K, (r0 * rowK + c0) * 4, KOOB)
    CQLV = min(NQV, 8); SGLV = 32 // CQLV; NCQHV = NQV // CQLV
    cv = (lane & 31) % CQLV + CQLV * (hw % NCQHV)
    sv = (lane & 31) // CQLV + SGLV * (hw // NCQHV)
    vc0, rv0 = 4 * cv, sv * RPTV
    offV = np.where(vc0 < V, (rv0 * rowV + vc0) * es, KOOB)
    R = wave
    hh = np.arange(H, dtype=np.int64)[:, None]
    for gc, n, c, row0, L in _chunks(p):
        nval = min(C, L - c * C)
        e0 = (row0 + c * C) * H + hh
        for i in range(RPT):
            ok = r0 + i < nval
            ck.acc(p["k"], e0 * K * es, np.where(ok, offK, KOOB), i * rowK * es, 4 * es, "prep load k")
            ck.acc(p["g"], e0 * K * 4, np.where(ok, offG, KOOB), i * rowK * 4, 16, "prep load g")
        for i in range(RPTV):
            ck.acc(p["v"], e0 * V * es, np.where(rv0 + i < nval, offV, KOOB), i * rowV * es, 4 * es,
                   "prep load v")
        ck.acc(p["beta"], e0 * 4, np.where((tid < C) & (tid < nval), tid * H * 4, KOOB), 0, 4, "prep load beta")
        tok = 16 * R + l16
        for up in range(max(NKP, NVP)):
            if up < NVP:
                for vb in range(VH2 // 16):
                    col = up * VH2 + 16 * vb + 4 * lg
                    ck.acc(p["u"], e0 * V * 4, np.where((tok < nval) & (col < V), (tok * rowV + col) * 4, KOOB),
                           0, 16, "prep store u")
            if up < NKP:
                for kb in range(KH2 // 16):
                    col = up * KH2 + 16 * kb + 4 * lg
                    ck.acc(p["w"], e0 * K * 4, np.where((tok < nval) & (col < K), (tok * rowK + col) * 4, KOOB),
                           0, 16, "prep store w")
        if p.get("tt"):
            i, qq = tid >> 2, tid & 3
            for e in range(4):
                j0 = 16 * qq + 4 * e
                ck.acc(p["tt"], (gc * H + hh) * C * C * 4, (i * C + j0) * 4, 0, 16, "prep store T^T")


def kda_wy(ck: Checker, p: dict, es: int, fused: bool = False):
    """kda_wy_kernel<TIn, KP, VP> (csrc/kda_wy.hip).  fused: the WY group of
    kda_bwd_fused_kernel (csrc/kda_bwd_fused.hip, bf16): v_new comes from the dq/dk/dg group's
    plane, the epilogue reads k as 4 channels of one token, and the WY parts of dk / dg stay
    in LDS (its other accesses are those of gla_dqkg_kernel<bf16, fp32 v> without dk_add /
    dg_add)."""
    H, K, V = p["H"], p["K"], p["V"]
    KP, VP = _kp(K), _kp(V)
    NPS, VC, NVB = KP // 32, VP // 32, VP // 16
    NVW = (NVB + 3) // 4
    rowK, rowV = H * K, H * V
    tid, lane, wave = _tid(256)
    l16, lg = lane & 15, lane >> 4
    kb, tp = wave & 1, wave >> 1
    ch, sg = tid & 31, tid >> 5
    hh = np.arange(H, dtype=np.int64)[:, None]
    for gc, n, c, row0, L in _chunks(p):
        nval = min(C, L - c * C)
        e0 = (row0 + c * C) * H + hh
        blk = (gc * H + hh)
        ck.acc(p["beta"], e0 * 4, np.where((tid < C) & (tid < nval), tid * H * 4, KOOB), 0, 4, "wy load beta")
        for u in range(NVW):
            vb = wave + 4 * u
            v = 16 * vb + l16
            for kc in range(2):
                o = np.where((vb < NVB) & (v < V), (v * C + 32 * kc + 8 * lg) * 4, KOOB)
                ck.acc(p["dvnt"], blk * V * C * 4, o, 0, 32, "wy load dv_new^T")
            for I in range(4):
                i = 16 * I + l16
                col = 16 * vb + 4 * lg
                o = np.where((vb < NVB) & (i < nval) & (col < V), (i * rowV + col) * es, KOOB)
                ck.acc(p["v"], e0 * V * es, o, 0, 4 * es, "wy load v")
                ck.acc(p["dv"], e0 * V * es, o, 0, 4 * es, "wy store dv")
        for I in range(4):
            for kc in range(2):
                if kc == 1 or I < 2:
                    ck.acc(p["tt"], blk * C * C * 4, ((16 * I + l16) * C + 32 * kc + 8 * lg) * 4, 0, 32,
                           "wy load T^T")
        for a in range(2 if not fused else 0):
            j = 16 * (2 * tp + a) + l16
            for vc in range(VC):
                v0 = 32 * vc + 8 * lg
                ck.acc(p["vnew"], e0 * V * 4, np.where((j < nval) & (v0 < V), (j * rowV + v0) * 4, KOOB),
                       0, 32, "wy load v_new")
        for ps in range(NPS):
            cb = ps * 32
            kk = cb + 16 * kb + l16
            for vc in range(VC):
                v0 = 32 * vc + 8 * lg
                ck.acc(p["hs"], blk * K * V * 4, np.where((kk < K) & (v0 < V), (kk * V + v0) * 4, KOOB),
                       0, 32, "wy load state")
            kc = cb + ch
            for i in range(8 if not fused else 0):   # fused: the gated k plane comes from LDS
                r = 8 * sg + i
                ok = (kc < K) & (r < nval)
                off = r * rowK + kc
                if es == 4:
                    ck.acc(p["k"], e0 * K * 4, np.where(ok, off * 4, KOOB), 0, 4, "wy load k")
                else:
                    ck.acc(p["k"], e0 * K * 2, np.where(ok, (off & ~1) * 2, KOOB), 0, 4, "wy load k")
                ck.acc(p["g"], e0 * K * 4, np.where(ok, off * 4, KOOB), 0, 4, "wy load g")
            if fused:
                for a in range(2):
                    tok = 16 * (2 * tp + a) + l16
                    kq = cb + 16 * kb + 4 * lg
                    ok = (kq < K) & (tok < nval)
                    ck.acc(p["k"], e0 * K * 2, np.where(ok, (tok * rowK + kq) * 2, KOOB), 0, 8,
                           "fused wy load k (epilogue)")
                continue
            for a in range(2):
                t = 2 * tp + a
                for r in range(4):
                    tok = 16 * t + 4 * lg + r
                    ok = (kk < K) & (tok < nval)
                    off = tok * rowK + kk
                    if es == 4:
                        ck.acc(p["k"], e0 * K * 4, np.where(ok, off * 4, KOOB), 0, 4, "wy load k (epilogue)")
                    else:
                        ck.acc(p["k"], e0 * K * 2, np.where(ok, (off & ~1) * 2, KOOB), 0, 4, "wy load k (epilogue)")
                    for nm in ("dk_wy", "dg_wy"):
                        ck.acc(p[nm], e0 * K * 4, np.where(ok, off * 4, KOOB), 0, 4, f"wy store {nm}")
        ck.acc(p["dbeta"], e0 * 4, np.where(tid < nval, tid * H * 4, KOOB), 0, 4, "wy store dbeta")


# --------------------------------------------------------------------------- fr_decode_kernel
def fr_decode(ck: Checker, p: dict, es: int):
    """fr_decode_kernel<TIn, KP> (csrc/gla_recurrent.hip): a 256-thread workgroup per (sequence,
    head, group tg of four 32-column tiles); wave w holds tile 4 tg + w (a wave past the last
    tile only stages), and its lane (kr, cq) = (lane % 8, lane / 8) owns rows RL kr .. + RL - 1
    (RL = KP / 8) and columns 32 tile + 4 cq .. + 3 of the state.  Tokens are staged 8 at a
    time for the whole workgroup: element e = tid + 256 u of the [8][KP] q / k / gk block and of
    the [8][128] v / gv block (columns 128 tg + c).
    p: B, T, H, K, V, cu (host list or None), reverse, and which of gk / gv / s0 / s_fin / o32
    are bound.  Plain pointer accesses (no buffer resource)."""
    B, T, H, K, V = (p[x] for x in ("B", "T", "H", "K", "V"))
    cu = p.get("cu")
    N = len(cu) - 1 if cu is not None else B
    KP = _kp(K)
    RL, DT, WV = KP // 8, 8, 4
    tid, lane, wave = _tid(256)
    kr, cq = lane & 7, lane >> 3
    r0 = RL * kr
    NT = (V + 31) // 32
    NG = (NT + WV - 1) // WV
    for n in range(N):
        bos, L = (cu[n], cu[n + 1] - cu[n]) if cu is not None else (n * T, T)
        tok = (lambda j: bos + L - 1 - j) if p.get("reverse") else (lambda j: bos + j)
        for hh in range(H):
            sbase = (n * H + hh) * K * V
            for tg in range(NG):
                tile = WV * tg + wave
                live = tile < NT
                c0 = 32 * tile + 4 * cq
                vec = (V % 4 == 0) & (c0 + 3 < V)
                for i in range(RL):
                    rok = r0 + 4 * (i // 4) < K
                    o = sbase + (r0 + i) * V + c0
                    if p.get("s0"):
                        ck.acc(p["s0"], 0, np.where(rok & vec & live, o * 4, KOOB), 0, 16,
                               "decode s0 (vector)")
                        for c in range(4):
                            ok = rok & ~(vec & live) & live & (c0 + c < V)
                            ck.acc(p["s0"], 0, np.where(ok, (o + c) * 4, KOOB), 0, 4, "decode s0")
                    if p.get("s_fin"):
                        ck.acc(p["s_fin"], 0, np.where(rok & vec & live, o * 4, KOOB), 0, 16,
                               "decode s_fin (vector)")
                        for c in range(4):
                            ok = rok & ~vec & live & (c0 + c < V)
                            ck.acc(p["s_fin"], 0, np.where(ok, (o + c) * 4, KOOB), 0, 4,
                                   "decode s_fin")
                for b0 in range(0, L, DT):
                    nb = min(DT, L - b0)
                    for u in range(DT * KP // 256):
                        e = tid + 256 * u
                        j, r = e // KP, e % KP
                        ok = (j < nb) & (r < K)
                        t = np.array([tok(b0 + x) for x in np.minimum(j, nb - 1)])
                        o = (t * H + hh) * K + r
                        ck.acc("q", 0, np.where(ok, o * es, KOOB), 0, es, "decode stage q")
                        ck.acc("k", 0, np.where(ok, o * es, KOOB), 0, es, "decode stage k")
                        if p.get("gk"):
                            ck.acc("gk", 0, np.where(ok, o * 4, KOOB), 0, 4, "decode stage gk")
                    for u in range(DT * 32 * WV // 256):
                        e = tid + 256 * u
                        j, c = e // (32 * WV), e % (32 * WV)
                        col = 32 * WV * tg + c
                        ok = (j < nb) & (col < V)
                        t = np.array([tok(b0 + x) for x in np.minimum(j, nb - 1)])
                        o = (t * H + hh) * V + col
                        ck.acc("v", 0, np.where(ok, o * es, KOOB), 0, es, "decode stage v")
                        if p.get("gv"):
                            ck.acc("gv", 0, np.where(ok, o * 4, KOOB), 0, 4, "decode stage gv")
                    if p.get("beta"):         # the KDA instance: threads < nb read beta [B,T,H]
                        bt = np.array([tok(b0 + min(x, nb - 1)) for x in range(256)])
                        ck.acc("beta", 0, np.where(tid < nb, (bt * H + hh) * 4, KOOB), 0, 4,
                               "decode stage beta")
                    for j in range(nb):
                        ov = (tok(b0 + j) * H + hh) * V + c0
                        for c in range(4):
                            st = live & (c0 + c < V) & (kr == 0)
                            ck.acc("o", 0, np.where(st, (ov + c) * es, KOOB), 0, es, "decode store o")
                            if p.get("o32"):
                                ck.acc("o32", 0, np.where(st, (ov + c) * 4, KOOB), 0, 4, "decode store o32")
