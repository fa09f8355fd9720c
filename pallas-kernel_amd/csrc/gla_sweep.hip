// GLA chunk sweeps for gfx950: the fused forward, and the reverse state-gradient sweep
// of the backward.  One kernel template serves both directions.
//
// Forward (REV = false) replaces the reference's K1 chunk_local_cumsum_vector
// (tops/ops/gla/chunk.py:55-198), K7 chunk_fwd_h (tops/ops/common/chunk_h.py:22-272),
// K2 chunk_gla_fwd_intra_gk (tops/ops/gla/chunk.py:351-438) and K3 chunk_gla_fwd_o_gk
// (chunk.py:1279-1440).  Reverse (REV = true) replaces K8 chunk_bwd_dh
// (tops/ops/common/chunk_h.py:685-878) plus the dv part of K4 (chunk.py:1447-1509),
// following the oracle tops/cpu/ops/gla/chunk.py:310-354, 387-427.
//
// One workgroup (8 wave64, two per SIMD) owns one (sequence, head, 64-wide V tile) and
// walks the sequence chunk by chunk (C = 64), forwards or backwards.  A K x 64 fp32 state S
// lives in MFMA accumulators for the whole walk (4 tiles per wave at K = 128).  Per chunk,
// with G the in-chunk inclusive gate cumsum (log2 units), Gamma = G[last], Gm = Gamma / 2,
// q~ = q 2^(G-Gm), k~ = k 2^(Gm-G):
//
//   forward:  S = h (state before the chunk), Y = v
//     o^T   = (scale 2^Gm S)^T q~^T + v^T M^T,   M[i][j] = scale q~_i.k~_j  (j <= i)
//     S     = 2^Gamma S + 2^(Gamma-Gm) (k~^T v)
//   reverse:  S = dh (gradient w.r.t. the state after the chunk), Y = dO
//     dv^T  = (2^(Gamma-Gm) S)^T k~^T + dO^T M,  (M as above, contracted over i >= j)
//     S     = 2^Gamma S + scale 2^Gm (q~^T dO)
//
// i.e. out^T = (alpha S)^T X~^T + Y^T D with (X~, Z~) = (q~, k~) forward and (k~, q~)
// reverse, D[p][r] = scale Z~_p.X~_r on the causal side, and S = 2^Gamma S + beta Z~^T Y.
// The midpoint Gm bounds every exponent by |Gamma|/2, the stabilisation of
// tops/ops/gla/chunk.py:371-375.  Wave w computes the output tiles of token block w / 2 and
// column tiles 2 (w % 2), 2 (w % 2) + 1 (the two waves of a token block both compute its
// intra-chunk D tiles: MFMA has the headroom, a split would cost a barrier).
//
// DELTA (the KDA delta rule): forward, Y = v_new = u - w S is computed per chunk before the
// output and the state update (w 2^-Gm is read from HBM as the MFMA A operand against
// H^T = 2^Gm S); reverse, the state update gains - w^T dv_new, and dv_new is written
// transposed per chunk for the WY backward.
//
// YG (bf16): the gate is applied on the value side.  YG = 1 (forward): one log-gate per
// (token, V column) (fused_recurrent_gla's gv), S[:, v] <- 2^gv S[:, v] + k v^T.  YG = 2
// (forward and reverse): one log-gate per token (simple GLA's g [B,T,H], or g_gamma [H]),
// which factors out of every q.k product: D[i][j] = 2^(G_i - G_j) (q_i.k_j).  Either way q and
// k enter ungated (exact bf16: the X / Z planes carry no lo half), Y~ = Y 2^(s(Gm - G)) is
// split into hi / lo (s = 1 forward, -1 reverse), every output element is multiplied by
// 2^(s(G - Gm)) of its (token, column) from an fp32 LDS plane, and S decays per column:
//   forward:  o^T = (scale 2^Gm S)^T q^T + v~^T M,  S = 2^Gamma S + 2^(Gamma-Gm) (k^T v~)
//   reverse:  dv^T = (2^(Gamma-Gm) S)^T k^T + dO~^T M,  S = 2^Gamma S + scale 2^Gm (q^T dO~)
// with M[i][j] = scale q_i.k_j on the causal side.
//
// Every workgroup also writes S at the start of each chunk to `ckpt` when given (the
// forward's state checkpoints, or the reverse sweep's dh per chunk), or, in the
// interleaved layout, at the start of every even (forward) or odd (reverse) global chunk.
//
// Pipelining: the raw q/k/g/Y of chunk c+1 are loaded into registers while chunk c is
// computed; a full chunk takes a branch-free path (masked rows read out of range and are
// zeroed by the buffer range check).  Two barriers per chunk (three or four with DELTA).
#include <type_traits>

#include "gla_sweep.h"
#include "tops_common.h"
#include "tops_hip.h"

namespace tops {

// GK: the per-channel gate mode only (kGateK, the GLA and KDA path), compiled on its own so
// that the hot path carries no gate-mode branches; !GK serves the per-token and constant
// gates (kGateS, kGateGamma, kGateGammaK) chosen at run time.
// VAR selects the features an instance compiles (as in gla_sweep_pipe.hip): 1 = fp16
// checkpoints of every chunk, whole-width rows, no slices; 2 = no checkpoints and no slices;
// 0 = the rest (fp32 or paired checkpoints, channel slices; no fp16 checkpoints).
template <typename TIn, int KP, bool REV, bool DELTA, bool ST, bool GK, int YG = 0, int VAR = 0>
__global__ __launch_bounds__(512) void gla_sweep_kernel(SweepParams p) {
  constexpr int NW = 8;                  // wave64s per workgroup
  constexpr int NTH = 64 * NW;
  constexpr int C = kChunk, BV = 64;
  constexpr int NQ = KP / 4;             // column quads of a [C][KP] tile
  constexpr int NSEG = NTH / NQ;         // row segments
  constexpr int RPT = C / NSEG;          // rows per thread (4, 2, 1)
  // staging thread mapping: a 32-lane half-wave covers CQL column quads x SGL row segments,
  // which keeps the row-major and the transposed plane writes (nearly) free of bank conflicts
  constexpr int CQL = 8, SGL = 32 / CQL;  // 8 column quads x 4 row segments per half-wave
  constexpr int NCQH = NQ / CQL;         // half-waves across the columns
  constexpr int NSGH = NSEG / SGL;       // segment groups (half-waves down the rows)
  static_assert(NQ % CQL == 0, "KP must be a multiple of 32");
  static_assert(CQL == 8 && SGL == 4, "the segment scan takes 8 column quads x 4 segments");
  constexpr bool SIN = !In<TIn>::kExactBf16;
  constexpr bool FWD_DELTA = DELTA && !REV;
  constexpr bool REV_DELTA = DELTA && REV;
  constexpr bool GV = YG != 0;           // value-side gate (either form)
  constexpr bool SY = SIN || FWD_DELTA || GV;  // the Y plane carries a lo half (fp32 Y, v_new, Y~)
  constexpr bool XL = !GV;               // the X / Z planes carry a lo half (gated q / k)
  static_assert(!GV || (!DELTA && !ST && !GK && !SIN), "YG: the bf16 full sweeps only");
  constexpr int LQ = KP + 8, LT = C + 8, LH = KP + 8;
  constexpr int NHT = (KP / 16) * (BV / 16) / NW;  // state tiles per wave (4, 2, 1), one K block
  constexpr int ES = sizeof(TIn);
  constexpr int YR = C * BV / (2 * NTH);           // Y rows per thread (2 columns each)
  static_assert(RPT == 1 || RPT == 2 || RPT == 4, "KP must be 32, 64 or 128");
  static_assert(YR == 4, "Y staging assumes 4 rows x 2 columns per thread");
  typedef Words<TIn> Wd;

  __shared__ __attribute__((aligned(16))) uint16_t sX[(XL ? 2 : 1) * C * LQ];
  __shared__ __attribute__((aligned(16))) uint16_t sZ[(XL ? 2 : 1) * C * LQ];
  // the reverse delta rule's w^T plane [K][C]; the forward delta rule's causal D tiles
  // (10 tiles x 64 lanes x 16 B, written after the output pass while the Z~ plane is still
  // read by the state update).  The other sweeps read Z~ transposed out of its row-major
  // plane and need neither.
  __shared__ __attribute__((aligned(16))) uint16_t sZT[REV_DELTA ? 2 * KP * LT : (FWD_DELTA ? 10 * 64 * 8 : 1)];
  __shared__ __attribute__((aligned(16))) uint16_t sYT[(SY ? 2 : 1) * BV * LT];
  // (the reverse delta rule reuses sHT for the [BV][LT] dv_new^T plane: size for both)
  constexpr int NHTS = 2 * BV * (REV_DELTA && LT > LH ? LT : LH);
  __shared__ __attribute__((aligned(16))) uint16_t sHT[NHTS];
  __shared__ __attribute__((aligned(16))) float sTot[NSGH * KP]; // gate totals per segment group
  // GV: the output factors 2^(G - Gm) [C][BV + 4] and the gate totals of the 16-row groups
  constexpr int LE = BV + 4;
  __shared__ __attribute__((aligned(16))) float sE[GV ? C * LE : 1];
  __shared__ __attribute__((aligned(16))) float sGvTot[GV ? 4 * BV : 1];
  // Causal D tiles of the chunk shared through LDS (bf16 hi/lo per lane, 10 tiles x 1 KB):
  // each tile is computed once instead of once per column-tile wave, and the work is spread
  // evenly over the waves.  Only where the 160 KB budget allows (not the delta sweeps).
  constexpr int LDS_BASE = 2 * ((XL ? 2 : 1) * C * LQ) * 2 +
                           (REV_DELTA ? 2 * KP * LT * 2 : (FWD_DELTA ? 10 * 64 * 16 : 0)) +
                           (SY ? 2 : 1) * BV * LT * 2 + NHTS * 2 + NSGH * KP * 4 +
                           (GV ? (C * LE + 4 * BV) * 4 : 0);
  constexpr bool SHARED_D = !DELTA && !ST && LDS_BASE + 10 * 64 * 16 <= 160 * 1024;
  __shared__ __attribute__((aligned(16))) uint4 sDt[SHARED_D ? 10 * 64 : 1];
  __shared__ uint32_t sMx[NW];   // fp16 checkpoints: each wave's largest |S| (fp32 bits)
  // (forward delta rule) 2^-Gm of channel c, Gm = Gamma / 2, sits in the padding columns of the
  // X hi plane (row c / 4, word c % 4): no MFMA fragment or staging write touches columns >= KP
  auto egm_at = [&](int c4) { return (float*)(sX + (c4 >> 2) * LQ + KP); };

  const Plane PX{sX, XL ? sX + C * LQ : sX, LQ};
  const Plane PZ{sZ, XL ? sZ + C * LQ : sZ, LQ};
  const Plane PYt{sYT, SY ? sYT + BV * LT : sYT, LT};
  const Plane PHt{sHT, sHT + BV * LH, LH};
  // reverse delta rule: once the output pass is done, w^T [K][C] goes to sZT and
  // dv_new^T [BV][C] reuses sHT
  const Plane PWt{sZT, sZT + KP * LT, LT};
  const Plane PDt{sHT, sHT + BV * LT, LT};

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int l16 = lane & 15, lg = lane >> 4;
  const int R = wave >> 1;               // token block of this wave's output tiles
  const int nh = wave & 1;               // output column tiles nn = 2 nh, 2 nh + 1
  const int msb = (wave * NHT) / (BV / 16);   // K block of this wave's state tiles
  const int wg = xcd_remap(blockIdx.x, gridDim.x, p.NV);
  const int vt = wg % p.NV;
  const int hh = (wg / p.NV) % p.H;
  int n = wg / (p.NV * p.H);
  // sequence j covers rows [cu_seqlens[j], end of j): the next start, or seg_end[j] when the
  // sequences are a list of disjoint segments
  auto seq_end = [&](int j) { return p.seg_end ? p.seg_end[j] : p.cu_seqlens[j + 1]; };
  if (p.cu_seqlens && p.N > 1 && p.N <= 256) {
    // Varlen: dispatch sequences longest first (LPT), so the workgroups that share a CU
    // balance; slot r takes the sequence of rank r in descending length (ties by index).
    const int slot = n;
    if (tid < p.N) {
      const int li = seq_end(tid) - p.cu_seqlens[tid];
      int rank = 0;
      for (int j = 0; j < p.N; ++j) {
        const int lj = seq_end(j) - p.cu_seqlens[j];
        rank += (lj > li) || (lj == li && j < tid);
      }
      if (rank == slot) *(int*)sTot = tid;
    }
    __syncthreads();
    n = *(const int*)sTot;
    __syncthreads();  // sTot is reused by the chunk loop
  }
  n = __builtin_amdgcn_readfirstlane(n);
  const int H = p.H, K = p.K, V = p.V;
  // row length of q / k / g and of the state rows
  const int LDK = (VAR == 0 && p.ldk > 0) ? p.ldk : K;
  const float scale = p.scale;

  int L, row0, cbase;
  if (p.cu_seqlens) {
    row0 = p.cu_seqlens[n];
    L = seq_end(n) - row0;
    cbase = p.chunk_offsets ? p.chunk_offsets[n] : 0;
  } else {
    row0 = n * p.T;
    L = p.T;
    cbase = n * cdiv(p.T, C);
  }
  const int NTs = cdiv(L, C);                          // 0 for an empty sequence

  // ---- staging coordinates and per-thread byte offsets within a chunk
  const int hw = tid >> 5;               // half-wave
  const int sgl = (lane & 31) / CQL;     // row segment within the half-wave
  const int sgh = hw / NCQH;             // segment group
  const int cq = (lane & 31) % CQL + CQL * (hw % NCQH), seg = sgl + SGL * sgh;
  const int c0 = 4 * cq, r0 = seg * RPT;
  const bool colok = c0 < K;
  // Y: 2 columns x 4 rows per thread; a half-wave covers 8 column pairs x 4 row groups
  const int yc = (lane & 7) + 8 * (hw & 3), yseg = ((lane >> 3) & 3) + 4 * (hw >> 2);
  const int yv = vt * BV + 2 * yc;
  const bool ycolok = yv < V;
  const uint32_t rowK = (uint32_t)(H * LDK), rowV = (uint32_t)(H * V);
  const uint32_t offQ = colok ? ((uint32_t)r0 * rowK + c0) * ES : kOOB;        // q, k
  const uint32_t offG = colok ? ((uint32_t)r0 * rowK + c0) * 4u : kOOB;        // g, w
  const uint32_t offY = ycolok ? ((uint32_t)(yseg * YR) * rowV + yv) * ES : kOOB;
  const uint32_t offYg = ycolok ? ((uint32_t)(yseg * YR) * rowV + yv) * 4u : kOOB;   // GV gates
  // gate load: per-channel [.., K] float4, or the per-(token, head) scalar read as the first
  // word of a 16-byte load; the gamma mode loads nothing (out of range -> 0)
  const int gmode = GK ? kGateK : (GV ? kGateGamma : p.gate_mode);   // YG: no K-side gate
  // YG = 2: the value-side gate is per token, g [B,T,H] (kGateS) or the constant g_gamma [H]
  const bool yg_s = YG == 2 && p.gate_mode == kGateS;
  const float yg_gam = (YG == 2 && p.gate_mode == kGateGamma) ? p.g[hh] : 0.f;
  const bool gk_mode = GK || gmode == kGateK;
  const uint32_t offGm = gk_mode ? offG : (gmode == kGateS ? (uint32_t)r0 * H * 4u : kOOB);
  const uint32_t gstride = gk_mode ? rowK * 4 : (uint32_t)H * 4;
  const float gam_h = gmode == kGateGamma && !GV ? p.g[hh] : 0.f;
  // constant per-(head, channel) gate: the four channels c0..c0+3 of this thread
  float gam4[4] = {gam_h, gam_h, gam_h, gam_h};
  if (gmode == kGateGammaK) {
#pragma unroll
    for (int j = 0; j < 4; ++j) gam4[j] = colok ? p.g[(size_t)hh * LDK + c0 + j] : 0.f;
  }

  // ---- state tiles: tile i of this wave -> (msb, nn)
  f32x4 S[NHT];
  // s0 / s_fin rows of this (sequence, head) through one buffer resource each: lane (l16, lg)
  // of tile i holds rows 16 msb + 4 lg + r (K % 4 == 0: all four inside or none), column
  // 16 nn + l16; no s0: an empty range loads zeros
  const size_t s_base = (size_t)(n * H + hh) * LDK * V;
  auto sel_off = [&](int i) {
    const int kr = 16 * msb + 4 * lg;
    const int vv = vt * BV + 16 * ((wave * NHT + i) % (BV / 16)) + l16;
    return (kr < K && vv < V) ? ((uint32_t)kr * V + vv) * 4u : kOOB;
  };
  {
    const rsrc_t Rs0 = make_rsrc(p.s0 ? p.s0 + s_base : nullptr, p.s0 ? (long long)LDK * V * 4 : 0);
#pragma unroll
    for (int i = 0; i < NHT; ++i) {
      const uint32_t o = sel_off(i);
#pragma unroll
      for (int r = 0; r < 4; ++r) S[i][r] = __uint_as_float(bld32(Rs0, o, (uint32_t)(r * V * 4)));
    }
  }
  // reverse-time recurrence (gshift): the state entering the last token is h0 decayed by
  // that token's gate
  constexpr bool RSH = REV && !ST && !DELTA;
  const bool gsh = RSH && p.gshift;
  if (gsh && L > 0) {
    const size_t el = (size_t)(row0 + L - 1) * H + hh;
    float fac[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int kr = 16 * msb + 4 * lg + r;
      float gl = gam_h;
      if (gk_mode) gl = kr < K ? p.g[el * LDK + kr] : 0.f;
      else if (gmode == kGateS) gl = p.g[el];
      else if (gmode == kGateGammaK) gl = kr < K ? p.g[(size_t)hh * LDK + kr] : 0.f;
      fac[r] = fast_exp2(gl * kLog2e);
    }
#pragma unroll
    for (int i = 0; i < NHT; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) S[i][r] *= fac[r];
    }
  }
  // Drain these loads here: a load still in flight when the chunk loop starts makes the
  // compiler's wait before the first use of S inside the loop a full vmcnt(0) on every
  // iteration, which also waits for the previous chunk's output and checkpoint stores.
  __builtin_amdgcn_s_waitcnt(0);

  // ---- raw chunk registers (prefetch targets): PF sets, the chunk PF steps ahead is
  // loaded into the set just consumed.  One set is issued a whole chunk ahead (after B2),
  // which covers the load latency; the second set pays off only for the instances whose
  // output block keeps fewer registers live (bf16 without shared D tiles).
  constexpr int PF = (DELTA || SIN || SHARED_D) ? 1 : 2;
  struct Raw {
    typename Wd::W4 rq[RPT], rk[RPT];
    uint4 rg[RPT];
    typename Wd::W2 ry[YR];
    uint2 rgv[GV ? YR : 1];              // YG: the gates of the two Y columns
  };
  Raw rsA, rsB;
  auto load_chunk = [&](int c, Raw& rs) {
    const int t0 = c * C;
    const int nval = min(C, L - t0);
    const size_t e0 = (size_t)(row0 + t0) * H + hh;     // first row of the chunk, this head
    // chunk-bounded resources (chunk_rsrc): rows past the chunk's nval tokens load zeros
    const rsrc_t Rq = chunk_rsrc((const TIn*)p.q, e0, nval, (int)rowK, LDK);
    const rsrc_t Rk = chunk_rsrc((const TIn*)p.k, e0, nval, (int)rowK, LDK);
    // gshift: token t reads the gate row of token t - 1, so the rows start one token earlier,
    // except in the sequence's first chunk, whose row 0 reads nothing (gate 0)
    const int gadj = (gsh && t0 == 0) ? 1 : 0;
    const size_t eg = gsh && t0 > 0 ? e0 - (size_t)H : e0;
    const rsrc_t Rg = gk_mode ? chunk_rsrc(p.g, eg, nval, (int)rowK, LDK)
                              : chunk_rsrc(p.g, eg, nval, H, 1);
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      rs.rq[i] = Wd::ld4(Rq, offQ, i * rowK * ES);
      rs.rk[i] = Wd::ld4(Rk, offQ, i * rowK * ES);
      // the gate mode's transform is applied when the chunk is consumed, so the prefetch
      // never waits: four channels [.., K], or the one per-(token, head) word [.., 1]
      // (gamma: offGm is out of range, nothing is read)
      uint32_t go = !GV ? offGm : kOOB, gs = i * gstride;
      if constexpr (RSH) {
        // row r0 + i - gadj (>= 0 where read), as one vector offset; masked columns and the
        // constant gates (offGm out of range) read nothing.  The token mask stays: shifted by
        // one row, the gate row of the first token past nval is still inside Rg's range
        const bool rd = r0 + i < nval && r0 + i >= gadj && offGm != kOOB;
        go = rd ? offGm + (uint32_t)(i - gadj) * gstride : kOOB;
        gs = 0;
      }
      if constexpr (GV) rs.rg[i] = make_uint4(0u, 0u, 0u, 0u);
      else if constexpr (GK) rs.rg[i] = bld128(Rg, go, gs);
      else if (gk_mode) rs.rg[i] = bld128(Rg, go, gs);
      else rs.rg[i] = make_uint4(bld32(Rg, go, gs), 0u, 0u, 0u);
    }
    if constexpr (!FWD_DELTA) {
      const rsrc_t Ry = chunk_rsrc((const TIn*)p.y, e0, nval, (int)rowV, V);
#pragma unroll
      for (int i = 0; i < YR; ++i) rs.ry[i] = Wd::ld2(Ry, offY, i * rowV * ES);
      if constexpr (YG == 1) {
        const rsrc_t Rgv = chunk_rsrc(p.g, e0, nval, (int)rowV, V);
#pragma unroll
        for (int i = 0; i < YR; ++i) rs.rgv[i] = bld64(Rgv, offYg, i * rowV * 4);
      } else if constexpr (YG == 2) {
        // one word per row (the constant gate reads nothing: out of range)
        const rsrc_t Rgs = chunk_rsrc(p.g, e0, nval, H, 1);
#pragma unroll
        for (int i = 0; i < YR; ++i) {
          const bool ok = yg_s;
          const uint32_t w = bld32(Rgs, ok ? (uint32_t)(yseg * YR) * H * 4u : kOOB, i * H * 4);
          rs.rgv[i] = make_uint2(w, w);
        }
      }
    }
  };

  auto cidx = [&](int it) { return REV ? NTs - 1 - it : it; };
  float dsum[4] = {0.f, 0.f, 0.f, 0.f};   // state-only pass: sum of Gamma of this lane's rows
  // (an empty sequence has no chunk: nothing is loaded, and the state passes through)
  if (NTs > 0) load_chunk(cidx(0), rsA);
  if constexpr (PF == 2) {
    if (NTs > 1) load_chunk(cidx(1), rsB);
  }

  auto body = [&](int it, Raw& rs) {
    const int c = cidx(it);
    const int t0 = c * C;
    const int nval = min(C, L - t0);

    // ---------------- forward delta rule: w rows of this wave's token block (MFMA row layout)
    // and u in the result layout, issued now so their latency overlaps the staging
    // (bf16 only: the fp32 instantiation has no register room and loads them after B2)
    constexpr bool HOIST = FWD_DELTA && !SIN;
    uint4 wraw[KP / 32][2];
    float ur[2][4];
    auto load_wu = [&]() {
      const size_t e0 = (size_t)(row0 + t0) * H + hh;
      const rsrc_t Rw = chunk_rsrc(p.w, e0, nval, (int)rowK, LDK);
      const rsrc_t Ru = chunk_rsrc(p.u, e0, nval, (int)rowV, V);
      const int trow = 16 * R + l16;
#pragma unroll
      for (int kc = 0; kc < KP / 32; ++kc) {
        const int k0 = 32 * kc + 8 * lg;
        const uint32_t o = k0 < K ? ((uint32_t)trow * rowK + k0) * 4u : kOOB;
        wraw[kc][0] = bld128(Rw, o, 0);
        wraw[kc][1] = bld128(Rw, o == kOOB ? kOOB : o + 16u, 0);
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int vv = vt * BV + 16 * (2 * nh + j) + l16;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int tok = 16 * R + 4 * lg + r;
          ur[j][r] = __uint_as_float(bld32(Ru, vv < V ? ((uint32_t)tok * rowV + vv) * 4u : kOOB, 0));
        }
      }
    };
    if constexpr (HOIST) load_wu();

    // ---------------- reverse delta rule: w rows of this thread, consumed after barrier B3
    float4 rw[RPT];
    if constexpr (REV_DELTA) {
      const size_t e0 = (size_t)(row0 + t0) * H + hh;
      const rsrc_t Rw = chunk_rsrc(p.w, e0, nval, (int)rowK, LDK);
#pragma unroll
      for (int i = 0; i < RPT; ++i) {
        const uint4 x = bld128(Rw, offG, i * rowK * 4);
        rw[i] = make_float4(__uint_as_float(x.x), __uint_as_float(x.y), __uint_as_float(x.z),
                            __uint_as_float(x.w));
      }
    }

    // ---------------- gate cumsum: thread rows, a DPP scan over the half-wave's row
    // segments, then segment-group totals through LDS
    float G[RPT][4];
    float pre[4], gam[4];
    // GV: the value-side gate cumsum of this thread's two Y columns (rows yseg*YR..+3), the
    // prefix of the earlier row groups of its half-wave, and (after B1) of the earlier groups
    float gvc[YR][2], prev[2] = {0.f, 0.f};
    if constexpr (GV) {
#pragma unroll
      for (int i = 0; i < RPT; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) G[i][j] = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) pre[j] = gam[j] = 0.f;
#pragma unroll
      for (int i = 0; i < YR; ++i) {
        float a = __uint_as_float(rs.rgv[i].x), b = __uint_as_float(rs.rgv[i].y);
        if (YG == 2 && !yg_s) a = b = yseg * YR + i < nval ? yg_gam : 0.f;
        gvc[i][0] = a * kLog2e + (i > 0 ? gvc[i - 1][0] : 0.f);
        gvc[i][1] = b * kLog2e + (i > 0 ? gvc[i - 1][1] : 0.f);
      }
#pragma unroll
      for (int c2 = 0; c2 < 2; ++c2) {
        const float t = gvc[YR - 1][c2];
        const float x = seg8x4_scan(t, lane);   // over the row segments (lane >> 3) & 3
        prev[c2] = x - t;
        if (((lane >> 3) & 3) == 3) sGvTot[(hw >> 2) * BV + 2 * yc + c2] = x;
      }
    } else {
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      float x[4];
      unpack4(rs.rg[i], x);
      if constexpr (GK) {
      } else if (gmode == kGateS) {
        x[1] = x[2] = x[3] = x[0];
      } else if (!gk_mode) {   // constant gates: zero on the rows past the sequence (and, with
                               // gshift, on the sequence's first token)
        const bool on = r0 + i < nval && !(gsh && t0 == 0 && r0 + i == 0);
#pragma unroll
        for (int j = 0; j < 4; ++j) x[j] = on ? gam4[j] : 0.f;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) G[i][j] = x[j] * kLog2e + (i > 0 ? G[i - 1][j] : 0.f);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float t = G[RPT - 1][j];
      const float x = seg8x4_scan(t, lane);   // over the row segments sgl of the half-wave
      pre[j] = x - t;                    // segments before this one, within the half-wave
      gam[j] = x;                        // inclusive; the last segment holds the group total
    }
    if (sgl == SGL - 1) *(float4*)(sTot + sgh * KP + c0) = make_float4(gam[0], gam[1], gam[2], gam[3]);
    }  // !GV
    __syncthreads();  // B1: totals visible; every wave is done with the previous chunk's planes

    if constexpr (!GV) {
#pragma unroll
    for (int j = 0; j < 4; ++j) gam[j] = 0.f;
#pragma unroll
    for (int s2 = 0; s2 < NSGH; ++s2) {
      const float4 t = *(const float4*)(sTot + s2 * KP + c0);
      if (s2 < sgh) { pre[0] += t.x; pre[1] += t.y; pre[2] += t.z; pre[3] += t.w; }
      gam[0] += t.x; gam[1] += t.y; gam[2] += t.z; gam[3] += t.w;
    }
    }
    // YG: Gm of the thread's Y columns (and the prefix of its rows), and per state tile the
    // factors of the lane's column 16 nn + l16: 2^Gamma (decay), the update scaling and alpha
    // (forward 2^(Gamma - Gm) and scale 2^Gm, reverse scale 2^Gm and 2^(Gamma - Gm))
    float gmv[2] = {0.f, 0.f};
    float cga[NHT], cbe[NHT], cal[NHT];
    if constexpr (GV) {
#pragma unroll
      for (int c2 = 0; c2 < 2; ++c2) {
        float tot = 0.f;
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2) {
          const float t = sGvTot[s2 * BV + 2 * yc + c2];
          if (s2 < (hw >> 2)) prev[c2] += t;
          tot += t;
        }
        gmv[c2] = 0.5f * tot;
      }
#pragma unroll
      for (int i = 0; i < NHT; ++i) {
        const int col = 16 * ((wave * NHT + i) % (BV / 16)) + l16;
        const float tot = sGvTot[col] + sGvTot[BV + col] + sGvTot[2 * BV + col] + sGvTot[3 * BV + col];
        cga[i] = fast_exp2(tot);
        const float hf = fast_exp2(0.5f * tot);
        cbe[i] = REV ? scale * hf : hf;
        cal[i] = REV ? hf : scale * hf;
      }
    }
    float gm[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) gm[j] = 0.5f * gam[j];
    if constexpr (FWD_DELTA) {
      if (seg == 0)
        *(float4*)egm_at(c0) =
            make_float4(fast_exp2(-gm[0]), fast_exp2(-gm[1]), fast_exp2(-gm[2]), fast_exp2(-gm[3]));
    }
    // Gamma of this lane's state rows kr = 16 msb + 4 lg + r
    float sgam[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s2 = 0; s2 < (GV ? 0 : NSGH); ++s2) {
      const float4 t = *(const float4*)(sTot + s2 * KP + 16 * msb + 4 * lg);
      sgam[0] += t.x; sgam[1] += t.y; sgam[2] += t.z; sgam[3] += t.w;
    }
    float sga[4], sal[4], sbe[4];        // 2^Gamma, alpha (H^T scaling), beta (update scaling)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float g2 = 0.5f * sgam[r];
      sga[r] = fast_exp2(sgam[r]);
      sal[r] = REV ? fast_exp2(sgam[r] - g2) : (DELTA ? 1.f : scale) * fast_exp2(g2);
      sbe[r] = REV ? scale * fast_exp2(g2) : fast_exp2(sgam[r] - g2);
    }

    // ---------------- state -> H^T plane (alpha S)
    if constexpr (ST) {
#pragma unroll
      for (int r = 0; r < 4; ++r) dsum[r] += sgam[r];
    } else {
#pragma unroll
      for (int i = 0; i < NHT; ++i) {
        const int nn = (wave * NHT + i) % (BV / 16);
        const int kr = 16 * msb + 4 * lg;
        float x[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) x[r] = (GV ? cal[i] : sal[r]) * S[i][r];
        put_n<true, 4>(PHt, 16 * nn + l16, kr, x);
      }
    }
    // checkpoint of S (the state at the start of the chunk).  Issued here, ahead of the
    // staging: stored after the next chunk's prefetch instead, the checkpoints measured
    // slower (the memory counter retires in issue order, so the waits for the prefetched
    // loads at the top of the next chunk then also cover the stores).
    if constexpr (!ST && VAR == 1) {
      state_absmax<NHT>(S, sMx, wave, lane);   // the tile maximum is read after B2
    } else if constexpr (!ST && VAR == 0) {
      if (p.ckpt && (p.ckpt_par == 0 || ((cbase + c) & 1) == p.ckpt_par - 1)) {
        const rsrc_t Rck = make_rsrc(p.ckpt + ((size_t)(cbase + c) * H + hh) * LDK * V,
                                     (long long)K * V * 4);
#pragma unroll
        for (int i = 0; i < NHT; ++i) {
          const int nn = (wave * NHT + i) % (BV / 16);
          const int kr = 16 * msb + 4 * lg;
          const int vv = vt * BV + 16 * nn + l16;
          const uint32_t vo = (kr < K && vv < V) ? ((uint32_t)kr * V + vv) * 4u : kOOB;  // K % 4 == 0
#pragma unroll
          for (int r = 0; r < 4; ++r)
            bst32(Rck, __float_as_uint(S[i][r]), vo, (uint32_t)(r * V * 4));
        }
      }
    }
    // ---------------- gated operands for the staging rows (Z~ row-major: the state update
    // reads it transposed, ds_read_b64_tr_b16)
    {
      uint32_t zh[RPT][2], zl[RPT][2];
#pragma unroll
      for (int i = 0; i < RPT; ++i) {
        float qv[4], kv[4], xq[4], xk[4];
        unpack4(rs.rq[i], qv);
        unpack4(rs.rk[i], kv);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if constexpr (GV) {
            xq[j] = qv[j];
            xk[j] = kv[j];
          } else {
            const float Gv = G[i][j] + pre[j];
            xq[j] = (FWD_DELTA ? scale : 1.f) * qv[j] * fast_exp2(Gv - gm[j]);
            xk[j] = kv[j] * fast_exp2(gm[j] - Gv);
          }
        }
        const float* xx = REV ? xk : xq;
        const float* zz = REV ? xq : xk;
        if constexpr (!ST) put_n<XL, 4>(PX, r0 + i, c0, xx);
        split_bf16x2(zz[0], zz[1], zh[i][0], zl[i][0]);
        split_bf16x2(zz[2], zz[3], zh[i][1], zl[i][1]);
        *(uint2*)(PZ.hi + (r0 + i) * PZ.ld + c0) = make_uint2(zh[i][0], zh[i][1]);
        if constexpr (XL) *(uint2*)(PZ.lo + (r0 + i) * PZ.ld + c0) = make_uint2(zl[i][0], zl[i][1]);
      }
      if constexpr (!FWD_DELTA) {
        float ya[YR], yb[YR];
#pragma unroll
        for (int i = 0; i < YR; ++i) unpack2(rs.ry[i], ya[i], yb[i]);
        if constexpr (GV) {
          // Y~ = Y 2^(s(Gm - G)) into the Y plane; the output factor 2^(s(G - Gm)) into sE
#pragma unroll
          for (int i = 0; i < YR; ++i) {
            float ga = gvc[i][0] + prev[0] - gmv[0], gb = gvc[i][1] + prev[1] - gmv[1];
            if constexpr (REV) { ga = -ga; gb = -gb; }
            ya[i] *= fast_exp2(-ga);
            yb[i] *= fast_exp2(-gb);
            *(float2*)(sE + (yseg * YR + i) * LE + 2 * yc) = make_float2(fast_exp2(ga), fast_exp2(gb));
          }
        }
        put_n<SY, YR>(PYt, 2 * yc, yseg * YR, ya);
        put_n<SY, YR>(PYt, 2 * yc + 1, yseg * YR, yb);
      }
    }
    __syncthreads();  // B2: all planes visible

    // fp16 checkpoint of S, from the wave maxima taken before B2 (stored ahead of the
    // prefetch below: the memory counter retires in issue order)
    if constexpr (!ST && VAR == 1)
      store_state16<NHT, NW>(S, sMx, (uint16_t*)p.ckpt + ((size_t)(cbase + c) * H + hh) * LDK * V,
                             p.ckpt_scale + ((size_t)(cbase + c) * H + hh) * p.NV + vt, K, V,
                             vt, wave, msb, lane, tid);

    // ---------------- prefetch the chunk PF steps ahead while this one is computed
    if (it + PF < NTs) load_chunk(cidx(it + PF), rs);

    // ---------------- reverse delta rule: first half of the state update (Z~^T Y)
    f32x4 d1[NHT];
    if constexpr (REV_DELTA) {
#pragma unroll
      for (int i = 0; i < NHT; ++i) {
        const int nn = (wave * NHT + i) % (BV / 16);
        d1[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kc = 0; kc < C / 32; ++kc) {
          const bf16x8 bh = PYt.hi8(16 * nn + l16, 32 * kc + 8 * lg);
          bf16x8 bl = bh;
          if constexpr (SY) bl = PYt.lo8(16 * nn + l16, 32 * kc + 8 * lg);
          d1[i] = mma<true, SY>(d1[i], tr_read8(PZ.hi, PZ.ld, 32 * kc, 16 * msb, lane),
                                tr_read8(PZ.lo, PZ.ld, 32 * kc, 16 * msb, lane), bh, bl);
        }
      }
    }

    // ---------------- state update: S = 2^Gamma S + beta (Z~^T Y) [- w^T dv_new]
    auto state_update = [&]() {
      // (shared-D build) every fragment first, then the NHT independent accumulation chains
      // interleaved term by term, so neither LDS latency nor MFMA dependencies serialise
      f32x4 dsu[NHT];
      if constexpr (SHARED_D) {
        bf16x8 zh[C / 32], zl[C / 32], yh[NHT][C / 32], yl[NHT][C / 32];
#pragma unroll
        for (int kc = 0; kc < C / 32; ++kc) {
          zh[kc] = tr_read8(PZ.hi, PZ.ld, 32 * kc, 16 * msb, lane);
          if constexpr (XL) zl[kc] = tr_read8(PZ.lo, PZ.ld, 32 * kc, 16 * msb, lane);
#pragma unroll
          for (int i = 0; i < NHT; ++i) {
            const int nn = (wave * NHT + i) % (BV / 16);
            yh[i][kc] = PYt.hi8(16 * nn + l16, 32 * kc + 8 * lg);
            if constexpr (SY) yl[i][kc] = PYt.lo8(16 * nn + l16, 32 * kc + 8 * lg);
          }
        }
#pragma unroll
        for (int i = 0; i < NHT; ++i) dsu[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kc = 0; kc < C / 32; ++kc) {
          if constexpr (XL) {
#pragma unroll
            for (int i = 0; i < NHT; ++i) dsu[i] = mfma(zl[kc], yh[i][kc], dsu[i]);
          }
          if constexpr (SY) {
#pragma unroll
            for (int i = 0; i < NHT; ++i) dsu[i] = mfma(zh[kc], yl[i][kc], dsu[i]);
          }
#pragma unroll
          for (int i = 0; i < NHT; ++i) dsu[i] = mfma(zh[kc], yh[i][kc], dsu[i]);
        }
      }
#pragma unroll
      for (int i = 0; i < NHT; ++i) {
        const int nn = (wave * NHT + i) % (BV / 16);
        f32x4 d = {0.f, 0.f, 0.f, 0.f};
        if constexpr (REV_DELTA) {
#pragma unroll
          for (int kc = 0; kc < C / 32; ++kc)
            d = mma<true, true>(d, PWt.hi8(16 * msb + l16, 32 * kc + 8 * lg), PWt.lo8(16 * msb + l16, 32 * kc + 8 * lg),
                                PDt.hi8(16 * nn + l16, 32 * kc + 8 * lg), PDt.lo8(16 * nn + l16, 32 * kc + 8 * lg));
        } else if constexpr (!SHARED_D) {
#pragma unroll
          for (int kc = 0; kc < C / 32; ++kc) {
            const bf16x8 bh = PYt.hi8(16 * nn + l16, 32 * kc + 8 * lg);
            bf16x8 bl = bh;
            if constexpr (SY) bl = PYt.lo8(16 * nn + l16, 32 * kc + 8 * lg);
            const bf16x8 zh8 = tr_read8(PZ.hi, PZ.ld, 32 * kc, 16 * msb, lane);
            bf16x8 zl8 = zh8;
            if constexpr (XL) zl8 = tr_read8(PZ.lo, PZ.ld, 32 * kc, 16 * msb, lane);
            d = mma<XL, SY>(d, zh8, zl8, bh, bl);
          }
        } else {
          d = dsu[i];
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if constexpr (REV_DELTA) S[i][r] = sga[r] * S[i][r] + sbe[r] * d1[i][r] - d[r];
          else if constexpr (GV) S[i][r] = cga[i] * S[i][r] + cbe[i] * d[r];
          else S[i][r] = sga[r] * S[i][r] + sbe[r] * d[r];
        }
      }
    };

    // ---------------- output block: token block R, column tiles 2 nh, 2 nh + 1
    if constexpr (!ST) {
    // X rows of this wave's token block (with shared D tiles: loaded after B3, so they do not
    // hold registers through the D tiles and the state update)
    bf16x8 xh[KP / 32], xl[KP / 32];
    auto load_x = [&]() {
#pragma unroll
      for (int kc = 0; kc < KP / 32; ++kc) {
        xh[kc] = PX.hi8(16 * R + l16, 32 * kc + 8 * lg);
        xl[kc] = xh[kc];
        if constexpr (XL) xl[kc] = PX.lo8(16 * R + l16, 32 * kc + 8 * lg);
      }
    };
    if constexpr (!SHARED_D) load_x();
    // D tiles (P, R) on the causal side: lane holds D[16P+4lg+r][16R+l16]
    const float dsc = FWD_DELTA ? 1.f : scale;   // the delta forward folds scale into X
    uint2 dh[4], dl[4];
    // causal D tile t = Rc (Rc + 1) / 2 + Pc, Pc <= Rc (Rc = R, Pc = P forward; 3 - R, 3 - P
    // reverse), packed bf16 hi / lo per lane; three independent MFMA chains (lo.hi, hi.lo,
    // hi.hi), the fragments of step kc + 1 read before the products of step kc
    auto dtile = [&](int t) -> uint4 {
      const int Rc = t >= 6 ? 3 : (t >= 3 ? 2 : (t >= 1 ? 1 : 0));
      const int Pc = t - Rc * (Rc + 1) / 2;
      const int Rt = REV ? 3 - Rc : Rc, Pt = REV ? 3 - Pc : Pc;
      f32x4 a0 = {0.f, 0.f, 0.f, 0.f}, a1 = a0, a2 = a0;
      bf16x8 fz[2][2], fx[2][2];
      auto ld = [&](int kc, int b) {
        fz[b][0] = PZ.hi8(16 * Pt + l16, 32 * kc + 8 * lg);
        fx[b][0] = PX.hi8(16 * Rt + l16, 32 * kc + 8 * lg);
        if constexpr (XL) {
          fz[b][1] = PZ.lo8(16 * Pt + l16, 32 * kc + 8 * lg);
          fx[b][1] = PX.lo8(16 * Rt + l16, 32 * kc + 8 * lg);
        }
      };
      ld(0, 0);
#pragma unroll
      for (int kc = 0; kc < KP / 32; ++kc) {
        const int b = kc & 1;
        if (kc + 1 < KP / 32) ld(kc + 1, b ^ 1);
        if constexpr (XL) {
          a0 = mfma(fz[b][1], fx[b][0], a0);
          a1 = mfma(fz[b][0], fx[b][1], a1);
        }
        a2 = mfma(fz[b][0], fx[b][0], a2);
      }
      f32x4 acc;
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[r] = (a0[r] + a1[r]) + a2[r];
      const int rr = 16 * Rt + l16;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int pp = 16 * Pt + 4 * lg + r;
        const bool keep = REV ? (pp >= rr) : (pp <= rr);
        acc[r] = keep ? acc[r] * dsc : 0.f;
      }
      uint2 th, tl;
      acc_to_bf16x4(acc, th, tl);
      return make_uint4(th.x, th.y, tl.x, tl.y);
    };
    auto read_d = [&](const uint4* base) {
#pragma unroll
      for (int P = 0; P < 4; ++P) {
        dh[P] = make_uint2(0u, 0u);
        dl[P] = make_uint2(0u, 0u);
        const bool live = REV ? (P >= R) : (P <= R);
        if (live) {
          const int Rc = REV ? 3 - R : R, Pc = REV ? 3 - P : P;
          const uint4 x = base[(Rc * (Rc + 1) / 2 + Pc) * 64 + lane];
          dh[P] = make_uint2(x.x, x.y);
          dl[P] = make_uint2(x.z, x.w);
        }
      }
    };
    // forward delta rule (no LDS left for the shared tiles): the D tiles are computed now, in
    // the same even split (wave w: tiles w, w + 8), and handed over through the Z plane once
    // the v_new phase below has passed B3 (Z is not read after the D tiles)
    uint4 dz[2];
    if constexpr (SHARED_D) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int t = wave + 8 * u;
        if (t < 10) sDt[t * 64 + lane] = dtile(t);
      }
      // the state update reads only the Z^T / Y^T planes: it fills the wait for the D tiles
      state_update();
      __syncthreads();  // B3: D tiles visible
      load_x();
      read_d(sDt);
    } else if constexpr (FWD_DELTA) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int t = wave + 8 * u;
        if (t < 10) dz[u] = dtile(t);
      }
    } else {
#pragma unroll
    for (int P = 0; P < 4; ++P) {
      dh[P] = make_uint2(0u, 0u);
      dl[P] = make_uint2(0u, 0u);
      const bool live = REV ? (P >= R) : (P <= R);
      if (live) {
        f32x4 t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kc = 0; kc < KP / 32; ++kc)
          t = mma<XL, XL>(t, PZ.hi8(16 * P + l16, 32 * kc + 8 * lg),
                          PZ.lo8(16 * P + l16, 32 * kc + 8 * lg), xh[kc], xl[kc]);
        const int rr = 16 * R + l16;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int pp = 16 * P + 4 * lg + r;
          const bool keep = REV ? (pp >= rr) : (pp <= rr);
          t[r] = keep ? t[r] * dsc : 0.f;
        }
        acc_to_bf16x4(t, dh[P], dl[P]);
      }
    }
    }  // SHARED_D

    if constexpr (FWD_DELTA) {
      // v_new = u - w S for (token block R, column tiles 2nh, 2nh+1).  The A operand
      // w 2^-Gm is read straight from HBM in the MFMA row layout (against H^T = 2^Gm S).
      const size_t e0 = (size_t)(row0 + t0) * H + hh;
      const rsrc_t Rvn = chunk_rsrc(p.y32, e0, nval, (int)rowV, V);
      const rsrc_t Rw = chunk_rsrc(p.w, e0, nval, (int)rowK, LDK);
      const rsrc_t Ru = chunk_rsrc(p.u, e0, nval, (int)rowV, V);
      bf16x8 wh[KP / 32], wl[KP / 32];
#pragma unroll
      for (int kc = 0; kc < KP / 32; ++kc) {
        const int k0 = 32 * kc + 8 * lg;
        float a[8];
        if constexpr (HOIST) {
          unpack4(wraw[kc][0], a);
          unpack4(wraw[kc][1], a + 4);
        } else {
          const int trow = 16 * R + l16;
          const uint32_t o = k0 < K ? ((uint32_t)trow * rowK + k0) * 4u : kOOB;
          unpack4(bld128(Rw, o, 0), a);
          unpack4(bld128(Rw, o == kOOB ? kOOB : o + 16u, 0), a + 4);
        }
        const float4 g0 = *(const float4*)egm_at(k0), g1 = *(const float4*)egm_at(k0 + 4);
        const float eg[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
        uint32_t h4[4], l4[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) split_bf16x2(a[2 * e] * eg[2 * e], a[2 * e + 1] * eg[2 * e + 1], h4[e], l4[e]);
        wh[kc] = __builtin_bit_cast(bf16x8, make_uint4(h4[0], h4[1], h4[2], h4[3]));
        wl[kc] = __builtin_bit_cast(bf16x8, make_uint4(l4[0], l4[1], l4[2], l4[3]));
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int nn = 2 * nh + j;
        const int vv = vt * BV + 16 * nn + l16;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kc = 0; kc < KP / 32; ++kc)
          acc = mma<true, true>(acc, wh[kc], wl[kc], PHt.hi8(16 * nn + l16, 32 * kc + 8 * lg),
                                PHt.lo8(16 * nn + l16, 32 * kc + 8 * lg));
        // lane holds (token 16R + 4lg + r, column 16nn + l16)
        float vn[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int tok = 16 * R + 4 * lg + r;
          const uint32_t o = vv < V ? ((uint32_t)tok * rowV + vv) * 4u : kOOB;
          vn[r] = (HOIST ? ur[j][r] : __uint_as_float(bld32(Ru, o, 0))) - acc[r];
          bst32(Rvn, __float_as_uint(vn[r]), o, 0);
        }
        put_n<true, 4>(PYt, 16 * nn + l16, 16 * R + 4 * lg, vn);
      }
      __syncthreads();  // B3: v_new^T plane complete
      uint4* zD = (uint4*)sZT;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int t = wave + 8 * u;
        if (t < 10) zD[t * 64 + lane] = dz[u];
      }
      __syncthreads();  // B3b: D tiles visible
      read_d(zD);
    }

    if constexpr (REV_DELTA) {
      // dv_new = k~ (alpha dS) + D^T dO, token-major: lane holds (token 16R + 4lg + r,
      // column 16nn + l16); stored transposed per chunk ([V][C]) and kept for the update
      f32x4 dvn[2];
      const rsrc_t Rd = make_rsrc(p.y32 + ((size_t)(cbase + c) * H + hh) * V * C, (long long)V * C * 4);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int nn = 2 * nh + j;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kc = 0; kc < KP / 32; ++kc)
          acc = mma<true, true>(acc, xh[kc], xl[kc], PHt.hi8(16 * nn + l16, 32 * kc + 8 * lg),
                                PHt.lo8(16 * nn + l16, 32 * kc + 8 * lg));
#pragma unroll
        for (int Pp = 0; Pp < 2; ++Pp) {
          const int P0 = 2 * Pp, P1 = 2 * Pp + 1;
          if (P1 >= R) {
            const bf16x8 bh = PYt.hi44(16 * nn + l16, 16 * P0 + 4 * lg, 16 * P1 + 4 * lg);
            bf16x8 bl = bh;
            if constexpr (SY) bl = PYt.lo44(16 * nn + l16, 16 * P0 + 4 * lg, 16 * P1 + 4 * lg);
            acc = mma<true, SY>(acc, cat44(dh[P0], dh[P1]), cat44(dl[P0], dl[P1]), bh, bl);
          }
        }
        dvn[j] = acc;
        const int vv = vt * BV + 16 * nn + l16;
        bst128(Rd, make_uint4(__float_as_uint(acc[0]), __float_as_uint(acc[1]), __float_as_uint(acc[2]),
                              __float_as_uint(acc[3])),
               vv < V ? ((uint32_t)vv * C + 16 * R + 4 * lg) * 4u : kOOB, 0);
      }
      __syncthreads();  // B3: every wave is done with X, Z, Z^T, Y^T and H^T
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const float x[4] = {dvn[j][0], dvn[j][1], dvn[j][2], dvn[j][3]};
        put_n<true, 4>(PDt, 16 * (2 * nh + j) + l16, 16 * R + 4 * lg, x);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float x[RPT];
#pragma unroll
        for (int i = 0; i < RPT; ++i) x[i] = j == 0 ? rw[i].x : (j == 1 ? rw[i].y : (j == 2 ? rw[i].z : rw[i].w));
        put_n<true, RPT>(PWt, c0 + j, r0, x);
      }
      __syncthreads();  // B4: w^T and dv_new^T planes visible
    } else {
      // out^T tiles (nn, R); lane writes out[token 16R + l16][v = 16 nn + 4 lg + 0..3]
      const int tok = 16 * R + l16;
      const size_t eo = (size_t)(row0 + t0) * H + hh;
      const rsrc_t Ro = chunk_rsrc((const TIn*)p.out, eo, nval, (int)rowV, V);
      const uint32_t oo = ((uint32_t)tok * rowV + vt * BV + 4 * lg) * ES;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int nn = 2 * nh + j;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kc = 0; kc < KP / 32; ++kc)
          acc = mma<true, XL>(acc, PHt.hi8(16 * nn + l16, 32 * kc + 8 * lg),
                              PHt.lo8(16 * nn + l16, 32 * kc + 8 * lg), xh[kc], xl[kc]);
        // out^T += Y^T D  (contraction over p, two 16-blocks per MFMA)
#pragma unroll
        for (int Pp = 0; Pp < 2; ++Pp) {
          const int P0 = 2 * Pp, P1 = 2 * Pp + 1;
          const bool live = REV ? (P1 >= R) : (P0 <= R);
          if (live) {
            const bf16x8 ah = PYt.hi44(16 * nn + l16, 16 * P0 + 4 * lg, 16 * P1 + 4 * lg);
            bf16x8 al = ah;
            if constexpr (SY) al = PYt.lo44(16 * nn + l16, 16 * P0 + 4 * lg, 16 * P1 + 4 * lg);
            acc = mma<SY, true>(acc, ah, al, cat44(dh[P0], dh[P1]), cat44(dl[P0], dl[P1]));
          }
        }
        if constexpr (RSH) {
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[r] *= p.oscale;
        }
        if constexpr (GV) {
          const float4 e4 = *(const float4*)(sE + tok * LE + 16 * nn + 4 * lg);
          acc[0] *= e4.x; acc[1] *= e4.y; acc[2] *= e4.z; acc[3] *= e4.w;
        }
        const int v0 = vt * BV + 16 * nn + 4 * lg;
        if (VAR != 0 || p.acc_mode == 0) {
          Wd::st4(Ro, acc, v0 < V ? oo : kOOB, (uint32_t)(16 * nn * ES));
        } else {
          // channel slices: the fp32 sum of the slices' outputs (element offset as oo's)
          const rsrc_t Ra = chunk_rsrc(p.acc32, eo, nval, (int)rowV, V);
          const uint32_t fo = (v0 < V) ? ((uint32_t)tok * rowV + v0) * 4u : kOOB;
          acc_slice_t<TIn>(Ro, Ra, acc, fo, v0 < V ? oo : kOOB, (uint32_t)(16 * nn * ES), p.acc_mode);
        }
      }
    }

    }  // !ST

    if constexpr (!SHARED_D) state_update();
  };

  if constexpr (PF == 2) {
    for (int it = 0; it < NTs; it += 2) {
      body(it, rsA);
      if (it + 1 < NTs) body(it + 1, rsB);
    }
  } else {
    for (int it = 0; it < NTs; ++it) body(it, rsA);
  }

  if constexpr (ST) {
    // one lane per K row (first wave of each K block, first column group, V tile 0)
    if (p.dec_fin && vt == 0 && ((wave * NHT) % (BV / 16)) == 0 && l16 == 0) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int kr = 16 * msb + 4 * lg + r;
        if (kr < K) p.dec_fin[(size_t)(n * H + hh) * LDK + kr] = dsum[r];
      }
    }
  }
  if (p.s_fin) {
    const rsrc_t Rsf = make_rsrc(p.s_fin + s_base, (long long)LDK * V * 4);
#pragma unroll
    for (int i = 0; i < NHT; ++i) {
      const uint32_t o = sel_off(i);
#pragma unroll
      for (int r = 0; r < 4; ++r) bst32(Rsf, __float_as_uint(S[i][r]), o, (uint32_t)(r * V * 4));
    }
  }
}

template <typename TIn, bool REV, bool DELTA>
hipError_t launch_gla_sweep(const SweepParams& p, hipStream_t s) {
  if constexpr (std::is_same<TIn, uint16_t>::value && !DELTA) {
    if (gla_pipe_eligible(p)) return launch_gla_pipe<REV>(p, s);
  }
  // fp16 checkpoints: whole-width state rows with the plain layout (ckpt_par 0, no slices)
  const bool plain = !p.acc_mode && !p.ldk;
  if (p.ckpt16 && (!p.ckpt || !p.ckpt_scale || p.ckpt_par || !plain)) return hipErrorInvalidValue;
  const int var = p.ckpt16 ? 1 : ((plain && !p.ckpt) ? 2 : 0);
  if (var == 1 && !std::is_same<TIn, uint16_t>::value) return hipErrorInvalidValue;
  const int kp = p.K <= 32 ? 32 : (p.K <= 64 ? 64 : 128);
  dim3 grid(p.NV * p.H * p.N);
  const bool gk = DELTA || p.gate_mode == kGateK;
#define TOPS_SWEEP(KPV, GKV) \
  hipLaunchKernelGGL((gla_sweep_kernel<TIn, KPV, REV, DELTA, false, GKV>), grid, dim3(512), 0, s, p)
  // the delta sweeps (KDA) and the bf16 value-side-gate sweeps are compiled per feature set
#define TOPS_SWEEP_V(KPV, GKV, YGV) \
  if (var == 1) { \
    if constexpr (std::is_same<TIn, uint16_t>::value) \
      hipLaunchKernelGGL((gla_sweep_kernel<TIn, KPV, REV, DELTA, false, GKV, YGV, 1>), grid, dim3(512), 0, s, p); \
  } else if (var == 2) hipLaunchKernelGGL((gla_sweep_kernel<TIn, KPV, REV, DELTA, false, GKV, YGV, 2>), grid, dim3(512), 0, s, p); \
  else hipLaunchKernelGGL((gla_sweep_kernel<TIn, KPV, REV, DELTA, false, GKV, YGV, 0>), grid, dim3(512), 0, s, p)
  // fp16 checkpoints: the delta sweeps and the bf16 one-gate-per-token sweeps here, the
  // per-channel-gate bf16 sweeps in the pipelined kernel (routed above)
  const bool yg2 = std::is_same<TIn, uint16_t>::value && !DELTA && !gk && !p.gshift &&
                   (p.gate_mode == kGateS || p.gate_mode == kGateGamma);
  if (var == 1 && !DELTA && !yg2) return hipErrorInvalidValue;
  if constexpr (DELTA) {
    if (kp == 32) { TOPS_SWEEP_V(32, true, 0); }
    else if (kp == 64) { TOPS_SWEEP_V(64, true, 0); }
    else { TOPS_SWEEP_V(128, true, 0); }
  } else if (gk) {
    if (kp == 32) TOPS_SWEEP(32, true);
    else if (kp == 64) TOPS_SWEEP(64, true);
    else TOPS_SWEEP(128, true);
  } else if (std::is_same<TIn, uint16_t>::value && !p.gshift &&
             (p.gate_mode == kGateS || p.gate_mode == kGateGamma)) {
    // one gate per token (bf16): on the value side, q and k stay exact
#define TOPS_SWEEP_YG(KPV, VARV) \
  hipLaunchKernelGGL((gla_sweep_kernel<uint16_t, KPV, REV, false, false, false, 2, VARV>), grid, dim3(512), 0, s, p)
    if constexpr (std::is_same<TIn, uint16_t>::value && !DELTA) {
#define TOPS_SWEEP_YGV(KPV) \
  if (var == 1) TOPS_SWEEP_YG(KPV, 1); else if (var == 2) TOPS_SWEEP_YG(KPV, 2); else TOPS_SWEEP_YG(KPV, 0)
      if (kp == 32) { TOPS_SWEEP_YGV(32); }
      else if (kp == 64) { TOPS_SWEEP_YGV(64); }
      else { TOPS_SWEEP_YGV(128); }
#undef TOPS_SWEEP_YGV
    }
#undef TOPS_SWEEP_YG
  } else {
    if (kp == 32) TOPS_SWEEP(32, false);
    else if (kp == 64) TOPS_SWEEP(64, false);
    else TOPS_SWEEP(128, false);
  }
#undef TOPS_SWEEP_V
#undef TOPS_SWEEP
  return hipGetLastError();
}

template <bool REV>
hipError_t launch_gla_sweep_gv(const SweepParams& p, hipStream_t s) {
  const int kp = p.K <= 32 ? 32 : (p.K <= 64 ? 64 : 128);
  dim3 grid(p.NV * p.H * p.N);
#define TOPS_SWEEP_GV(KPV) \
  hipLaunchKernelGGL((gla_sweep_kernel<uint16_t, KPV, REV, false, false, false, 1>), grid, dim3(512), 0, s, p)
  if (kp == 32) TOPS_SWEEP_GV(32);
  else if (kp == 64) TOPS_SWEEP_GV(64);
  else TOPS_SWEEP_GV(128);
#undef TOPS_SWEEP_GV
  return hipGetLastError();
}

template <typename TIn, bool REV>
hipError_t launch_gla_state_pass(const SweepParams& p, hipStream_t s) {
  const int kp = p.K <= 32 ? 32 : (p.K <= 64 ? 64 : 128);
  dim3 grid(p.NV * p.H * p.N);
#define TOPS_STATE(KPV, GKV) \
  hipLaunchKernelGGL((gla_sweep_kernel<TIn, KPV, REV, false, true, GKV>), grid, dim3(512), 0, s, p)
  if (p.gate_mode == kGateK) {
    if (kp == 32) TOPS_STATE(32, true);
    else if (kp == 64) TOPS_STATE(64, true);
    else TOPS_STATE(128, true);
  } else {
    if (kp == 32) TOPS_STATE(32, false);
    else if (kp == 64) TOPS_STATE(64, false);
    else TOPS_STATE(128, false);
  }
#undef TOPS_STATE
  return hipGetLastError();
}

template hipError_t launch_gla_state_pass<uint16_t, false>(const SweepParams&, hipStream_t);
template hipError_t launch_gla_state_pass<uint16_t, true>(const SweepParams&, hipStream_t);
template hipError_t launch_gla_state_pass<float, false>(const SweepParams&, hipStream_t);
template hipError_t launch_gla_state_pass<float, true>(const SweepParams&, hipStream_t);
template hipError_t launch_gla_state_pass<_Float16, false>(const SweepParams&, hipStream_t);
template hipError_t launch_gla_state_pass<_Float16, true>(const SweepParams&, hipStream_t);

template hipError_t launch_gla_sweep<uint16_t, false, false>(const SweepParams&, hipStream_t);
template hipError_t launch_gla_sweep<uint16_t, true, false>(const SweepParams&, hipStream_t);
template hipError_t launch_gla_sweep<float, false, false>(const SweepParams&, hipStream_t);
template hipError_t launch_gla_sweep<float, true, false>(const SweepParams&, hipStream_t);
template hipError_t launch_gla_sweep<_Float16, false, false>(const SweepParams&, hipStream_t);
template hipError_t launch_gla_sweep<_Float16, true, false>(const SweepParams&, hipStream_t);
template hipError_t launch_gla_sweep<uint16_t, false, true>(const SweepParams&, hipStream_t);
template hipError_t launch_gla_sweep<uint16_t, true, true>(const SweepParams&, hipStream_t);
template hipError_t launch_gla_sweep<float, false, true>(const SweepParams&, hipStream_t);
template hipError_t launch_gla_sweep<float, true, true>(const SweepParams&, hipStream_t);

}  // namespace tops

using namespace tops;

static int chunk_fwd_impl(const void* q, const void* k, const void* v, const float* g,
                          const float* h0, void* o, float* ht, float* h_ckpt,
                          const int32_t* cu_seqlens, const int32_t* chunk_offsets, int B, int T,
                          int H, int K, int V, int N, int dtype, float scale, int gate_mode,
                          void* stream, int ckpt_par = 0, int ldk = 0, float* o_sum = nullptr,
                          int acc_mode = 0, float* ckpt_scale = nullptr) {
  if (!q || !k || !v || !g || !o) return tops_set_error(TOPS_ERR_NULL, "gla_chunk_fwd: null tensor");
  if (B <= 0 || T <= 0 || H <= 0 || K <= 0 || V <= 0 || N <= 0)
    return tops_set_error(TOPS_ERR_SHAPE, "gla_chunk_fwd: non-positive dimension");
  if (K > 128 || (K % 8) || (V % 8))
    return tops_set_error(TOPS_ERR_SHAPE, "gla_chunk_fwd: need K <= 128, K % 8 == 0, V % 8 == 0");
  if (cu_seqlens && B != 1) return tops_set_error(TOPS_ERR_SHAPE, "gla_chunk_fwd: varlen needs B == 1");
  const int kw = ldk > 0 ? ldk : K;
  if (ldk && (ldk < K || (ldk % 8)))
    return tops_set_error(TOPS_ERR_SHAPE, "gla_chunk_fwd: ldk must be a multiple of 8, at least K");
  if ((long long)kChunk * H * (kw > V ? kw : V) * 4 >= (1LL << 31))
    return tops_set_error(TOPS_ERR_SHAPE, "gla_chunk_fwd: H * max(K, V) too large for 32-bit chunk offsets");
  if (acc_mode < 0 || acc_mode > 3 || (acc_mode && !o_sum))
    return tops_set_error(TOPS_ERR_SHAPE, "gla_chunk_fwd: acc_mode 1..3 needs the fp32 sum buffer");
  if (!cu_seqlens && N != B) return tops_set_error(TOPS_ERR_SHAPE, "gla_chunk_fwd: N must equal B");
  if (h_ckpt && cu_seqlens && !chunk_offsets)
    return tops_set_error(TOPS_ERR_NULL, "gla_chunk_fwd: varlen checkpoints need chunk_offsets");
  SweepParams p{q, k, g, v, h0, o, ht, h_ckpt, cu_seqlens, chunk_offsets,
                B, T, H, K, V, N, (V + 63) / 64, scale, gate_mode};
  p.ckpt_par = ckpt_par;
  p.ldk = ldk;
  p.acc32 = o_sum;
  p.acc_mode = acc_mode;
  if (ckpt_scale) {
    if (dtype != TOPS_BF16 || (gate_mode != kGateK && gate_mode != kGateS && gate_mode != kGateGamma) ||
        V > 128 || ldk || ckpt_par || !h_ckpt)
      return tops_set_error(TOPS_ERR_SHAPE, "chunk_fwd_c16: bf16, per-channel or per-token gates, V <= 128, no slices");
    p.ckpt16 = 1;
    p.ckpt_scale = ckpt_scale;
  }
  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  if (dtype == TOPS_BF16) e = launch_gla_sweep<uint16_t, false>(p, s);
  else if (dtype == TOPS_F32) e = launch_gla_sweep<float, false>(p, s);
  else if (dtype == TOPS_F16) e = launch_gla_sweep<_Float16, false>(p, s);
  else return tops_set_error(TOPS_ERR_DTYPE, "gla_chunk_fwd: dtype must be TOPS_F32, TOPS_BF16 or TOPS_F16");
  if (e != hipSuccess) return tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
  return TOPS_OK;
}

extern "C" int tops_gla_chunk_fwd(const void* q, const void* k, const void* v, const float* g,
                                  const float* h0, void* o, float* ht, float* h_ckpt,
                                  const int32_t* cu_seqlens, const int32_t* chunk_offsets,
                                  int B, int T, int H, int K, int V, int N, int dtype,
                                  float scale, void* stream) {
  return chunk_fwd_impl(q, k, v, g, h0, o, ht, h_ckpt, cu_seqlens, chunk_offsets, B, T, H, K, V, N,
                        dtype, scale, kGateK, stream);
}

extern "C" int tops_gla_chunk_fwd_c16(const void* q, const void* k, const void* v, const float* g,
                                      const float* h0, void* o, float* ht, uint16_t* h_ckpt16,
                                      float* h_scale, const int32_t* cu_seqlens,
                                      const int32_t* chunk_offsets, int B, int T, int H, int K,
                                      int V, int N, int dtype, float scale, void* stream) {
  if (!h_ckpt16 || !h_scale) return tops_set_error(TOPS_ERR_NULL, "gla_chunk_fwd_c16: null checkpoint");
  return chunk_fwd_impl(q, k, v, g, h0, o, ht, (float*)h_ckpt16, cu_seqlens, chunk_offsets, B, T, H,
                        K, V, N, dtype, scale, kGateK, stream, 0, 0, nullptr, 0, h_scale);
}

extern "C" int tops_simple_gla_chunk_fwd(const void* q, const void* k, const void* v,
                                         const float* g, const float* g_gamma, const float* h0,
                                         void* o, float* ht, float* h_ckpt,
                                         const int32_t* cu_seqlens, const int32_t* chunk_offsets,
                                         int B, int T, int H, int K, int V, int N, int dtype,
                                         float scale, void* stream) {
  if ((g == nullptr) == (g_gamma == nullptr))
    return tops_set_error(TOPS_ERR_NULL, "simple_gla_chunk_fwd: pass exactly one of g, g_gamma");
  return chunk_fwd_impl(q, k, v, g ? g : g_gamma, h0, o, ht, h_ckpt, cu_seqlens, chunk_offsets, B, T,
                        H, K, V, N, dtype, scale, g ? kGateS : kGateGamma, stream);
}

extern "C" int tops_simple_gla_chunk_fwd_c16(const void* q, const void* k, const void* v,
                                             const float* g, const float* g_gamma,
                                             const float* h0, void* o, float* ht,
                                             uint16_t* h_ckpt16, float* h_scale,
                                             const int32_t* cu_seqlens,
                                             const int32_t* chunk_offsets, int B, int T, int H,
                                             int K, int V, int N, int dtype, float scale,
                                             void* stream) {
  if ((g == nullptr) == (g_gamma == nullptr))
    return tops_set_error(TOPS_ERR_NULL, "simple_gla_chunk_fwd_c16: pass exactly one of g, g_gamma");
  if (!h_ckpt16 || !h_scale) return tops_set_error(TOPS_ERR_NULL, "simple_gla_chunk_fwd_c16: null checkpoint");
  return chunk_fwd_impl(q, k, v, g ? g : g_gamma, h0, o, ht, (float*)h_ckpt16, cu_seqlens,
                        chunk_offsets, B, T, H, K, V, N, dtype, scale, g ? kGateS : kGateGamma,
                        stream, 0, 0, nullptr, 0, h_scale);
}

extern "C" int tops_gla_chunk_fwd_gamma(const void* q, const void* k, const void* v,
                                        const float* g_gamma, const float* h0, void* o, float* ht,
                                        float* h_ckpt, const int32_t* cu_seqlens,
                                        const int32_t* chunk_offsets, int B, int T, int H, int K,
                                        int V, int N, int dtype, float scale, void* stream) {
  if (!g_gamma) return tops_set_error(TOPS_ERR_NULL, "gla_chunk_fwd_gamma: null g_gamma");
  return chunk_fwd_impl(q, k, v, g_gamma, h0, o, ht, h_ckpt, cu_seqlens, chunk_offsets, B, T, H, K,
                        V, N, dtype, scale, kGateGammaK, stream);
}

extern "C" int tops_chunk_fwd_paired(const void* q, const void* k, const void* v, const float* g,
                                     int gate_mode, const float* h0, void* o, float* ht,
                                     float* ckpt, const int32_t* cu_seqlens,
                                     const int32_t* chunk_offsets, int B, int T, int H, int K,
                                     int V, int N, int dtype, float scale, void* stream) {
  if (gate_mode < kGateK || gate_mode > kGateGammaK)
    return tops_set_error(TOPS_ERR_SHAPE, "chunk_fwd_paired: gate_mode must be 0..3");
  if (dtype != TOPS_BF16)
    return tops_set_error(TOPS_ERR_DTYPE, "chunk_fwd_paired: the interleaved layout takes TOPS_BF16");
  if (!ckpt) return tops_set_error(TOPS_ERR_NULL, "chunk_fwd_paired: null ckpt");
  return chunk_fwd_impl(q, k, v, g, h0, o, ht, ckpt, cu_seqlens, chunk_offsets, B, T, H, K, V, N,
                        dtype, scale, gate_mode, stream, 1);
}

extern "C" int tops_chunk_fwd_slice(const void* q, const void* k, const void* v, const float* g,
                                    int gate_mode, const float* h0, void* o, float* o_sum,
                                    int acc_mode, float* ht, float* h_ckpt,
                                    const int32_t* cu_seqlens, const int32_t* chunk_offsets, int B,
                                    int T, int H, int K, int V, int N, int ldk, int dtype,
                                    float scale, void* stream) {
  if (gate_mode < kGateK || gate_mode > kGateGammaK)
    return tops_set_error(TOPS_ERR_SHAPE, "chunk_fwd_slice: gate_mode must be 0..3");
  if (acc_mode != 1 && acc_mode != 2 && !o)
    return tops_set_error(TOPS_ERR_NULL, "chunk_fwd_slice: null o");
  // o is written only by acc_mode 0 and 3; the generic null check needs a pointer
  return chunk_fwd_impl(q, k, v, g, h0, o ? o : (void*)o_sum, ht, h_ckpt, cu_seqlens,
                        chunk_offsets, B, T, H, K, V, N, dtype, scale, gate_mode, stream, 0, ldk,
                        o_sum, acc_mode);
}

extern "C" int tops_chunk_reverse_fwd(const void* q, const void* k, const void* v, const float* g,
                                      int gate_mode, const float* h0, void* o, float* ht,
                                      const int32_t* cu_seqlens, int B, int T, int H, int K, int V,
                                      int N, int dtype, float scale, void* stream) {
  if (!q || !k || !v || !g || !o) return tops_set_error(TOPS_ERR_NULL, "chunk_reverse_fwd: null tensor");
  if (gate_mode < kGateK || gate_mode > kGateGammaK)
    return tops_set_error(TOPS_ERR_SHAPE, "chunk_reverse_fwd: gate_mode must be 0..3");
  if (B <= 0 || T <= 0 || H <= 0 || K <= 0 || V <= 0 || N <= 0)
    return tops_set_error(TOPS_ERR_SHAPE, "chunk_reverse_fwd: non-positive dimension");
  if (K > 128 || (K % 8) || (V % 8))
    return tops_set_error(TOPS_ERR_SHAPE, "chunk_reverse_fwd: need K <= 128, K % 8 == 0, V % 8 == 0");
  if (cu_seqlens && B != 1) return tops_set_error(TOPS_ERR_SHAPE, "chunk_reverse_fwd: varlen needs B == 1");
  if (!cu_seqlens && N != B) return tops_set_error(TOPS_ERR_SHAPE, "chunk_reverse_fwd: N must equal B");
  if ((long long)kChunk * H * (K > V ? K : V) * 4 >= (1LL << 31))
    return tops_set_error(TOPS_ERR_SHAPE, "chunk_reverse_fwd: H * max(K, V) too large for 32-bit chunk offsets");
  // The reverse sweep's state gradient recurrence D_t = diag(2^g'_(t+1)) D_(t+1) + q'_t dO'_t^T,
  // out_t = D_t^T k'_t, with q' = k, k' = q, dO' = v, scale 1 and g'_t = g_(t-1) (gshift) is
  // the reverse-time recurrence itself; o = scale * out.
  SweepParams p{k, q, g, v, h0, o, ht, nullptr, cu_seqlens, nullptr,
                B, T, H, K, V, N, (V + 63) / 64, 1.f, gate_mode};
  p.gshift = 1;
  p.oscale = scale;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  if (dtype == TOPS_BF16) e = launch_gla_sweep<uint16_t, true>(p, s);
  else if (dtype == TOPS_F32) e = launch_gla_sweep<float, true>(p, s);
  else if (dtype == TOPS_F16) e = launch_gla_sweep<_Float16, true>(p, s);
  else return tops_set_error(TOPS_ERR_DTYPE, "chunk_reverse_fwd: dtype must be TOPS_F32, TOPS_BF16 or TOPS_F16");
  if (e != hipSuccess) return tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
  return TOPS_OK;
}

static int gla_chunk_fwd_gv_impl(const void* q, const void* k, const void* v, const float* gv,
                                 const float* h0, void* o, float* o32, float* ht,
                                 const int32_t* cu_seqlens, int B, int T, int H, int K, int V,
                                 int N, int dtype, float scale, void* stream) {
  if (!q || !k || !v || !gv || (!o && !o32)) return tops_set_error(TOPS_ERR_NULL, "gla_chunk_fwd_gv: null tensor");
  if (dtype != TOPS_BF16)
    return tops_set_error(TOPS_ERR_DTYPE, "gla_chunk_fwd_gv: the value-gate sweep takes TOPS_BF16");
  if (B <= 0 || T <= 0 || H <= 0 || K <= 0 || V <= 0 || N <= 0)
    return tops_set_error(TOPS_ERR_SHAPE, "gla_chunk_fwd_gv: non-positive dimension");
  if (K > 128 || (K % 8) || (V % 8))
    return tops_set_error(TOPS_ERR_SHAPE, "gla_chunk_fwd_gv: need K <= 128, K % 8 == 0, V % 8 == 0");
  if (cu_seqlens && B != 1) return tops_set_error(TOPS_ERR_SHAPE, "gla_chunk_fwd_gv: varlen needs B == 1");
  if (!cu_seqlens && N != B) return tops_set_error(TOPS_ERR_SHAPE, "gla_chunk_fwd_gv: N must equal B");
  if ((long long)kChunk * H * (K > V ? K : V) * 4 >= (1LL << 31))
    return tops_set_error(TOPS_ERR_SHAPE, "gla_chunk_fwd_gv: H * max(K, V) too large for 32-bit chunk offsets");
  SweepParams p{q, k, gv, v, h0, o ? o : (void*)o32, ht, nullptr, cu_seqlens, nullptr,
                B, T, H, K, V, N, (V + 63) / 64, scale, kGateGamma};
  if (o32) {
    // the output in fp32 (acc_mode 1 writes the sum buffer only), and in bf16 as well when o
    // is given (acc_mode 4, both from the same accumulator)
    p.acc32 = o32;
    p.acc_mode = o ? 4 : 1;
  }
  hipError_t e = launch_gla_sweep_gv<false>(p, (hipStream_t)stream);
  if (e != hipSuccess) return tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
  return TOPS_OK;
}

extern "C" int tops_gla_chunk_fwd_gv(const void* q, const void* k, const void* v, const float* gv,
                                     const float* h0, void* o, float* ht,
                                     const int32_t* cu_seqlens, int B, int T, int H, int K, int V,
                                     int N, int dtype, float scale, void* stream) {
  if (!o) return tops_set_error(TOPS_ERR_NULL, "gla_chunk_fwd_gv: null tensor");
  return gla_chunk_fwd_gv_impl(q, k, v, gv, h0, o, nullptr, ht, cu_seqlens, B, T, H, K, V, N,
                               dtype, scale, stream);
}

extern "C" int tops_gla_chunk_fwd_gv32(const void* q, const void* k, const void* v, const float* gv,
                                       const float* h0, float* o32, void* o, float* ht,
                                       const int32_t* cu_seqlens, int B, int T, int H, int K,
                                       int V, int N, int dtype, float scale, void* stream) {
  if (!o32) return tops_set_error(TOPS_ERR_NULL, "gla_chunk_fwd_gv32: null tensor");
  return gla_chunk_fwd_gv_impl(q, k, v, gv, h0, o, o32, ht, cu_seqlens, B, T, H, K, V, N,
                               dtype, scale, stream);
}

// the shape checks of the chunked value-gate and reverse entries
static int gv_shape_check(const char* who, int B, int T, int H, int K, int V, int N,
                          const int32_t* cu_seqlens, int dtype) {
  char msg[160];
  if (dtype != TOPS_BF16) {
    snprintf(msg, sizeof msg, "%s: dtype must be TOPS_BF16", who);
    return tops_set_error(TOPS_ERR_DTYPE, msg);
  }
  if (B <= 0 || T <= 0 || H <= 0 || K <= 0 || V <= 0 || N <= 0 || K > 128 || (K % 8) || (V % 8) ||
      (cu_seqlens && B != 1) || (!cu_seqlens && N != B) ||
      (long long)kChunk * H * (K > V ? K : V) * 4 >= (1LL << 31)) {
    snprintf(msg, sizeof msg, "%s: need positive sizes, K <= 128, K and V multiples of 8, "
             "varlen with B == 1 (else N == B)", who);
    return tops_set_error(TOPS_ERR_SHAPE, msg);
  }
  return TOPS_OK;
}

extern "C" int tops_gla_chunk_bwd_dv_gv32(const void* q, const void* k, const void* do_,
                                          const float* gv, const float* dht, float* dv32,
                                          float* dh0, const int32_t* cu_seqlens, int B, int T,
                                          int H, int K, int V, int N, int dtype, float scale,
                                          void* stream) {
  if (!q || !k || !do_ || !gv || !dv32) return tops_set_error(TOPS_ERR_NULL, "gla_chunk_bwd_dv_gv32: null tensor");
  int rc = gv_shape_check("gla_chunk_bwd_dv_gv32", B, T, H, K, V, N, cu_seqlens, dtype);
  if (rc != TOPS_OK) return rc;
  SweepParams p{q, k, gv, do_, dht, dv32, dh0, nullptr, cu_seqlens, nullptr,
                B, T, H, K, V, N, (V + 63) / 64, scale, kGateGamma};
  p.acc32 = dv32;
  p.acc_mode = 1;
  hipError_t e = launch_gla_sweep_gv<true>(p, (hipStream_t)stream);
  if (e != hipSuccess) return tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
  return TOPS_OK;
}

extern "C" int tops_gla_chunk_rev_dv(const void* q, const void* k, const float* g, const void* do_,
                                     const float* dht, void* dv, float* dh0,
                                     const int32_t* cu_seqlens, int B, int T, int H, int K, int V,
                                     int N, int dtype, float scale, void* stream) {
  if (!q || !k || !g || !do_ || !dv) return tops_set_error(TOPS_ERR_NULL, "gla_chunk_rev_dv: null tensor");
  int rc = gv_shape_check("gla_chunk_rev_dv", B, T, H, K, V, N, cu_seqlens, dtype);
  if (rc != TOPS_OK) return rc;
  SweepParams p{q, k, g, do_, dht, dv, dh0, nullptr, cu_seqlens, nullptr,
                B, T, H, K, V, N, (V + 63) / 64, scale, kGateK};
  hipError_t e = launch_gla_sweep<uint16_t, true>(p, (hipStream_t)stream);
  if (e != hipSuccess) return tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
  return TOPS_OK;
}
