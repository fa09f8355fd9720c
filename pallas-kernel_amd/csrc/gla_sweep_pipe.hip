// Software-pipelined GLA chunk sweep for bf16 inputs with per-channel gates (the chunk_gla
// hot path: the forward of tops/ops/gla/chunk.py:1103-1199 and the state-gradient sweep of its
// backward, chunk.py:1447-1509 with tops/ops/common/chunk_h.py:685-878).
//
// Same products and operand values as gla_sweep_kernel (gla_sweep.hip, instance TIn = bf16,
// DELTA = ST = false, GK = true, YG = 0); the schedule differs, the state is held transposed
// (each lane keeps four adjacent V columns of one K row, so it needs one decay factor instead
// of four and stores its fp16 checkpoint run directly; the state update computes S^T tiles,
// a last-bit difference in the fp32 sums), and so do the planes: the state update and the intra output products read
// Z~ and Y transposed out of their row-major planes (ds_read_b64_tr_b16) where the serial
// kernel writes separate Z~^T / Y^T planes, 40 KB fewer LDS writes per chunk and 126 KB of
// LDS instead of 163 KB.  The serial kernel runs each chunk as
//   gate cumsum | B1 | VALU staging (exponentials, bf16 hi / lo splits) + plane writes | B2 |
//   D tiles + state update (MFMA) | B3 | output products (MFMA)
// and the VALU staging (~600 VALU instructions per wave, 4 cycles each on a 16-lane SIMD)
// cannot overlap the LDS-bound MFMA phases behind the barriers.  Here the staging of chunk
// c + 1 is computed into registers while chunk c's MFMA phase runs, so each chunk is
//   B1 | plane writes from registers, partial gate cumsum of c + 1 | B2 |
//   D tiles + state update of c, staging of c + 1 (VALU) | B3 | output products of c
// The gate totals of chunk c + 1 are exchanged across the B2 barrier of chunk c (sTot is read
// only between B2 and B3 and written only between B1 and B2, so one buffer serves).
#include <stdlib.h>

#include "gla_sweep.h"
#include "tops_common.h"
#include "tops_hip.h"

namespace tops {

// Keeps the computation of x at this point of the program: the compiler may otherwise sink
// the staging arithmetic past the barriers to its first use (the plane writes of the next
// chunk), where nothing overlaps it.
__device__ __forceinline__ void pin(uint32_t& x) { asm volatile("" : "+v"(x)); }
__device__ __forceinline__ void pin(float& x) { asm volatile("" : "+v"(x)); }

// Phase clocks (a library built with -DTOPS_PHASE_CLOCKS only; the regular build compiles
// none of this): per wave, the shader clock (s_memtime) spent in each interval of the chunk
// loop, summed over the chunks, slots 0 B1 wait, 1 plane writes + next gate scan, 2 B2 wait,
// 3 matrix phase (H^T plane, checkpoint, D tiles, state update, next chunk's staging and
// loads), 4 B3 wait, 5 output products; slot 6 the loop's s_memtime span, slot 7 its
// s_memrealtime (100 MHz) span.  The reads sit at barriers, where the LDS counter is
// drained anyway, and at the loop's ends.
#ifdef TOPS_PHASE_CLOCKS
constexpr bool kPhaseClocks = true;
#else
constexpr bool kPhaseClocks = false;
#endif
template <bool ON>
struct PhaseClock {
  __device__ void start() {}
  __device__ void tick(int) {}
  __device__ void finish(unsigned long long*, int) {}
};
template <>
struct PhaseClock<true> {
  uint64_t ph[6], t, t0, r0;
  __device__ void start() {
#pragma unroll
    for (int j = 0; j < 6; ++j) ph[j] = 0;
    t = t0 = __builtin_amdgcn_s_memtime();
    r0 = __builtin_amdgcn_s_memrealtime();
  }
  __device__ void tick(int j) {
    const uint64_t x = __builtin_amdgcn_s_memtime();
    ph[j] += x - t;
    t = x;
  }
  // slot: workgroup * 8 + wave; lane 0 writes (vector stores)
  __device__ void finish(unsigned long long* out, int slot) {
    const uint64_t t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
    if (out == nullptr || (threadIdx.x & 63) != 0) return;
    const rsrc_t R = make_rsrc(out + (size_t)slot * 8, 64);
    const uint64_t v[8] = {ph[0], ph[1], ph[2], ph[3], ph[4], ph[5], t1 - t0, r1 - r0};
#pragma unroll
    for (int j = 0; j < 8; ++j) bst64(R, make_uint2((uint32_t)v[j], (uint32_t)(v[j] >> 32)), 8u * j, 0);
  }
};

// VAR selects the features an instance compiles: 1 = training with fp16 checkpoints (every
// chunk, whole-width rows, no slices), 2 = no checkpoints and no slices (inference), 0 = the
// rest (fp32 or paired checkpoints, channel slices).  Fewer live values keep the scalar
// registers from spilling into VGPR lanes.
template <int KP, bool REV, int VAR>
__global__ __launch_bounds__(512) void gla_pipe_kernel(SweepParams p) {
  constexpr int NW = 8;
  constexpr int NTH = 64 * NW;
  constexpr int C = kChunk, BV = 64;
  constexpr int NQ = KP / 4;             // column quads of a [C][KP] tile
  constexpr int NSEG = NTH / NQ;         // row segments
  constexpr int RPT = C / NSEG;          // rows per thread (4, 2, 1)
  constexpr int CQL = 8, SGL = 32 / CQL; // a half-wave: 8 column quads x 4 row segments
  constexpr int NCQH = NQ / CQL;
  constexpr int NSGH = NSEG / SGL;       // segment groups
  static_assert(NQ % CQL == 0, "KP must be a multiple of 32");
  static_assert(CQL == 8 && SGL == 4, "the segment scan takes 8 column quads x 4 segments");
  static_assert(RPT == 1 || RPT == 2 || RPT == 4, "KP must be 32, 64 or 128");
  constexpr int LQ = KP + 8, LY = BV + 8, LH = BV + 8;
  constexpr int NHT = (KP / 16) * (BV / 16) / NW;  // state tiles per wave
  constexpr int YR = C * BV / (2 * NTH);
  static_assert(YR == 4, "Y staging assumes 4 rows x 2 columns per thread");
  constexpr int ES = 2;

  __shared__ __attribute__((aligned(16))) uint16_t sX[2 * C * LQ];
  __shared__ __attribute__((aligned(16))) uint16_t sZ[2 * C * LQ];
  __shared__ __attribute__((aligned(16))) uint16_t sY[C * LY];
  __shared__ __attribute__((aligned(16))) uint16_t sH[2 * KP * LH];   // alpha S, [K][BV] hi / lo
  __shared__ __attribute__((aligned(16))) float sTot[NSGH * KP];
  __shared__ __attribute__((aligned(16))) uint4 sDt[10 * 64];
  __shared__ uint32_t sMx[NW];                // fp16 checkpoints: each wave's largest |S|

  const Plane PX{sX, sX + C * LQ, LQ};
  const Plane PZ{sZ, sZ + C * LQ, LQ};
  const Plane PY{sY, sY, LY};   // Y = v (forward) or dO (reverse), [C][BV], bf16 as read
  const Plane PH{sH, sH + KP * LH, LH};

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lg = lane >> 4;
  // output token block of the wave (the reverse sweep numbers its blocks from the end, so that
  // in both directions a wave's first D tile lies in its output block for waves 0, 2, 4-7)
  const int R = REV ? 3 - (wave >> 1) : (wave >> 1);
  const int nh = wave & 1;
  const int msb = (wave * NHT) / (BV / 16);
  const int wg = xcd_remap(blockIdx.x, gridDim.x, p.NV);
  const int vt = wg % p.NV;
  const int hh = (wg / p.NV) % p.H;
  int n = wg / (p.NV * p.H);
  auto seq_end = [&](int j) { return p.seg_end ? p.seg_end[j] : p.cu_seqlens[j + 1]; };
  if (p.cu_seqlens && p.N > 1 && p.N <= 256) {
    // varlen: longest sequence first (LPT) over the slots, ties by index
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
    __syncthreads();
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
  const int NTs = cdiv(L, C);

  // ---- staging coordinates (as gla_sweep_kernel)
  const int hw = tid >> 5;
  const int sgl = (lane & 31) / CQL;
  const int sgh = hw / NCQH;
  const int cq = (lane & 31) % CQL + CQL * (hw % NCQH), seg = sgl + SGL * sgh;
  const int c0 = 4 * cq, r0 = seg * RPT;
  const bool colok = c0 < K;
  const int yc = (lane & 7) + 8 * (hw & 3), yseg = ((lane >> 3) & 3) + 4 * (hw >> 2);
  const int yv = vt * BV + 2 * yc;
  const bool ycolok = yv < V;
  const uint32_t rowK = (uint32_t)(H * LDK), rowV = (uint32_t)(H * V);
  const uint32_t offQ = colok ? ((uint32_t)r0 * rowK + c0) * ES : kOOB;
  const uint32_t offG = colok ? ((uint32_t)r0 * rowK + c0) * 4u : kOOB;
  const uint32_t offY = ycolok ? ((uint32_t)(yseg * YR) * rowV + yv) * ES : kOOB;

  // ---- state tiles: tile i of this wave -> (msb, nn), held transposed: lane (l16, lg) has
  // S[k = 16 msb + l16][v = 16 nn + 4 lg + r], r = 0..3 (four adjacent columns of one row)
  f32x4 S[NHT];
  const int krow = 16 * msb + l16;
  // s0 / s_fin rows of this (sequence, head): one 16-byte run per tile and lane (V % 8 == 0
  // keeps a run that starts inside a row inside it); no s0: an empty range loads zeros
  const size_t s_base = (size_t)(n * H + hh) * LDK * V;
  auto srun = [&](int i) {
    const int vv = vt * BV + 16 * ((wave * NHT + i) % (BV / 16)) + 4 * lg;
    return (krow < K && vv < V) ? ((uint32_t)krow * V + vv) * 4u : kOOB;
  };
  {
    const rsrc_t Rs0 = make_rsrc(p.s0 ? p.s0 + s_base : nullptr, p.s0 ? (long long)LDK * V * 4 : 0);
#pragma unroll
    for (int i = 0; i < NHT; ++i) S[i] = __builtin_bit_cast(f32x4, bld128(Rs0, srun(i), 0));
  }
  __builtin_amdgcn_s_waitcnt(0);

  // ---- raw chunk registers: loaded one chunk ahead of their staging
  struct Raw {
    uint2 rq[RPT], rk[RPT];
    uint4 rg[RPT];
    uint32_t ry[YR];
  };
  Raw rs;
  // The chunk's resources end at its last valid token (chunk_rsrc), so the rows past it load
  // zeros without a mask; a chunk index outside the sequence has an empty range.
  auto load_chunk = [&](int c) {
    const bool in = c >= 0 && c < NTs;
    if (!in) c = 0;
    const int t0 = c * C;
    const int nval = in ? min(C, L - t0) : 0;
    const size_t e0 = (size_t)(row0 + t0) * H + hh;
    const rsrc_t Rq = chunk_rsrc((const uint16_t*)p.q, e0, nval, (int)rowK, LDK);
    const rsrc_t Rk = chunk_rsrc((const uint16_t*)p.k, e0, nval, (int)rowK, LDK);
    const rsrc_t Rg = chunk_rsrc(p.g, e0, nval, (int)rowK, LDK);
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      rs.rq[i] = bld64(Rq, offQ, i * rowK * ES);
      rs.rk[i] = bld64(Rk, offQ, i * rowK * ES);
      rs.rg[i] = bld128(Rg, offG, i * rowK * 4);
    }
    const rsrc_t Ry = chunk_rsrc((const uint16_t*)p.y, e0, nval, (int)rowV, V);
#pragma unroll
    for (int i = 0; i < YR; ++i) rs.ry[i] = bld32(Ry, offY, i * rowV * ES);
  };
  auto cidx = [&](int it) { return REV ? NTs - 1 - it : it; };

  // ---- the staged chunk: plane words and state factors, computed one chunk ahead
  uint32_t xh[RPT][2], xl[RPT][2], zh[RPT][2], zl[RPT][2], yw[YR];
  float sga, sal, sbe;                 // factors of this lane's state row krow
  // partial gate cumsum of the raw chunk (thread rows, then the half-wave scan); the group
  // totals go to sTot.  The scan over the four row segments of a column quad (lanes cq,
  // cq + 8, cq + 16, cq + 24 of the half-wave) runs on the VALU (seg8x4_scan).
  float G[RPT][4], pre[4];
  auto cumsum = [&]() {
    float gam[4];
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      float x[4];
      unpack4(rs.rg[i], x);
#pragma unroll
      for (int j = 0; j < 4; ++j) G[i][j] = x[j] * kLog2e + (i > 0 ? G[i - 1][j] : 0.f);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float t = G[RPT - 1][j];
      const float x = seg8x4_scan(t, lane);
      pre[j] = x - t;
      gam[j] = x;
    }
    if (sgl == SGL - 1) *(float4*)(sTot + sgh * KP + c0) = make_float4(gam[0], gam[1], gam[2], gam[3]);
  };
  // staging of the raw chunk after its totals are visible, in two parts so that each can be
  // scheduled beside one group of matrix products: stage_sums() completes the gate prefix
  // and the state factors, stage_rows(i0, i1) the X / Z plane words (bf16 hi / lo) of rows
  // i0 .. i1 - 1 of the thread
  float gm[4];
  auto stage_sums = [&]() {
    float gam[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) gam[j] = 0.f;
#pragma unroll
    for (int s2 = 0; s2 < NSGH; ++s2) {
      const float4 t = *(const float4*)(sTot + s2 * KP + c0);
      if (s2 < sgh) { pre[0] += t.x; pre[1] += t.y; pre[2] += t.z; pre[3] += t.w; }
      gam[0] += t.x; gam[1] += t.y; gam[2] += t.z; gam[3] += t.w;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) gm[j] = 0.5f * gam[j];
    float sgam = 0.f;
#pragma unroll
    for (int s2 = 0; s2 < NSGH; ++s2) sgam += sTot[s2 * KP + krow];
    const float g2 = 0.5f * sgam;
    sga = fast_exp2(sgam);
    sal = REV ? fast_exp2(sgam - g2) : scale * fast_exp2(g2);
    sbe = REV ? scale * fast_exp2(g2) : fast_exp2(sgam - g2);
    pin(sga); pin(sal); pin(sbe);
  };
  auto stage_rows = [&](int i0, int i1) {
#pragma unroll
    for (int i = i0; i < i1; ++i) {
      float qv[4], kv[4], xq[4], xk[4];
      unpack4(rs.rq[i], qv);
      unpack4(rs.rk[i], kv);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float Gv = G[i][j] + pre[j];
        xq[j] = 1.f * qv[j] * fast_exp2(Gv - gm[j]);
        xk[j] = kv[j] * fast_exp2(gm[j] - Gv);
      }
      const float* xx = REV ? xk : xq;
      const float* zz = REV ? xq : xk;
      split_bf16x2(xx[0], xx[1], xh[i][0], xl[i][0]);
      split_bf16x2(xx[2], xx[3], xh[i][1], xl[i][1]);
      split_bf16x2(zz[0], zz[1], zh[i][0], zl[i][0]);
      split_bf16x2(zz[2], zz[3], zh[i][1], zl[i][1]);
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        pin(xh[i][e]); pin(xl[i][e]); pin(zh[i][e]); pin(zl[i][e]);
      }
    }
  };
  auto stage = [&]() {
    stage_sums();
    stage_rows(0, RPT);
#pragma unroll
    for (int i = 0; i < YR; ++i) yw[i] = rs.ry[i];
  };
  // plane writes of the staged chunk (after B1: no wave reads the previous chunk's planes)
  auto write_planes = [&]() {
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      *(uint2*)(PX.hi + (r0 + i) * PX.ld + c0) = make_uint2(xh[i][0], xh[i][1]);
      *(uint2*)(PX.lo + (r0 + i) * PX.ld + c0) = make_uint2(xl[i][0], xl[i][1]);
      *(uint2*)(PZ.hi + (r0 + i) * PZ.ld + c0) = make_uint2(zh[i][0], zh[i][1]);
      *(uint2*)(PZ.lo + (r0 + i) * PZ.ld + c0) = make_uint2(zl[i][0], zl[i][1]);
    }
    // Y rows yseg * 4 + 0..3, columns 2 yc, 2 yc + 1
#pragma unroll
    for (int i = 0; i < YR; ++i) *(uint32_t*)(PY.hi + (yseg * YR + i) * PY.ld + 2 * yc) = yw[i];
  };

  // checkpoint: S as the state entering chunk c (stored at the start of the chunk's matrix
  // phase, which measured fastest of the placements tried: there, at the end of that phase,
  // and after the output products)
  auto ckpt_on = [&](int c) {
    if constexpr (VAR == 1) return true;
    if constexpr (VAR == 2) return false;
    return p.ckpt && (p.ckpt_par == 0 || ((cbase + c) & 1) == p.ckpt_par - 1);
  };
  // fp16 checkpoints: this wave's largest |S| into sMx (between B1 and B2; read after B2)
  auto ckpt_max = [&]() { state_absmax<NHT>(S, sMx, wave, lane); };
  auto store_ckpt = [&](int c) {
    if (!ckpt_on(c)) return;
    if constexpr (VAR == 1) {
      store_state16_t<NHT, NW>(S, sMx, (uint16_t*)p.ckpt + ((size_t)(cbase + c) * H + hh) * LDK * V,
                               p.ckpt_scale + ((size_t)(cbase + c) * H + hh) * p.NV + vt, K, V, vt,
                               wave, msb, lane, tid);
      return;
    }
    const rsrc_t Rck = make_rsrc(p.ckpt + ((size_t)(cbase + c) * H + hh) * LDK * V,
                                 (long long)K * V * 4);
#pragma unroll
    for (int i = 0; i < NHT; ++i) {
      const int nn = (wave * NHT + i) % (BV / 16);
      const int vv = vt * BV + 16 * nn + 4 * lg;
      // (V % 8 == 0: vv < V keeps the four columns inside the row)
      const uint32_t vo = (krow < K && vv < V) ? ((uint32_t)krow * V + vv) * 4u : kOOB;
      bst128(Rck, make_uint4(__float_as_uint(S[i][0]), __float_as_uint(S[i][1]),
                             __float_as_uint(S[i][2]), __float_as_uint(S[i][3])), vo, 0);
    }
  };

  // ---- prologue: chunk 0 staged, chunk 1 loaded
  if (NTs > 0) {
    load_chunk(cidx(0));
    cumsum();
    __syncthreads();
    stage();
    if (NTs > 1) load_chunk(cidx(1));
  }

  PhaseClock<kPhaseClocks> clk;
  clk.start();
  for (int it = 0; it < NTs; ++it) {
    const int c = cidx(it);
    const int t0 = c * C;
    const int nval = min(C, L - t0);

    if (it > 0) clk.tick(5);
    __syncthreads();  // B1: the previous chunk's planes and the totals are no longer read
    clk.tick(0);
    write_planes();
    if constexpr (VAR == 1) ckpt_max();
    // the state factors of this chunk, kept for its update (stage() overwrites them)
    const float cga = sga, cbe = sbe;
    cumsum();         // (past the last chunk: zeros, never staged into planes)
    clk.tick(1);
    __syncthreads();  // B2: planes and the next chunk's totals visible
    clk.tick(2);

    // H plane = alpha S (the state entering this chunk; read after B3 only)
#pragma unroll
    for (int i = 0; i < NHT; ++i) {
      const int nn = (wave * NHT + i) % (BV / 16);
      float x[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) x[r] = sal * S[i][r];
      put_n<true, 4>(PH, krow, 16 * nn + 4 * lg, x);
    }
    store_ckpt(c);

    // ---------------- D tiles of this chunk (shared through LDS), staging of the next
    // the output block's X~ fragments: kept from the wave's first D tile when that tile lies in
    // the output block (wave w: tile w, row block Rc(w) = w / 2 for w = 0, 2, 4..7)
    bf16x8 fxh[KP / 32], fxl[KP / 32];
    const bool xkeep = (wave == 0 || wave == 2 || wave >= 4);
    auto dtile = [&](int t) -> uint4 {
      const int Rc = t >= 6 ? 3 : (t >= 3 ? 2 : (t >= 1 ? 1 : 0));
      const int Pc = t - Rc * (Rc + 1) / 2;
      const int Rt = REV ? 3 - Rc : Rc, Pt = REV ? 3 - Pc : Pc;
      f32x4 a0 = {0.f, 0.f, 0.f, 0.f}, a1 = a0, a2 = a0;
#pragma unroll
      for (int kc = 0; kc < KP / 32; ++kc) {
        const bf16x8 zh8 = PZ.hi8(16 * Pt + l16, 32 * kc + 8 * lg);
        const bf16x8 xh8 = PX.hi8(16 * Rt + l16, 32 * kc + 8 * lg);
        const bf16x8 zl8 = PZ.lo8(16 * Pt + l16, 32 * kc + 8 * lg);
        const bf16x8 xl8 = PX.lo8(16 * Rt + l16, 32 * kc + 8 * lg);
        if (t == wave) {
          fxh[kc] = xh8;
          fxl[kc] = xl8;
        }
        a0 = mfma(zl8, xh8, a0);
        a1 = mfma(zh8, xl8, a1);
        a2 = mfma(zh8, xh8, a2);
      }
      f32x4 acc;
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[r] = (a0[r] + a1[r]) + a2[r];
      const int rr = 16 * Rt + l16;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int pp = 16 * Pt + 4 * lg + r;
        const bool keep = REV ? (pp >= rr) : (pp <= rr);
        acc[r] = keep ? acc[r] * scale : 0.f;
      }
      uint2 th, tl;
      acc_to_bf16x4(acc, th, tl);
      return make_uint4(th.x, th.y, tl.x, tl.y);
    };
    // (the staging of the next chunk is issued between the matrix products; past the last
    // chunk it stages zeros that are never written)
    stage_sums();
    sDt[wave * 64 + lane] = dtile(wave);
    stage_rows(0, RPT / 2 > 0 ? RPT / 2 : RPT);
    if (wave < 2) sDt[(wave + 8) * 64 + lane] = dtile(wave + 8);

    // state update: S = 2^Gamma S + beta (Z~^T Y)
    {
      f32x4 dsu[NHT];
#pragma unroll
      for (int i = 0; i < NHT; ++i) dsu[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kc = 0; kc < C / 32; ++kc) {
        const bf16x8 fzh = tr_read8(PZ.hi, PZ.ld, 32 * kc, 16 * msb, lane);
        const bf16x8 fzl = tr_read8(PZ.lo, PZ.ld, 32 * kc, 16 * msb, lane);
        bf16x8 fyh[NHT];
#pragma unroll
        for (int i = 0; i < NHT; ++i) {
          const int nn = (wave * NHT + i) % (BV / 16);
          fyh[i] = tr_read8(PY.hi, PY.ld, 32 * kc, 16 * nn, lane);
        }
#pragma unroll
        for (int i = 0; i < NHT; ++i) dsu[i] = mfma(fyh[i], fzl, dsu[i]);
#pragma unroll
        for (int i = 0; i < NHT; ++i) dsu[i] = mfma(fyh[i], fzh, dsu[i]);
      }
      if constexpr (RPT > 1) stage_rows(RPT / 2, RPT);
#pragma unroll
      for (int i = 0; i < YR; ++i) yw[i] = rs.ry[i];
      load_chunk(cidx(it + 2));
#pragma unroll
      for (int i = 0; i < NHT; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float x = cga * S[i][r] + cbe * dsu[i][r];
          pin(x);
          S[i][r] = x;
        }
    }
    clk.tick(3);
    __syncthreads();  // B3: D tiles visible
    clk.tick(4);

    // ---------------- output block: token block R, column tiles 2 nh, 2 nh + 1
    if (!xkeep) {
#pragma unroll
      for (int kc = 0; kc < KP / 32; ++kc) {
        fxh[kc] = PX.hi8(16 * R + l16, 32 * kc + 8 * lg);
        fxl[kc] = PX.lo8(16 * R + l16, 32 * kc + 8 * lg);
      }
    }
    uint2 dh[4], dl[4];
#pragma unroll
    for (int P = 0; P < 4; ++P) {
      dh[P] = make_uint2(0u, 0u);
      dl[P] = make_uint2(0u, 0u);
      const bool live = REV ? (P >= R) : (P <= R);
      if (live) {
        const int Rc = REV ? 3 - R : R, Pc = REV ? 3 - P : P;
        const uint4 x = sDt[(Rc * (Rc + 1) / 2 + Pc) * 64 + lane];
        dh[P] = make_uint2(x.x, x.y);
        dl[P] = make_uint2(x.z, x.w);
      }
    }
    const int tok = 16 * R + l16;
    const size_t eo = (size_t)(row0 + t0) * H + hh;
    // (tokens past the chunk's valid rows are outside Ro's range)
    const rsrc_t Ro = chunk_rsrc((const uint16_t*)p.out, eo, nval, (int)rowV, V);
    const uint32_t oo = ((uint32_t)tok * rowV + vt * BV + 4 * lg) * ES;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int nn = 2 * nh + j;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kc = 0; kc < KP / 32; ++kc)
        acc = mma<true, true>(acc, tr_read8(PH.hi, PH.ld, 32 * kc, 16 * nn, lane),
                              tr_read8(PH.lo, PH.ld, 32 * kc, 16 * nn, lane), fxh[kc], fxl[kc]);
#pragma unroll
      for (int Pp = 0; Pp < 2; ++Pp) {
        const int P0 = 2 * Pp, P1 = 2 * Pp + 1;
        const bool live = REV ? (P1 >= R) : (P0 <= R);
        if (live) {
          const bf16x8 ah = tr_read44(PY.hi, PY.ld, 16 * P0, 16 * P1, 16 * nn, lane);
          acc = mma<false, true>(acc, ah, ah, cat44(dh[P0], dh[P1]), cat44(dl[P0], dl[P1]));
        }
      }
      const int v0 = vt * BV + 16 * nn + 4 * lg;
      if (VAR != 0 || p.acc_mode == 0) {
        Words<uint16_t>::st4(Ro, acc, v0 < V ? oo : kOOB, (uint32_t)(16 * nn * ES));
      } else {
        // channel slices: the fp32 sum of the slices' outputs
        const rsrc_t Ra = chunk_rsrc(p.acc32, eo, nval, (int)rowV, V);
        const uint32_t fo = (v0 < V) ? ((uint32_t)tok * rowV + v0) * 4u : kOOB;
        acc_slice_t<uint16_t>(Ro, Ra, acc, fo, v0 < V ? oo : kOOB, (uint32_t)(16 * nn * ES),
                              p.acc_mode);
      }
    }
  }

  if (NTs > 0) clk.tick(5);
  clk.finish(p.clocks, blockIdx.x * NW + wave);

  if (p.s_fin) {
    const rsrc_t Rsf = make_rsrc(p.s_fin + s_base, (long long)LDK * V * 4);
#pragma unroll
    for (int i = 0; i < NHT; ++i) bst128(Rsf, __builtin_bit_cast(uint4, S[i]), srun(i), 0);
  }
}

// Whether launch_gla_sweep routes a call to the pipelined kernel: bf16, per-channel gates,
// not the delta rule, no gate shift.  TOPS_SWEEP_SERIAL=1 in the environment keeps such calls
// on gla_sweep_kernel (the serial schedule, for A/B comparisons), except those that write
// fp16 checkpoints, which only this kernel does.
bool gla_pipe_eligible(const SweepParams& p) {
  if (p.gate_mode != kGateK || p.gshift) return false;
  if (p.ckpt16) return true;   // only this kernel writes fp16 checkpoints
  const char* e = getenv("TOPS_SWEEP_SERIAL");
  return !(e && e[0] == '1');
}

template <bool REV>
hipError_t launch_gla_pipe(const SweepParams& p, hipStream_t s) {
  const int kp = p.K <= 32 ? 32 : (p.K <= 64 ? 64 : 128);
  const bool plain = !p.acc_mode && !p.ldk;
  if (p.ckpt16 && (!plain || p.ckpt_par || !p.ckpt || !p.ckpt_scale)) return hipErrorInvalidValue;
  const int var = p.ckpt16 ? 1 : ((plain && !p.ckpt) ? 2 : 0);
  dim3 grid(p.NV * p.H * p.N);
#define TOPS_PIPE(KPV, VARV) hipLaunchKernelGGL((gla_pipe_kernel<KPV, REV, VARV>), grid, dim3(512), 0, s, p)
#define TOPS_PIPE_K(KPV) \
  if (var == 1) TOPS_PIPE(KPV, 1); else if (var == 2) TOPS_PIPE(KPV, 2); else TOPS_PIPE(KPV, 0)
  if (kp == 32) { TOPS_PIPE_K(32); }
  else if (kp == 64) { TOPS_PIPE_K(64); }
  else { TOPS_PIPE_K(128); }
#undef TOPS_PIPE_K
#undef TOPS_PIPE
  return hipGetLastError();
}

template hipError_t launch_gla_pipe<false>(const SweepParams&, hipStream_t);
template hipError_t launch_gla_pipe<true>(const SweepParams&, hipStream_t);

#ifdef TOPS_PHASE_CLOCKS
// Instrumented build only (libtops_pipe_clocks.so, pallas-kernel_amd/phase_clocks.py): one
// pipelined sweep over B fixed-length sequences of bf16 q, k, y (v forward, dO reverse) and
// fp32 per-channel log gates g [B, T, H, K]; out [B, T, H, V] bf16; fp16 checkpoints when
// ckpt16 / ckpt_scale are given (the training instance), none otherwise (inference); the
// phase clocks of every wave into clocks [B * H * ceil(V / 64), 8, 8].
extern "C" int tops_pipe_phase_clocks(const void* q, const void* k, const float* g, const void* y,
                                      void* out, void* ckpt16, float* ckpt_scale,
                                      unsigned long long* clocks, int B, int T, int H, int K,
                                      int V, int rev, float scale, void* stream) {
  if (!q || !k || !g || !y || !out || !clocks || (!ckpt16) != (!ckpt_scale) || B <= 0 || T <= 0 ||
      H <= 0 || K <= 0 || K > 128 || V <= 0 || K % 4 || V % 8)
    return (int)hipErrorInvalidValue;
  SweepParams p{};
  p.q = q; p.k = k; p.g = g; p.y = y; p.out = out;
  p.ckpt = (float*)ckpt16;
  p.ckpt16 = ckpt16 != nullptr;
  p.ckpt_scale = ckpt_scale;
  p.B = B; p.T = T; p.H = H; p.K = K; p.V = V; p.N = B; p.NV = (V + 63) / 64;
  p.scale = scale;
  p.gate_mode = kGateK;
  p.clocks = clocks;
  const hipError_t e = rev ? launch_gla_pipe<true>(p, (hipStream_t)stream)
                           : launch_gla_pipe<false>(p, (hipStream_t)stream);
  return (int)e;
}
#endif

}  // namespace tops
