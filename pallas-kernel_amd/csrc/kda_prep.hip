// KDA forward preparation for gfx950: the chunk-parallel WY step.
//
// Replaces the reference's kda_gate_chunk_cumsum (tops/ops/kda/gate.py:19-51) and the
// u / w / Akk^-1 part of kda_intra_chunk_fwd (tops/ops/kda/chunk_intra.py:28-165, K16),
// following the oracle tops/cpu/ops/kda/naive.py:121-313.  Per (chunk, head), with G the
// in-chunk inclusive cumsum of the natural-log gates in log2 units (2^G = e^Gn),
// Gm = G[last] / 2 and beta the per-token delta-rule rate:
//
//   Akk[i][j] = beta_i sum_d (k_id 2^(G_id - Gm_d)) (k_jd 2^(Gm_d - G_jd))   (i > j)
//   T         = (I + Akk)^-1
//   u = T (beta v),   w = T (beta 2^G k)
//
// The Akk product and the u / w products run on bf16 MFMA with hi/lo split operands.
// T is computed in fp32 in LDS: each wave inverts one 16 x 16 diagonal block by forward
// substitution, then the off-diagonal blocks follow level by level,
// T[I][J] = -T[I][I] sum_{J <= k < I} Akk[I][k] T[k][J].
// Outputs: u [B,T,H,V], w [B,T,H,K] (fp32, read by the state sweep) and, for the
// backward, T transposed per chunk [total,H,C,C] (row i holds column i of T).  The Akk and
// u / w products run in passes of 64 channels (columns) so the workgroup needs < 80 KB of
// LDS and two share a CU: one's serial triangular solve overlaps the other's products.
#include "kda.h"
#include "tops_common.h"
#include "tops_hip.h"

namespace tops {

template <typename TIn, int KP, int VP>
__global__ __launch_bounds__(256) void kda_prep_kernel(KdaPrepParams p) {
  constexpr int C = kChunk;
  constexpr int NQ = KP / 4, NSEG = 256 / NQ, RPT = C / NSEG;        // k / g staging
  constexpr int NQV = VP / 4, NSEGV = 256 / NQV, RPTV = C / NSEGV;   // v staging
  constexpr int ES = sizeof(TIn);
  constexpr int KH2 = KP < 64 ? KP : 64;   // channels per Akk / w pass
  constexpr int VH2 = VP < 64 ? VP : 64;   // columns per u pass
  constexpr int NKP = KP / KH2, NVP = VP / VH2;
  constexpr int NUW = NKP > NVP ? NKP : NVP;
  constexpr int LQ = KH2 + 8;  // row-major gated-k planes [C][LQ]
  constexpr int LT = C + 8;    // transposed planes [channel][LT]
  constexpr int LA = C + 4;    // fp32 [C][LA]
  static_assert(RPT == 2 || RPT == 4 || RPT == 8, "KP must be 32, 64 or 128");
  static_assert(RPTV == 2 || RPTV == 4 || RPTV == 8, "VP must be 32, 64 or 128");
  typedef Words<TIn> Wd;

  // Region R1: K1 | K2 (row-major, hi+lo, one channel pass) for the Akk product, then
  // BKt | BVt (transposed beta 2^G k and beta v, hi+lo, one pass) for the u / w products.
  // Passes of 64 channels / columns keep the workgroup under 80 KB: two per CU.
  constexpr int R1A = 4 * C * LQ;
  constexpr int R1B = 2 * KH2 * LT + 2 * VH2 * LT;
  constexpr int R1 = R1A > R1B ? R1A : R1B;
  __shared__ __attribute__((aligned(16))) uint16_t sR1[R1];
  __shared__ __attribute__((aligned(16))) float sA[C * LA];     // Akk (strictly lower)
  __shared__ __attribute__((aligned(16))) float sT[C * LA];     // T (unit lower)
  __shared__ __attribute__((aligned(16))) float sX[3 * 16 * 20];
  __shared__ __attribute__((aligned(16))) float sTot[NSEG * KP];
  __shared__ float sBeta[C];

  const Plane PK1{sR1, sR1 + C * LQ, LQ};
  const Plane PK2{sR1 + 2 * C * LQ, sR1 + 3 * C * LQ, LQ};
  const Plane PBK{sR1, sR1 + KH2 * LT, LT};
  const Plane PBV{sR1 + 2 * KH2 * LT, sR1 + 2 * KH2 * LT + VH2 * LT, LT};

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lg = lane >> 4;
  const int hh = blockIdx.x % p.H;
  const int gc = blockIdx.x / p.H;
  const int H = p.H, K = p.K, V = p.V;

  int c, L, row0;
  if (p.cu_seqlens) {
    const int n = p.chunk_map[gc];
    c = gc - p.chunk_offsets[n];
    row0 = p.cu_seqlens[n];
    L = p.cu_seqlens[n + 1] - row0;
  } else {
    const int nt = cdiv(p.T, C);
    const int n = gc / nt;
    c = gc % nt;
    row0 = n * p.T;
    L = p.T;
  }
  const int t0 = c * C;
  const int nval = min(C, L - t0);
  const size_t e0 = (size_t)(row0 + t0) * H + hh;
  const long long nrows = (long long)p.B * p.T * H;     // (token, head) rows of [B,T,H,.]
  const uint32_t rowK = (uint32_t)(H * K), rowV = (uint32_t)(H * V);
  const rsrc_t Rk = make_rsrc_rows((const TIn*)p.k, e0, nrows, K);
  const rsrc_t Rg = make_rsrc_rows(p.g, e0, nrows, K);
  const rsrc_t Rv = make_rsrc_rows((const TIn*)p.v, e0, nrows, V);
  const rsrc_t Rb = make_rsrc_rows(p.beta, e0, nrows, 1);

  // ---------------- loads: k / g rows r0.. (4 channels), v rows rv0.. (4 columns), beta
  // a 32-lane half-wave covers 8 channel quads x 4 row segments: the row-major K1 / K2 writes
  // and the transposed BKt writes then (nearly) avoid LDS bank conflicts
  constexpr int CQL = NQ < 8 ? NQ : 8, SGL = 32 / CQL, NCQH = NQ / CQL;
  const int hw = tid >> 5;
  const int cq = (lane & 31) % CQL + CQL * (hw % NCQH), seg = (lane & 31) / CQL + SGL * (hw / NCQH);
  const int c0 = 4 * cq, r0 = seg * RPT;
  const bool colok = c0 < K;
  const uint32_t offK = colok ? ((uint32_t)r0 * rowK + c0) * ES : kOOB;
  const uint32_t offG = colok ? ((uint32_t)r0 * rowK + c0) * 4u : kOOB;
  constexpr int CQLV = NQV < 8 ? NQV : 8, SGLV = 32 / CQLV, NCQHV = NQV / CQLV;
  const int cv = (lane & 31) % CQLV + CQLV * (hw % NCQHV), sv = (lane & 31) / CQLV + SGLV * (hw / NCQHV);
  const int vc0 = 4 * cv, rv0 = sv * RPTV;
  const uint32_t offV = vc0 < V ? ((uint32_t)rv0 * rowV + vc0) * ES : kOOB;
  typename Wd::W4 rk[RPT], rv[RPTV];
  uint4 rg[RPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const bool ok = r0 + i < nval;
    rk[i] = Wd::ld4(Rk, ok ? offK : kOOB, i * rowK * ES);
    rg[i] = bld128(Rg, ok ? offG : kOOB, i * rowK * 4);
  }
#pragma unroll
  for (int i = 0; i < RPTV; ++i) rv[i] = Wd::ld4(Rv, rv0 + i < nval ? offV : kOOB, i * rowV * ES);
  if (tid < C) sBeta[tid] = __uint_as_float(bld32(Rb, tid < nval ? (uint32_t)tid * H * 4u : kOOB, 0));
  for (int i = tid; i < C * LA; i += 256) sT[i] = 0.f;

  // ---------------- gate cumsum (log2 units): thread rows, then segment totals
  float G[RPT][4], kv[RPT][4];
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    float x[4];
    unpack4(rg[i], x);
    unpack4(rk[i], kv[i]);
#pragma unroll
    for (int j = 0; j < 4; ++j) G[i][j] = x[j] * kLog2e + (i > 0 ? G[i - 1][j] : 0.f);
  }
  *(float4*)(sTot + seg * KP + c0) = make_float4(G[RPT - 1][0], G[RPT - 1][1], G[RPT - 1][2], G[RPT - 1][3]);
  __syncthreads();
  float gm[4];
  {
    float pre[4] = {0.f, 0.f, 0.f, 0.f}, gam[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < NSEG; ++s) {
      const float4 t = *(const float4*)(sTot + s * KP + c0);
      if (s < seg) { pre[0] += t.x; pre[1] += t.y; pre[2] += t.z; pre[3] += t.w; }
      gam[0] += t.x; gam[1] += t.y; gam[2] += t.z; gam[3] += t.w;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) gm[j] = 0.5f * gam[j];
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
#pragma unroll
      for (int j = 0; j < 4; ++j) G[i][j] += pre[j];
    }
  }

  // ---------------- Akk: the 10 lower 16x16 tiles, dealt round-robin over the waves,
  // accumulated over channel passes of KH2
  f32x4 akk[3];
#pragma unroll
  for (int ti = 0; ti < 3; ++ti) akk[ti] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int hp = 0; hp < NKP; ++hp) {
    if (hp > 0) __syncthreads();  // the previous pass is done with K1 / K2
    if (c0 >= hp * KH2 && c0 < (hp + 1) * KH2) {
#pragma unroll
      for (int i = 0; i < RPT; ++i) {
        float x1[4], x2[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          x1[j] = kv[i][j] * fast_exp2(G[i][j] - gm[j]);
          x2[j] = kv[i][j] * fast_exp2(gm[j] - G[i][j]);
        }
        put_n<true, 4>(PK1, r0 + i, c0 - hp * KH2, x1);
        put_n<true, 4>(PK2, r0 + i, c0 - hp * KH2, x2);
      }
    }
    __syncthreads();  // K1 / K2 of the pass (and, first time, beta and the zeroed T) visible
#pragma unroll
    for (int ti = 0; ti < 3; ++ti) {
      const int t = wave + 4 * ti;
      if (t < 10) {
        const int I = t >= 6 ? 3 : (t >= 3 ? 2 : (t >= 1 ? 1 : 0));
        const int J = t - I * (I + 1) / 2;
#pragma unroll
        for (int kc = 0; kc < KH2 / 32; ++kc)
          akk[ti] = mma<true, true>(akk[ti], PK1.hi8(16 * I + l16, 32 * kc + 8 * lg), PK1.lo8(16 * I + l16, 32 * kc + 8 * lg),
                                    PK2.hi8(16 * J + l16, 32 * kc + 8 * lg), PK2.lo8(16 * J + l16, 32 * kc + 8 * lg));
      }
    }
  }
#pragma unroll
  for (int ti = 0; ti < 3; ++ti) {
    const int t = wave + 4 * ti;
    if (t < 10) {
      const int I = t >= 6 ? 3 : (t >= 3 ? 2 : (t >= 1 ? 1 : 0));
      const int J = t - I * (I + 1) / 2;
      const int j = 16 * J + l16;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * I + 4 * lg + r;
        sA[i * LA + j] = i > j ? sBeta[i] * akk[ti][r] : 0.f;
      }
    }
  }
  __syncthreads();  // Akk complete; K1 / K2 are dead

  // ---------------- BKt = (beta 2^G k)^T, BVt = (beta v)^T of u / w pass up into region R1
  auto write_bkbv = [&](int up) {
    if (up < NKP && c0 >= up * KH2 && c0 < (up + 1) * KH2) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float x[RPT];
#pragma unroll
        for (int i = 0; i < RPT; ++i) x[i] = sBeta[r0 + i] * fast_exp2(G[i][j]) * kv[i][j];
        put_n<true, RPT>(PBK, c0 - up * KH2 + j, r0, x);
      }
    }
    if (up < NVP && vc0 >= up * VH2 && vc0 < (up + 1) * VH2) {
      float vv[RPTV][4];
#pragma unroll
      for (int i = 0; i < RPTV; ++i) unpack4(rv[i], vv[i]);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float x[RPTV];
#pragma unroll
        for (int i = 0; i < RPTV; ++i) x[i] = sBeta[rv0 + i] * vv[i][j];
        put_n<true, RPTV>(PBV, vc0 - up * VH2 + j, rv0, x);
      }
    }
  };
  write_bkbv(0);

  // ---------------- diagonal blocks of T: wave b inverts I + Akk[b][b] (lane = column)
  {
    const int b = wave, cc = l16;
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float* arow = sA + (16 * b + i) * LA + 16 * b;
      float s = (i == cc) ? 1.f : 0.f;
#pragma unroll
      for (int j = 0; j < i; ++j) s -= arow[j] * x[j];
      x[i] = s;
    }
    if (lg == 0) {
#pragma unroll
      for (int i = 0; i < 16; ++i) sT[(16 * b + i) * LA + 16 * b + cc] = x[i];
    }
  }
  __syncthreads();

  // ---------------- off-diagonal blocks, level d = I - J: X = sum_k Akk[I][k] T[k][J], T[I][J] = -T[I][I] X
#pragma unroll
  for (int d = 1; d < 4; ++d) {
    const int ntask = 64 * (4 - d);
    const int bi = tid >> 6, I = d + bi, J = bi;
    const int i = (tid & 63) >> 2, q = tid & 3;
    if (tid < ntask) {
      float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
      for (int kb = J; kb < I; ++kb) {
        const float* arow = sA + (16 * I + i) * LA + 16 * kb;
#pragma unroll
        for (int m = 0; m < 16; ++m) {
          const float a = arow[m];
          const float4 t = *(const float4*)(sT + (16 * kb + m) * LA + 16 * J + 4 * q);
          acc.x += a * t.x; acc.y += a * t.y; acc.z += a * t.z; acc.w += a * t.w;
        }
      }
      *(float4*)(sX + (bi * 16 + i) * 20 + 4 * q) = acc;
    }
    __syncthreads();
    if (tid < ntask) {
      float4 y = make_float4(0.f, 0.f, 0.f, 0.f);
      const float* trow = sT + (16 * I + i) * LA + 16 * I;
#pragma unroll
      for (int m = 0; m < 16; ++m) {
        const float t = trow[m];
        const float4 x4 = *(const float4*)(sX + (bi * 16 + m) * 20 + 4 * q);
        y.x += t * x4.x; y.y += t * x4.y; y.z += t * x4.z; y.w += t * x4.w;
      }
      *(float4*)(sT + (16 * I + i) * LA + 16 * J + 4 * q) = make_float4(-y.x, -y.y, -y.z, -y.w);
    }
    __syncthreads();
  }

  // ---------------- u = T (beta v), w = T (beta 2^G k): wave R owns rows 16R..16R+15,
  // computed transposed (lane holds 4 consecutive columns of token 16R + l16)
  {
    const int R = wave;
    const int nkc = R >= 2 ? 2 : 1;       // T[i][j] = 0 for j > i
    bf16x8 th[2], tl[2];
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
      const float* trow = sT + (16 * R + l16) * LA + 32 * kc + 8 * lg;
      const float4 a = *(const float4*)trow, b = *(const float4*)(trow + 4);
      uint32_t h[4], l[4];
      split_bf16x2(a.x, a.y, h[0], l[0]);
      split_bf16x2(a.z, a.w, h[1], l[1]);
      split_bf16x2(b.x, b.y, h[2], l[2]);
      split_bf16x2(b.z, b.w, h[3], l[3]);
      th[kc] = __builtin_bit_cast(bf16x8, make_uint4(h[0], h[1], h[2], h[3]));
      tl[kc] = __builtin_bit_cast(bf16x8, make_uint4(l[0], l[1], l[2], l[3]));
    }
    const int tok = 16 * R + l16;
    const bool tok_ok = tok < nval;
    const rsrc_t Ru = make_rsrc_rows(p.u, e0, nrows, V);
    const rsrc_t Rw = make_rsrc_rows(p.w, e0, nrows, K);
#pragma unroll
    for (int up = 0; up < NUW; ++up) {
      if (up > 0) {
        __syncthreads();  // the previous pass is done with BKt / BVt
        write_bkbv(up);
        __syncthreads();
      }
      if (up < NVP) {
#pragma unroll
        for (int vb = 0; vb < VH2 / 16; ++vb) {
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int kc = 0; kc < 2; ++kc)
            if (kc < nkc)
              acc = mma<true, true>(acc, PBV.hi8(16 * vb + l16, 32 * kc + 8 * lg),
                                    PBV.lo8(16 * vb + l16, 32 * kc + 8 * lg), th[kc], tl[kc]);
          const int col = up * VH2 + 16 * vb + 4 * lg;
          bst128(Ru, make_uint4(__float_as_uint(acc[0]), __float_as_uint(acc[1]), __float_as_uint(acc[2]),
                                __float_as_uint(acc[3])),
                 (tok_ok && col < V) ? ((uint32_t)tok * rowV + col) * 4u : kOOB, 0);
        }
      }
      if (up < NKP) {
#pragma unroll
        for (int kb = 0; kb < KH2 / 16; ++kb) {
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int kc = 0; kc < 2; ++kc)
            if (kc < nkc)
              acc = mma<true, true>(acc, PBK.hi8(16 * kb + l16, 32 * kc + 8 * lg),
                                    PBK.lo8(16 * kb + l16, 32 * kc + 8 * lg), th[kc], tl[kc]);
          const int col = up * KH2 + 16 * kb + 4 * lg;
          bst128(Rw, make_uint4(__float_as_uint(acc[0]), __float_as_uint(acc[1]), __float_as_uint(acc[2]),
                                __float_as_uint(acc[3])),
                 (tok_ok && col < K) ? ((uint32_t)tok * rowK + col) * 4u : kOOB, 0);
        }
      }
    }
  }

  // ---------------- T transposed: thread (row i, 16 columns)
  if (p.tt) {
    const rsrc_t Rt = make_rsrc(p.tt + ((size_t)gc * H + hh) * C * C, (long long)C * C * 4);
    const int i = tid >> 2, q = tid & 3;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int j0 = 16 * q + 4 * e;
      bst128(Rt, make_uint4(__float_as_uint(sT[(j0 + 0) * LA + i]), __float_as_uint(sT[(j0 + 1) * LA + i]),
                            __float_as_uint(sT[(j0 + 2) * LA + i]), __float_as_uint(sT[(j0 + 3) * LA + i])),
             ((uint32_t)i * C + j0) * 4u, 0);
    }
  }
}

template <typename TIn>
hipError_t launch_kda_prep(const KdaPrepParams& p, hipStream_t s) {
  const int kp = p.K <= 32 ? 32 : (p.K <= 64 ? 64 : 128);
  const int vp = p.V <= 32 ? 32 : (p.V <= 64 ? 64 : 128);
  dim3 grid(p.total * p.H), block(256);
#define TOPS_KPREP(KPV, VPV) \
  if (kp == KPV && vp == VPV) { hipLaunchKernelGGL((kda_prep_kernel<TIn, KPV, VPV>), grid, block, 0, s, p); return hipGetLastError(); }
  TOPS_KPREP(32, 32) TOPS_KPREP(32, 64) TOPS_KPREP(32, 128)
  TOPS_KPREP(64, 32) TOPS_KPREP(64, 64) TOPS_KPREP(64, 128)
  TOPS_KPREP(128, 32) TOPS_KPREP(128, 64) TOPS_KPREP(128, 128)
#undef TOPS_KPREP
  return hipErrorInvalidValue;
}

template hipError_t launch_kda_prep<uint16_t>(const KdaPrepParams&, hipStream_t);
template hipError_t launch_kda_prep<float>(const KdaPrepParams&, hipStream_t);

}  // namespace tops
