// GLA chunked backward for gfx950.
//
// Replaces the reference's K8 (chunk_bwd_dh, tops/ops/common/chunk_h.py:685-878) and the
// fused K4 (chunk_gla_bwd_fused_kernel, tops/ops/gla/chunk.py:1447-1581), following the
// oracle tops/cpu/ops/gla/chunk.py:277-640.  Two kernels:
//
// 1. gla_bwd_rev_kernel -- reverse sweep, one workgroup per (sequence, head, 64-wide
//    V tile), the state gradient dh (K x 64 fp32) in MFMA accumulators.  Per chunk c
//    (last to first), with dh = dL/d(state after chunk c):
//        dh_ckpt[c] = dh
//        dv   = k~ (2^(Gamma-Gm) dh) + A^T do          (A = scale * tril(q~ k~^T))
//        dh   = 2^Gamma dh + scale 2^Gm (q~^T do)
//    and dh0 = dh at the end.  The same structure as the forward with q<->do roles.
// 2. gla_bwd_main_kernel -- chunk-parallel, one workgroup per (chunk, head), from the
//    forward state checkpoint h_c and dh_c:
//        dA   = scale * tril(do v^T)
//        dq   = 2^(G-Gm)  (dA k~          + do (scale 2^Gm h_c)^T)
//        dk   = 2^(Gm-G)  (dA^T q~        + v (2^(Gamma-Gm) dh_c)^T)
//        dg   = revcumsum_t(q dq - k dk) + 2^Gamma sum_v(h_c dh_c) + sum_t k dk_inter
//    (the gate gradient of tops/cpu/ops/gla/chunk.py:396-466).
#include <stdio.h>

#include "tops_common.h"
#include "tops_hip.h"

namespace tops {

struct GlaBwdParams {
  const void* q;
  const void* k;
  const void* v;
  const float* g;
  const void* dout;
  const float* dht;
  const float* hs;      // [total, H, K, V] state before each chunk
  float* dhs;           // [total, H, K, V] dL/d(state after each chunk)
  void* dq;
  void* dk;
  void* dv;
  float* dg;
  float* dh0;
  const int* cu_seqlens;
  const int* chunk_offsets;
  const int* chunk_map;
  int total, B, T, H, K, V, N, NV;
  float scale;
};

template <typename TIn, int KP>
__global__ __launch_bounds__(256) void gla_bwd_rev_kernel(GlaBwdParams p) {
  constexpr int C = kChunk, BV = 64;
  constexpr int NCP = KP / 2, NRS = 256 / NCP, RPS = C / NRS;
  constexpr bool SIN = !In<TIn>::kExactBf16;
  constexpr int LQ = KP + 8, LT = C + 8, LH = KP + 8;
  constexpr int NHT = (KP / 16) * (BV / 16) / 4;

  __shared__ __attribute__((aligned(16))) uint16_t sQ[2 * C * LQ];
  __shared__ __attribute__((aligned(16))) uint16_t sK[2 * C * LQ];
  __shared__ __attribute__((aligned(16))) uint16_t sQT[2 * KP * LT];
  __shared__ __attribute__((aligned(16))) uint16_t sDT[(SIN ? 2 : 1) * BV * LT];
  __shared__ __attribute__((aligned(16))) uint16_t sHT[2 * BV * LH];
  __shared__ float sTot[NRS * KP];
  __shared__ float sGam[KP];
  __shared__ float sGm[KP];

  const Plane Pq{sQ, sQ + C * LQ, LQ};
  const Plane Pk{sK, sK + C * LQ, LQ};
  const Plane Pqt{sQT, sQT + KP * LT, LT};
  const Plane Pdt{sDT, SIN ? sDT + BV * LT : sDT, LT};
  const Plane Pht{sHT, sHT + BV * LH, LH};

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l16 = lane & 15, lg = lane >> 4;
  const int wg = xcd_remap(blockIdx.x, gridDim.x, p.NV);
  const int vt = wg % p.NV;
  const int hh = (wg / p.NV) % p.H;
  const int n = wg / (p.NV * p.H);
  const int H = p.H, K = p.K, V = p.V;

  int L, row0, cbase;
  if (p.cu_seqlens) {
    row0 = p.cu_seqlens[n];
    L = p.cu_seqlens[n + 1] - row0;
    cbase = p.chunk_offsets[n];
  } else {
    row0 = n * p.T;
    L = p.T;
    cbase = n * cdiv(p.T, C);
  }
  const int NTs = cdiv(L, C);
  const TIn* __restrict__ q = (const TIn*)p.q;
  const TIn* __restrict__ kk = (const TIn*)p.k;
  const TIn* __restrict__ dout = (const TIn*)p.dout;
  const float* __restrict__ g = p.g;
  TIn* __restrict__ dv = (TIn*)p.dv;

  const int cp = tid % NCP, rs = tid / NCP;
  const int col = 2 * cp;
  const bool col_ok = col < K;
  const int vcol = tid & 63, vrs = tid >> 6;
  const int vg = vt * BV + vcol;
  const bool vcol_ok = vg < V;

  f32x4 dh[NHT];
#pragma unroll
  for (int i = 0; i < NHT; ++i) {
    const int t = wave + 4 * i, m = t / (BV / 16), nn = t % (BV / 16);
    const int vv = vt * BV + 16 * nn + l16;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int kr = 16 * m + 4 * lg + r;
      float x = 0.f;
      if (p.dht && kr < K && vv < V) x = p.dht[((size_t)(n * H + hh) * K + kr) * V + vv];
      dh[i][r] = x;
    }
  }

  for (int c = NTs - 1; c >= 0; --c) {
    const int t0 = c * C;
    const int nval = min(C, L - t0);
    float qa[RPS][2], ka[RPS][2], ga[RPS][2], da[16];
#pragma unroll
    for (int i = 0; i < RPS; ++i) {
      const int r = rs * RPS + i;
      if (r < nval && col_ok) {
        const size_t off = ((size_t)(row0 + t0 + r) * H + hh) * K + col;
        In<TIn>::ld2(q + off, qa[i][0], qa[i][1]);
        In<TIn>::ld2(kk + off, ka[i][0], ka[i][1]);
        float2 gg = *(const float2*)(g + off);
        ga[i][0] = gg.x * kLog2e;
        ga[i][1] = gg.y * kLog2e;
      } else {
        qa[i][0] = qa[i][1] = ka[i][0] = ka[i][1] = ga[i][0] = ga[i][1] = 0.f;
      }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = vrs * 16 + i;
      da[i] = (r < nval && vcol_ok)
                  ? In<TIn>::ld(dout + ((size_t)(row0 + t0 + r) * H + hh) * V + vg) : 0.f;
    }
#pragma unroll
    for (int i = 1; i < RPS; ++i) {
      ga[i][0] += ga[i - 1][0];
      ga[i][1] += ga[i - 1][1];
    }
    sTot[rs * KP + col] = ga[RPS - 1][0];
    sTot[rs * KP + col + 1] = ga[RPS - 1][1];
    __syncthreads();  // B1
    float pre0 = 0.f, pre1 = 0.f, gam0 = 0.f, gam1 = 0.f;
#pragma unroll
    for (int s = 0; s < NRS; ++s) {
      const float a = sTot[s * KP + col], b = sTot[s * KP + col + 1];
      if (s < rs) { pre0 += a; pre1 += b; }
      gam0 += a;
      gam1 += b;
    }
    const float gm0 = 0.5f * gam0, gm1 = 0.5f * gam1;
    if (rs == 0) {
      sGam[col] = gam0; sGam[col + 1] = gam1;
      sGm[col] = gm0;   sGm[col + 1] = gm1;
    }
    float qt0[RPS], qt1[RPS];
#pragma unroll
    for (int i = 0; i < RPS; ++i) {
      const int r = rs * RPS + i;
      const float G0 = ga[i][0] + pre0, G1 = ga[i][1] + pre1;
      qt0[i] = qa[i][0] * fast_exp2(G0 - gm0);
      qt1[i] = qa[i][1] * fast_exp2(G1 - gm1);
      Pq.put2<true>(r, col, qt0[i], qt1[i]);
      Pk.put2<true>(r, col, ka[i][0] * fast_exp2(gm0 - G0), ka[i][1] * fast_exp2(gm1 - G1));
    }
    Pqt.put_run<true, RPS>(col, rs * RPS, qt0);
    Pqt.put_run<true, RPS>(col + 1, rs * RPS, qt1);
    Pdt.put_run<SIN, 16>(vcol, vrs * 16, da);
    __syncthreads();  // B2: sGm / sGam visible
#pragma unroll
    for (int i = 0; i < NHT; ++i) {
      const int t = wave + 4 * i, m = t / (BV / 16), nn = t % (BV / 16);
      const int kr = 16 * m + 4 * lg;
      const int vv = vt * BV + 16 * nn + l16;
      float* dst = p.dhs + ((size_t)(cbase + c) * H + hh) * K * V;
      float x[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        x[r] = fast_exp2(sGam[kr + r] - sGm[kr + r]) * dh[i][r];
        if (kr + r < K && vv < V) dst[(size_t)(kr + r) * V + vv] = dh[i][r];
      }
      Pht.put_run<true, 4>(16 * nn + l16, kr, x);
    }
    __syncthreads();  // B3

    // ---------------- dv rows 16*wave .. +15
    {
      const int Jw = wave;
      f32x4 acc[BV / 16];
#pragma unroll
      for (int nn = 0; nn < BV / 16; ++nn) acc[nn] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kc = 0; kc < KP / 32; ++kc) {
        const bf16x8 ah = Pk.hi8(16 * Jw + l16, 32 * kc + 8 * lg);
        const bf16x8 al = Pk.lo8(16 * Jw + l16, 32 * kc + 8 * lg);
#pragma unroll
        for (int nn = 0; nn < BV / 16; ++nn) {
          const bf16x8 bh = Pht.hi8(16 * nn + l16, 32 * kc + 8 * lg);
          const bf16x8 bl = Pht.lo8(16 * nn + l16, 32 * kc + 8 * lg);
          acc[nn] = mma<true, true>(acc[nn], ah, al, bh, bl);
        }
      }
      // A tiles (I, Jw) for I >= Jw: lane holds A[16I+4lg+r][16Jw+l16]
      uint2 aah[4], aal[4];
#pragma unroll
      for (int I = 0; I < 4; ++I) {
        aah[I] = make_uint2(0u, 0u);
        aal[I] = make_uint2(0u, 0u);
        if (I >= Jw) {
          f32x4 t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int kc = 0; kc < KP / 32; ++kc) {
            const bf16x8 ah = Pq.hi8(16 * I + l16, 32 * kc + 8 * lg);
            const bf16x8 al = Pq.lo8(16 * I + l16, 32 * kc + 8 * lg);
            const bf16x8 bh = Pk.hi8(16 * Jw + l16, 32 * kc + 8 * lg);
            const bf16x8 bl = Pk.lo8(16 * Jw + l16, 32 * kc + 8 * lg);
            t = mma<true, true>(t, ah, al, bh, bl);
          }
          const int j = 16 * Jw + l16;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int i = 16 * I + 4 * lg + r;
            t[r] = (j <= i) ? t[r] * p.scale : 0.f;
          }
          acc_to_bf16x4(t, aah[I], aal[I]);
        }
      }
      // dv += A^T do (contraction over i)
#pragma unroll
      for (int Ip = 0; Ip < 2; ++Ip) {
        const int I0 = 2 * Ip, I1 = 2 * Ip + 1;
        if (I1 >= Jw) {
          const bf16x8 ah = cat44(aah[I0], aah[I1]);
          const bf16x8 al = cat44(aal[I0], aal[I1]);
#pragma unroll
          for (int nn = 0; nn < BV / 16; ++nn) {
            const bf16x8 bh = Pdt.hi44(16 * nn + l16, 16 * I0 + 4 * lg, 16 * I1 + 4 * lg);
            bf16x8 bl = bh;
            if constexpr (SIN) bl = Pdt.lo44(16 * nn + l16, 16 * I0 + 4 * lg, 16 * I1 + 4 * lg);
            acc[nn] = mma<true, SIN>(acc[nn], ah, al, bh, bl);
          }
        }
      }
#pragma unroll
      for (int nn = 0; nn < BV / 16; ++nn) {
        const int vv = vt * BV + 16 * nn + l16;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int j = 16 * Jw + 4 * lg + r;
          if (j < nval && vv < V) In<TIn>::st(dv + ((size_t)(row0 + t0 + j) * H + hh) * V + vv, acc[nn][r]);
        }
      }
    }
    // ---------------- dh update
#pragma unroll
    for (int i = 0; i < NHT; ++i) {
      const int t = wave + 4 * i, m = t / (BV / 16), nn = t % (BV / 16);
      f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kc = 0; kc < C / 32; ++kc) {
        const bf16x8 ah = Pqt.hi8(16 * m + l16, 32 * kc + 8 * lg);
        const bf16x8 al = Pqt.lo8(16 * m + l16, 32 * kc + 8 * lg);
        const bf16x8 bh = Pdt.hi8(16 * nn + l16, 32 * kc + 8 * lg);
        bf16x8 bl = bh;
        if constexpr (SIN) bl = Pdt.lo8(16 * nn + l16, 32 * kc + 8 * lg);
        d = mma<true, SIN>(d, ah, al, bh, bl);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int kr = 16 * m + 4 * lg + r;
        dh[i][r] = fast_exp2(sGam[kr]) * dh[i][r] + p.scale * fast_exp2(sGm[kr]) * d[r];
      }
    }
  }

  if (p.dh0) {
#pragma unroll
    for (int i = 0; i < NHT; ++i) {
      const int t = wave + 4 * i, m = t / (BV / 16), nn = t % (BV / 16);
      const int vv = vt * BV + 16 * nn + l16;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int kr = 16 * m + 4 * lg + r;
        if (kr < K && vv < V) p.dh0[((size_t)(n * H + hh) * K + kr) * V + vv] = dh[i][r];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// chunk-parallel dq / dk / dg
// ---------------------------------------------------------------------------
template <typename TIn, int KP, int VP>
__global__ __launch_bounds__(256) void gla_bwd_main_kernel(GlaBwdParams p) {
  constexpr int C = kChunk;
  constexpr int NCP = KP / 2, NRS = 256 / NCP, RPS = C / NRS;      // [C][KP] staging
  constexpr int VCP = VP / 2, VRS = 256 / VCP, VRPS = C / VRS;     // [C][VP] staging
  constexpr bool SIN = !In<TIn>::kExactBf16;
  constexpr int NPL = SIN ? 2 : 1;
  constexpr int LV = VP + 8;               // V / DO planes [C][VP]
  constexpr int LT = C + 8;                // Q~^T / K~^T planes [KP][C]
  constexpr int VH = VP < 64 ? VP : 64;    // state columns staged per pass
  constexpr int NVH = VP / VH;
  constexpr int LS = VH + 8;               // HP / DHP planes [KP][VH]
  constexpr int KT = KP / 16;
  constexpr int LX = KP + 4;               // fp32 [C][KP] arrays of the dg phase

  constexpr int kRegA = 2 * NPL * C * LV * 2;                   // V, DO
  constexpr int kRegB1 = 2 * 2 * KP * LT * 2;                   // Q~^T, K~^T
  constexpr int kRegB2 = 2 * 2 * KP * LS * 2;                   // HP, DHP
  constexpr int kRegB = kRegB1 > kRegB2 ? kRegB1 : kRegB2;
  constexpr int kDg = 3 * C * LX * 4;                           // X, Y, Z
  constexpr int kMain = (kRegA + kRegB) > kDg ? (kRegA + kRegB) : kDg;
  __shared__ __attribute__((aligned(16))) unsigned char smem[kMain];
  __shared__ float sTot[NRS * KP];
  __shared__ float sZk[NRS * KP];
  __shared__ float sGam[KP];
  __shared__ float sGm[KP];
  __shared__ float sB[KP];

  uint16_t* regA = (uint16_t*)smem;
  uint16_t* regB = (uint16_t*)(smem + kRegA);
  const Plane Pv{regA, SIN ? regA + C * LV : regA, LV};
  const Plane Pd{regA + NPL * C * LV, SIN ? regA + NPL * C * LV + C * LV : regA + NPL * C * LV, LV};
  const Plane Pqt{regB, regB + KP * LT, LT};
  const Plane Pkt{regB + 2 * KP * LT, regB + 3 * KP * LT, LT};
  const Plane Php{regB, regB + KP * LS, LS};
  const Plane Pdhp{regB + 2 * KP * LS, regB + 3 * KP * LS, LS};
  float* sX = (float*)smem;
  float* sY = sX + C * LX;
  float* sZ = sY + C * LX;

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l16 = lane & 15, lg = lane >> 4;
  const int hh = blockIdx.x % p.H;
  const int gc = blockIdx.x / p.H;
  const int H = p.H, K = p.K, V = p.V;

  int n, c, L, row0;
  if (p.cu_seqlens) {
    n = p.chunk_map[gc];
    c = gc - p.chunk_offsets[n];
    row0 = p.cu_seqlens[n];
    L = p.cu_seqlens[n + 1] - row0;
  } else {
    const int nt = cdiv(p.T, C);
    n = gc / nt;
    c = gc % nt;
    row0 = n * p.T;
    L = p.T;
  }
  const int t0 = c * C;
  const int nval = min(C, L - t0);
  const TIn* __restrict__ q = (const TIn*)p.q;
  const TIn* __restrict__ kk = (const TIn*)p.k;
  const TIn* __restrict__ v = (const TIn*)p.v;
  const TIn* __restrict__ dout = (const TIn*)p.dout;
  const float* __restrict__ g = p.g;

  // ---------------- phase 0: gates, gated q/k (transposed), v, do
  const int cp = tid % NCP, rs = tid / NCP;
  const int col = 2 * cp;
  const bool col_ok = col < K;
  float qa[RPS][2], ka[RPS][2], ga[RPS][2];
#pragma unroll
  for (int i = 0; i < RPS; ++i) {
    const int r = rs * RPS + i;
    if (r < nval && col_ok) {
      const size_t off = ((size_t)(row0 + t0 + r) * H + hh) * K + col;
      In<TIn>::ld2(q + off, qa[i][0], qa[i][1]);
      In<TIn>::ld2(kk + off, ka[i][0], ka[i][1]);
      float2 gg = *(const float2*)(g + off);
      ga[i][0] = gg.x * kLog2e;
      ga[i][1] = gg.y * kLog2e;
    } else {
      qa[i][0] = qa[i][1] = ka[i][0] = ka[i][1] = ga[i][0] = ga[i][1] = 0.f;
    }
  }
  {
    const int vcp = tid % VCP, vrs = tid / VCP, vc = 2 * vcp;
#pragma unroll
    for (int i = 0; i < VRPS; ++i) {
      const int r = vrs * VRPS + i;
      float a0 = 0.f, a1 = 0.f, b0 = 0.f, b1 = 0.f;
      if (r < nval && vc < V) {
        const size_t off = ((size_t)(row0 + t0 + r) * H + hh) * V + vc;
        In<TIn>::ld2(v + off, a0, a1);
        In<TIn>::ld2(dout + off, b0, b1);
      }
      Pv.put2<SIN>(r, vc, a0, a1);
      Pd.put2<SIN>(r, vc, b0, b1);
    }
  }
#pragma unroll
  for (int i = 1; i < RPS; ++i) {
    ga[i][0] += ga[i - 1][0];
    ga[i][1] += ga[i - 1][1];
  }
  sTot[rs * KP + col] = ga[RPS - 1][0];
  sTot[rs * KP + col + 1] = ga[RPS - 1][1];
  __syncthreads();
  float gam0 = 0.f, gam1 = 0.f;
  {
    float pre0 = 0.f, pre1 = 0.f;
#pragma unroll
    for (int s = 0; s < NRS; ++s) {
      const float a = sTot[s * KP + col], b = sTot[s * KP + col + 1];
      if (s < rs) { pre0 += a; pre1 += b; }
      gam0 += a;
      gam1 += b;
    }
#pragma unroll
    for (int i = 0; i < RPS; ++i) {
      ga[i][0] += pre0;
      ga[i][1] += pre1;
    }
  }
  const float gm0 = 0.5f * gam0, gm1 = 0.5f * gam1;
  if (rs == 0) {
    sGam[col] = gam0; sGam[col + 1] = gam1;
    sGm[col] = gm0;   sGm[col + 1] = gm1;
  }
  {
    float qt0[RPS], qt1[RPS], kt0[RPS], kt1[RPS];
#pragma unroll
    for (int i = 0; i < RPS; ++i) {
      qt0[i] = qa[i][0] * fast_exp2(ga[i][0] - gm0);
      qt1[i] = qa[i][1] * fast_exp2(ga[i][1] - gm1);
      kt0[i] = ka[i][0] * fast_exp2(gm0 - ga[i][0]);
      kt1[i] = ka[i][1] * fast_exp2(gm1 - ga[i][1]);
    }
    Pqt.put_run<true, RPS>(col, rs * RPS, qt0);
    Pqt.put_run<true, RPS>(col + 1, rs * RPS, qt1);
    Pkt.put_run<true, RPS>(col, rs * RPS, kt0);
    Pkt.put_run<true, RPS>(col + 1, rs * RPS, kt1);
  }
  __syncthreads();

  // ---------------- phase 1: dA tiles and intra-chunk dq / dk
  const int W = wave;
  f32x4 X[KT], Y[KT], Z[KT];
#pragma unroll
  for (int t = 0; t < KT; ++t) {
    X[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    Y[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    Z[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  {
    // dA^T tiles (J, W), J <= W: lane holds dA[16W+l16][16J+4lg+r]
    uint2 dth[4], dtl[4];
    // dA tiles (I, W), I >= W: lane holds dA[16I+4lg+r][16W+l16]
    uint2 dah[4], dal[4];
#pragma unroll
    for (int J = 0; J < 4; ++J) {
      dth[J] = dtl[J] = dah[J] = dal[J] = make_uint2(0u, 0u);
      if (J <= W) {
        f32x4 t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int vc = 0; vc < VP / 32; ++vc) {
          const bf16x8 ah = Pv.hi8(16 * J + l16, 32 * vc + 8 * lg);
          const bf16x8 bh = Pd.hi8(16 * W + l16, 32 * vc + 8 * lg);
          bf16x8 al = ah, bl = bh;
          if constexpr (SIN) {
            al = Pv.lo8(16 * J + l16, 32 * vc + 8 * lg);
            bl = Pd.lo8(16 * W + l16, 32 * vc + 8 * lg);
          }
          t = mma<SIN, SIN>(t, ah, al, bh, bl);
        }
        const int i = 16 * W + l16;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int j = 16 * J + 4 * lg + r;
          t[r] = (j <= i) ? t[r] * p.scale : 0.f;
        }
        acc_to_bf16x4(t, dth[J], dtl[J]);
      }
      const int I = J;
      if (I >= W) {
        f32x4 t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int vc = 0; vc < VP / 32; ++vc) {
          const bf16x8 ah = Pd.hi8(16 * I + l16, 32 * vc + 8 * lg);
          const bf16x8 bh = Pv.hi8(16 * W + l16, 32 * vc + 8 * lg);
          bf16x8 al = ah, bl = bh;
          if constexpr (SIN) {
            al = Pd.lo8(16 * I + l16, 32 * vc + 8 * lg);
            bl = Pv.lo8(16 * W + l16, 32 * vc + 8 * lg);
          }
          t = mma<SIN, SIN>(t, ah, al, bh, bl);
        }
        const int j = 16 * W + l16;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = 16 * I + 4 * lg + r;
          t[r] = (j <= i) ? t[r] * p.scale : 0.f;
        }
        acc_to_bf16x4(t, dah[I], dal[I]);
      }
    }
    // X = dA k~ (rows 16W..): contraction over j
#pragma unroll
    for (int Jp = 0; Jp < 2; ++Jp) {
      const int J0 = 2 * Jp, J1 = 2 * Jp + 1;
      if (J0 <= W) {
        const bf16x8 ah = cat44(dth[J0], dth[J1]);
        const bf16x8 al = cat44(dtl[J0], dtl[J1]);
#pragma unroll
        for (int t = 0; t < KT; ++t) {
          const bf16x8 bh = Pkt.hi44(16 * t + l16, 16 * J0 + 4 * lg, 16 * J1 + 4 * lg);
          const bf16x8 bl = Pkt.lo44(16 * t + l16, 16 * J0 + 4 * lg, 16 * J1 + 4 * lg);
          X[t] = mma<true, true>(X[t], ah, al, bh, bl);
        }
      }
    }
    // Y = dA^T q~ (rows 16W..): contraction over i
#pragma unroll
    for (int Ip = 0; Ip < 2; ++Ip) {
      const int I0 = 2 * Ip, I1 = 2 * Ip + 1;
      if (I1 >= W) {
        const bf16x8 ah = cat44(dah[I0], dah[I1]);
        const bf16x8 al = cat44(dal[I0], dal[I1]);
#pragma unroll
        for (int t = 0; t < KT; ++t) {
          const bf16x8 bh = Pqt.hi44(16 * t + l16, 16 * I0 + 4 * lg, 16 * I1 + 4 * lg);
          const bf16x8 bl = Pqt.lo44(16 * t + l16, 16 * I0 + 4 * lg, 16 * I1 + 4 * lg);
          Y[t] = mma<true, true>(Y[t], ah, al, bh, bl);
        }
      }
    }
  }

  // ---------------- phase 2: inter-chunk terms from the state checkpoints
  const float* __restrict__ hsrc = p.hs + ((size_t)gc * H + hh) * K * V;
  const float* __restrict__ dsrc = p.dhs + ((size_t)gc * H + hh) * K * V;
  constexpr int TPR = VH / 4;             // threads per state row (float4 each)
  constexpr int RPP = 256 / TPR;          // rows per pass
  constexpr int NRP = (KP + RPP - 1) / RPP;
  float bpart[NRP];
#pragma unroll
  for (int i = 0; i < NRP; ++i) bpart[i] = 0.f;
  const int sc4 = tid % TPR, sr = tid / TPR;
#pragma unroll
  for (int ph = 0; ph < NVH; ++ph) {
    __syncthreads();  // previous users of region B are done
#pragma unroll
    for (int i = 0; i < NRP; ++i) {
      const int kr = sr + RPP * i;
      if (kr < KP) {
        const int vv = ph * VH + 4 * sc4;
        float4 hv = make_float4(0.f, 0.f, 0.f, 0.f), dv4 = hv;
        if (kr < K && vv < V) {
          hv = *(const float4*)(hsrc + (size_t)kr * V + vv);
          dv4 = *(const float4*)(dsrc + (size_t)kr * V + vv);
        }
        bpart[i] += hv.x * dv4.x + hv.y * dv4.y + hv.z * dv4.z + hv.w * dv4.w;
        const float fh = p.scale * fast_exp2(sGm[kr]);
        const float fd = fast_exp2(sGam[kr] - sGm[kr]);
        const float xh[4] = {fh * hv.x, fh * hv.y, fh * hv.z, fh * hv.w};
        const float xd[4] = {fd * dv4.x, fd * dv4.y, fd * dv4.z, fd * dv4.w};
        Php.put_run<true, 4>(kr, 4 * sc4, xh);
        Pdhp.put_run<true, 4>(kr, 4 * sc4, xd);
      }
    }
    __syncthreads();
#pragma unroll
    for (int vc = 0; vc < VH / 32; ++vc) {
      const int cc = ph * VH + 32 * vc + 8 * lg;
      const bf16x8 ah = Pd.hi8(16 * W + l16, cc);
      const bf16x8 vh = Pv.hi8(16 * W + l16, cc);
      bf16x8 al = ah, vl = vh;
      if constexpr (SIN) {
        al = Pd.lo8(16 * W + l16, cc);
        vl = Pv.lo8(16 * W + l16, cc);
      }
#pragma unroll
      for (int t = 0; t < KT; ++t) {
        const bf16x8 bh = Php.hi8(16 * t + l16, 32 * vc + 8 * lg);
        const bf16x8 bl = Php.lo8(16 * t + l16, 32 * vc + 8 * lg);
        X[t] = mma<SIN, true>(X[t], ah, al, bh, bl);
        const bf16x8 ch = Pdhp.hi8(16 * t + l16, 32 * vc + 8 * lg);
        const bf16x8 cl = Pdhp.lo8(16 * t + l16, 32 * vc + 8 * lg);
        Z[t] = mma<SIN, true>(Z[t], vh, vl, ch, cl);
      }
    }
  }
  // reduce the h*dh row partials over the TPR threads of each row (contiguous lanes)
#pragma unroll
  for (int i = 0; i < NRP; ++i) {
    float x = bpart[i];
#pragma unroll
    for (int o = TPR / 2; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
    bpart[i] = x;
  }
  __syncthreads();  // all GEMMs done: smem can be reused for the dg phase
  if (sc4 == 0) {
#pragma unroll
    for (int i = 0; i < NRP; ++i) {
      const int kr = sr + RPP * i;
      if (kr < KP) sB[kr] = fast_exp2(sGam[kr]) * bpart[i];
    }
  }
#pragma unroll
  for (int t = 0; t < KT; ++t) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 16 * W + 4 * lg + r, kc = 16 * t + l16;
      sX[row * LX + kc] = X[t][r];
      sY[row * LX + kc] = Y[t][r] + Z[t][r];
      sZ[row * LX + kc] = Z[t][r];
    }
  }
  __syncthreads();

  // ---------------- phase 3: dq, dk, dg in the staging layout
  TIn* __restrict__ dq = (TIn*)p.dq;
  TIn* __restrict__ dk = (TIn*)p.dk;
  float dgr[RPS][2];
  float zk0 = 0.f, zk1 = 0.f;
#pragma unroll
  for (int i = 0; i < RPS; ++i) {
    const int r = rs * RPS + i;
    const float2 x = *(const float2*)(sX + r * LX + col);
    const float2 y = *(const float2*)(sY + r * LX + col);
    const float2 z = *(const float2*)(sZ + r * LX + col);
    const float eq0 = fast_exp2(ga[i][0] - gm0), eq1 = fast_exp2(ga[i][1] - gm1);
    const float ek0 = fast_exp2(gm0 - ga[i][0]), ek1 = fast_exp2(gm1 - ga[i][1]);
    const float dq0 = eq0 * x.x, dq1 = eq1 * x.y;
    const float dk0 = ek0 * y.x, dk1 = ek1 * y.y;
    zk0 += ka[i][0] * ek0 * z.x;
    zk1 += ka[i][1] * ek1 * z.y;
    dgr[i][0] = qa[i][0] * dq0 - ka[i][0] * dk0;
    dgr[i][1] = qa[i][1] * dq1 - ka[i][1] * dk1;
    if (r < nval && col_ok) {
      const size_t off = ((size_t)(row0 + t0 + r) * H + hh) * K + col;
      In<TIn>::st(dq + off, dq0);
      In<TIn>::st(dq + off + 1, dq1);
      In<TIn>::st(dk + off, dk0);
      In<TIn>::st(dk + off + 1, dk1);
    }
  }
  // reverse (suffix) scan within the segment
#pragma unroll
  for (int i = RPS - 2; i >= 0; --i) {
    dgr[i][0] += dgr[i + 1][0];
    dgr[i][1] += dgr[i + 1][1];
  }
  sTot[rs * KP + col] = dgr[0][0];
  sTot[rs * KP + col + 1] = dgr[0][1];
  sZk[rs * KP + col] = zk0;
  sZk[rs * KP + col + 1] = zk1;
  __syncthreads();
  float suf0 = 0.f, suf1 = 0.f, b0 = sB[col], b1 = sB[col + 1];
#pragma unroll
  for (int s = 0; s < NRS; ++s) {
    if (s > rs) {
      suf0 += sTot[s * KP + col];
      suf1 += sTot[s * KP + col + 1];
    }
    b0 += sZk[s * KP + col];
    b1 += sZk[s * KP + col + 1];
  }
#pragma unroll
  for (int i = 0; i < RPS; ++i) {
    const int r = rs * RPS + i;
    if (r < nval && col_ok) {
      const size_t off = ((size_t)(row0 + t0 + r) * H + hh) * K + col;
      *(float2*)(p.dg + off) = make_float2(dgr[i][0] + suf0 + b0, dgr[i][1] + suf1 + b1);
    }
  }
}

template <typename TIn, int KP>
static hipError_t launch_rev(const GlaBwdParams& p, hipStream_t s) {
  hipLaunchKernelGGL((gla_bwd_rev_kernel<TIn, KP>), dim3(p.NV * p.H * p.N), dim3(256), 0, s, p);
  return hipGetLastError();
}

template <typename TIn, int KP, int VP>
static hipError_t launch_main(const GlaBwdParams& p, hipStream_t s) {
  hipLaunchKernelGGL((gla_bwd_main_kernel<TIn, KP, VP>), dim3(p.total * p.H), dim3(256), 0, s, p);
  return hipGetLastError();
}

template <typename TIn>
static hipError_t launch_rev_t(const GlaBwdParams& p, hipStream_t s) {
  const int kp = p.K <= 32 ? 32 : (p.K <= 64 ? 64 : 128);
  return kp == 32 ? launch_rev<TIn, 32>(p, s)
       : kp == 64 ? launch_rev<TIn, 64>(p, s) : launch_rev<TIn, 128>(p, s);
}

template <typename TIn>
static hipError_t launch_main_t(const GlaBwdParams& p, hipStream_t s) {
  const int kp = p.K <= 32 ? 32 : (p.K <= 64 ? 64 : 128);
  const int vp = p.V <= 32 ? 32 : (p.V <= 64 ? 64 : 128);
#define TOPS_MAIN(KPV, VPV) if (kp == KPV && vp == VPV) return launch_main<TIn, KPV, VPV>(p, s);
  TOPS_MAIN(32, 32) TOPS_MAIN(32, 64) TOPS_MAIN(32, 128)
  TOPS_MAIN(64, 32) TOPS_MAIN(64, 64) TOPS_MAIN(64, 128)
  TOPS_MAIN(128, 32) TOPS_MAIN(128, 64) TOPS_MAIN(128, 128)
#undef TOPS_MAIN
  return hipErrorInvalidValue;
}

// Shape checks shared by the backward entry points; returns TOPS_OK or an error code.
static int check_bwd(const char* who, int B, int T, int H, int K, int V, int N, int total_chunks,
                     const int32_t* cu_seqlens, const int32_t* chunk_offsets,
                     const int32_t* chunk_map, bool need_map, int dtype) {
  char msg[160];
  if (B <= 0 || T <= 0 || H <= 0 || K <= 0 || V <= 0 || N <= 0) {
    snprintf(msg, sizeof(msg), "%s: non-positive dimension", who);
    return tops_set_error(TOPS_ERR_SHAPE, msg);
  }
  if (K > 128 || V > 128 || (K % 8) || (V % 8)) {
    snprintf(msg, sizeof(msg), "%s: need K, V <= 128 and multiples of 8", who);
    return tops_set_error(TOPS_ERR_SHAPE, msg);
  }
  if (cu_seqlens && (B != 1 || !chunk_offsets || (need_map && !chunk_map))) {
    snprintf(msg, sizeof(msg), "%s: varlen needs B == 1, chunk_offsets and chunk_map", who);
    return tops_set_error(TOPS_ERR_SHAPE, msg);
  }
  if (!cu_seqlens && N != B) {
    snprintf(msg, sizeof(msg), "%s: N must equal B", who);
    return tops_set_error(TOPS_ERR_SHAPE, msg);
  }
  if (!cu_seqlens && need_map && total_chunks != B * ((T + kChunk - 1) / kChunk)) {
    snprintf(msg, sizeof(msg), "%s: total_chunks must be B*ceil(T/64)", who);
    return tops_set_error(TOPS_ERR_SHAPE, msg);
  }
  if (need_map && total_chunks <= 0) {
    snprintf(msg, sizeof(msg), "%s: total_chunks must be positive", who);
    return tops_set_error(TOPS_ERR_SHAPE, msg);
  }
  if (dtype != TOPS_BF16 && dtype != TOPS_F32) {
    snprintf(msg, sizeof(msg), "%s: dtype must be TOPS_F32 or TOPS_BF16", who);
    return tops_set_error(TOPS_ERR_DTYPE, msg);
  }
  return TOPS_OK;
}

}  // namespace tops

using namespace tops;

extern "C" int tops_gla_chunk_bwd_dh(const void* q, const void* k, const float* g,
                                     const void* do_, const float* dht, float* dh_work, void* dv,
                                     float* dh0, const int32_t* cu_seqlens,
                                     const int32_t* chunk_offsets, int B, int T, int H, int K,
                                     int V, int N, int dtype, float scale, void* stream) {
  if (!q || !k || !g || !do_ || !dh_work || !dv)
    return tops_set_error(TOPS_ERR_NULL, "gla_chunk_bwd_dh: null tensor");
  int rc = check_bwd("gla_chunk_bwd_dh", B, T, H, K, V, N, 0, cu_seqlens, chunk_offsets, nullptr,
                     false, dtype);
  if (rc != TOPS_OK) return rc;
  GlaBwdParams p{q, k, nullptr, g, do_, dht, nullptr, dh_work, nullptr, nullptr, dv, nullptr, dh0,
                 cu_seqlens, chunk_offsets, nullptr, 0,
                 B, T, H, K, V, N, (V + 63) / 64, scale};
  hipStream_t s = (hipStream_t)stream;
  hipError_t e = dtype == TOPS_BF16 ? launch_rev_t<uint16_t>(p, s) : launch_rev_t<float>(p, s);
  if (e != hipSuccess) return tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
  return TOPS_OK;
}

extern "C" int tops_gla_chunk_bwd_dqkg(const void* q, const void* k, const void* v, const float* g,
                                       const void* do_, const float* h_ckpt, const float* dh_work,
                                       void* dq, void* dk, float* dg, const int32_t* cu_seqlens,
                                       const int32_t* chunk_offsets, const int32_t* chunk_map,
                                       int total_chunks, int B, int T, int H, int K, int V, int N,
                                       int dtype, float scale, void* stream) {
  if (!q || !k || !v || !g || !do_ || !h_ckpt || !dh_work || !dq || !dk || !dg)
    return tops_set_error(TOPS_ERR_NULL, "gla_chunk_bwd_dqkg: null tensor");
  int rc = check_bwd("gla_chunk_bwd_dqkg", B, T, H, K, V, N, total_chunks, cu_seqlens,
                     chunk_offsets, chunk_map, true, dtype);
  if (rc != TOPS_OK) return rc;
  GlaBwdParams p{q, k, v, g, do_, nullptr, h_ckpt, const_cast<float*>(dh_work), dq, dk, nullptr,
                 dg, nullptr, cu_seqlens, chunk_offsets, chunk_map, total_chunks,
                 B, T, H, K, V, N, (V + 63) / 64, scale};
  hipStream_t s = (hipStream_t)stream;
  hipError_t e = dtype == TOPS_BF16 ? launch_main_t<uint16_t>(p, s) : launch_main_t<float>(p, s);
  if (e != hipSuccess) return tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
  return TOPS_OK;
}

extern "C" int tops_gla_chunk_bwd(const void* q, const void* k, const void* v, const float* g,
                                  const void* do_, const float* dht, const float* h_ckpt,
                                  float* dh_work, void* dq, void* dk, void* dv, float* dg,
                                  float* dh0, const int32_t* cu_seqlens,
                                  const int32_t* chunk_offsets, const int32_t* chunk_map,
                                  int total_chunks, int B, int T, int H, int K, int V, int N,
                                  int dtype, float scale, void* stream) {
  if (!v || !h_ckpt || !dq || !dk || !dg)
    return tops_set_error(TOPS_ERR_NULL, "gla_chunk_bwd: null tensor");
  int rc = check_bwd("gla_chunk_bwd", B, T, H, K, V, N, total_chunks, cu_seqlens, chunk_offsets,
                     chunk_map, true, dtype);
  if (rc != TOPS_OK) return rc;
  rc = tops_gla_chunk_bwd_dh(q, k, g, do_, dht, dh_work, dv, dh0, cu_seqlens, chunk_offsets,
                             B, T, H, K, V, N, dtype, scale, stream);
  if (rc != TOPS_OK) return rc;
  return tops_gla_chunk_bwd_dqkg(q, k, v, g, do_, h_ckpt, dh_work, dq, dk, dg, cu_seqlens,
                                 chunk_offsets, chunk_map, total_chunks, B, T, H, K, V, N, dtype,
                                 scale, stream);
}
