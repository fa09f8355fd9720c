// GLA chunked forward for gfx950: gate cumsum + inter-chunk state recurrence +
// intra-chunk attention + output, fused in one kernel.
//
// Replaces the reference's K1 (chunk_local_cumsum_vector, tops/ops/gla/chunk.py:55-198),
// K7 (chunk_fwd_h, tops/ops/common/chunk_h.py:22-272), K2 (chunk_gla_fwd_intra_gk,
// tops/ops/gla/chunk.py:351-438) and K3 (chunk_gla_fwd_o_gk, chunk.py:1279-1440).
//
// One workgroup (4 wave64s) owns one (sequence, head, 64-wide V tile) and walks
// the sequence chunk by chunk (C = 64).  The K x 64 fp32 state lives in MFMA
// accumulator registers for the whole sequence; h is never written to HBM
// unless the caller asks for per-chunk checkpoints (training).  Per chunk:
//   G     = inclusive cumsum of log2-scaled gates, per channel (registers + LDS)
//   q~    = q * 2^(G - Gm),  k~ = k * 2^(Gm - G),   Gm = Gamma/2 (Gamma = G[last])
//   A^T   = k~ q~^T (masked j <= i, * scale)         -> kept in registers
//   o     = q~ (scale * 2^Gm * h) + A v
//   h     = 2^Gamma * h + 2^(Gamma - Gm) * (k~^T v)
// The midpoint reference Gm keeps every exponent within |Gamma|/2, the same
// stabilisation as tops/ops/gla/chunk.py:371-375.
#include "tops_common.h"
#include "tops_hip.h"

namespace tops {

struct GlaFwdParams {
  const void* q;
  const void* k;
  const void* v;
  const float* g;
  const float* h0;
  void* o;
  float* ht;
  float* hs;
  const int* cu_seqlens;
  const int* chunk_offsets;
  int B, T, H, K, V, N, NV;
  float scale;
};

template <typename TIn, int KP>
__global__ __launch_bounds__(256) void gla_fwd_kernel(GlaFwdParams p) {
  constexpr int C = kChunk, BV = 64;
  constexpr int NCP = KP / 2;          // column pairs of a [C][KP] tile
  constexpr int NRS = 256 / NCP;       // row segments
  constexpr int RPS = C / NRS;         // rows per segment
  constexpr bool SIN = !In<TIn>::kExactBf16;
  constexpr int LQ = KP + 8;           // [C][KP] planes (contraction = k)
  constexpr int LT = C + 8;            // [KP][C], [BV][C] planes (contraction = t)
  constexpr int LH = KP + 8;           // [BV][KP] plane (contraction = k)
  constexpr int NHT = (KP / 16) * (BV / 16) / 4;  // state tiles per wave

  __shared__ __attribute__((aligned(16))) uint16_t sQ[2 * C * LQ];
  __shared__ __attribute__((aligned(16))) uint16_t sK[2 * C * LQ];
  __shared__ __attribute__((aligned(16))) uint16_t sKT[2 * KP * LT];
  __shared__ __attribute__((aligned(16))) uint16_t sVT[(SIN ? 2 : 1) * BV * LT];
  __shared__ __attribute__((aligned(16))) uint16_t sHT[2 * BV * LH];
  __shared__ float sTot[NRS * KP];
  __shared__ float sGam[KP];
  __shared__ float sGm[KP];

  const Plane Pq{sQ, sQ + C * LQ, LQ};
  const Plane Pk{sK, sK + C * LQ, LQ};
  const Plane Pkt{sKT, sKT + KP * LT, LT};
  const Plane Pvt{sVT, SIN ? sVT + BV * LT : sVT, LT};
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
    cbase = p.chunk_offsets ? p.chunk_offsets[n] : 0;
  } else {
    row0 = n * p.T;
    L = p.T;
    cbase = n * cdiv(p.T, C);
  }
  const int NTs = cdiv(L, C);
  const TIn* __restrict__ q = (const TIn*)p.q;
  const TIn* __restrict__ kk = (const TIn*)p.k;
  const TIn* __restrict__ v = (const TIn*)p.v;
  const float* __restrict__ g = p.g;
  TIn* __restrict__ o = (TIn*)p.o;

  // staging coordinates for [C][KP] tiles
  const int cp = tid % NCP, rs = tid / NCP;
  const int col = 2 * cp;
  const bool col_ok = col < K;
  // staging coordinates for the [C][BV] v tile
  const int vcol = tid & 63, vrs = tid >> 6;
  const int vg = vt * BV + vcol;
  const bool vcol_ok = vg < V;

  // ---- state registers: tile t = wave + 4*i -> (m, nn)
  f32x4 hacc[NHT];
#pragma unroll
  for (int i = 0; i < NHT; ++i) {
    const int t = wave + 4 * i, m = t / (BV / 16), nn = t % (BV / 16);
    const int vv = vt * BV + 16 * nn + l16;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int kr = 16 * m + 4 * lg + r;
      float x = 0.f;
      if (p.h0 && kr < K && vv < V) x = p.h0[((size_t)(n * H + hh) * K + kr) * V + vv];
      hacc[i][r] = x;
    }
  }

  for (int c = 0; c < NTs; ++c) {
    const int t0 = c * C;
    const int nval = min(C, L - t0);
    // ---------------- load this chunk's q, k, g (RPS rows x 2 cols) and v
    float qa[RPS][2], ka[RPS][2], ga[RPS][2], va[16];
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
      va[i] = (r < nval && vcol_ok) ? In<TIn>::ld(v + ((size_t)(row0 + t0 + r) * H + hh) * V + vg)
                                    : 0.f;
    }
    // ---------------- local cumsum over the segment
#pragma unroll
    for (int i = 1; i < RPS; ++i) {
      ga[i][0] += ga[i - 1][0];
      ga[i][1] += ga[i - 1][1];
    }
    sTot[rs * KP + col] = ga[RPS - 1][0];
    sTot[rs * KP + col + 1] = ga[RPS - 1][1];
    __syncthreads();  // B1: segment totals visible; previous chunk's compute done
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
    float kt0[RPS], kt1[RPS];
#pragma unroll
    for (int i = 0; i < RPS; ++i) {
      const int r = rs * RPS + i;
      const float G0 = ga[i][0] + pre0, G1 = ga[i][1] + pre1;
      const float eq0 = fast_exp2(G0 - gm0), eq1 = fast_exp2(G1 - gm1);
      const float ek0 = fast_exp2(gm0 - G0), ek1 = fast_exp2(gm1 - G1);
      Pq.put2<true>(r, col, qa[i][0] * eq0, qa[i][1] * eq1);
      kt0[i] = ka[i][0] * ek0;
      kt1[i] = ka[i][1] * ek1;
      Pk.put2<true>(r, col, kt0[i], kt1[i]);
    }
    Pkt.put_run<true, RPS>(col, rs * RPS, kt0);
    Pkt.put_run<true, RPS>(col + 1, rs * RPS, kt1);
    Pvt.put_run<SIN, 16>(vcol, vrs * 16, va);
    __syncthreads();  // B2: sGm / sGam visible
    // ---------------- state -> LDS (scaled by scale * 2^Gm), optional checkpoint
#pragma unroll
    for (int i = 0; i < NHT; ++i) {
      const int t = wave + 4 * i, m = t / (BV / 16), nn = t % (BV / 16);
      const int kr = 16 * m + 4 * lg;
      float x[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) x[r] = p.scale * fast_exp2(sGm[kr + r]) * hacc[i][r];
      Pht.put_run<true, 4>(16 * nn + l16, kr, x);
      if (p.hs) {
        const int vv = vt * BV + 16 * nn + l16;
        float* dst = p.hs + ((size_t)(cbase + c) * H + hh) * K * V;
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (kr + r < K && vv < V) dst[(size_t)(kr + r) * V + vv] = hacc[i][r];
      }
    }
    __syncthreads();  // B3: all planes visible

    // ---------------- output rows 16*wave .. +15
    {
      const int I = wave;
      f32x4 acc[BV / 16];
#pragma unroll
      for (int nn = 0; nn < BV / 16; ++nn) acc[nn] = f32x4{0.f, 0.f, 0.f, 0.f};
      // inter-chunk: q~ . (scale 2^Gm h)
#pragma unroll
      for (int kc = 0; kc < KP / 32; ++kc) {
        const bf16x8 ah = Pq.hi8(16 * I + l16, 32 * kc + 8 * lg);
        const bf16x8 al = Pq.lo8(16 * I + l16, 32 * kc + 8 * lg);
#pragma unroll
        for (int nn = 0; nn < BV / 16; ++nn) {
          const bf16x8 bh = Pht.hi8(16 * nn + l16, 32 * kc + 8 * lg);
          const bf16x8 bl = Pht.lo8(16 * nn + l16, 32 * kc + 8 * lg);
          acc[nn] = mma<true, true>(acc[nn], ah, al, bh, bl);
        }
      }
      // intra-chunk attention A^T tiles (J, I), J <= I
      uint2 ath[4], atl[4];
#pragma unroll
      for (int J = 0; J < 4; ++J) {
        ath[J] = make_uint2(0u, 0u);
        atl[J] = make_uint2(0u, 0u);
        if (J <= I) {
          f32x4 t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int kc = 0; kc < KP / 32; ++kc) {
            const bf16x8 ah = Pk.hi8(16 * J + l16, 32 * kc + 8 * lg);
            const bf16x8 al = Pk.lo8(16 * J + l16, 32 * kc + 8 * lg);
            const bf16x8 bh = Pq.hi8(16 * I + l16, 32 * kc + 8 * lg);
            const bf16x8 bl = Pq.lo8(16 * I + l16, 32 * kc + 8 * lg);
            t = mma<true, true>(t, ah, al, bh, bl);
          }
          const int i = 16 * I + l16;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int j = 16 * J + 4 * lg + r;
            t[r] = (j <= i) ? t[r] * p.scale : 0.f;
          }
          acc_to_bf16x4(t, ath[J], atl[J]);
        }
      }
      // o += A v  (contraction over j, two 16-blocks per MFMA)
#pragma unroll
      for (int Jp = 0; Jp < 2; ++Jp) {
        if (2 * Jp <= I) {
          const int J0 = 2 * Jp, J1 = 2 * Jp + 1;
          const bf16x8 ah = cat44(ath[J0], ath[J1]);
          const bf16x8 al = cat44(atl[J0], atl[J1]);
#pragma unroll
          for (int nn = 0; nn < BV / 16; ++nn) {
            const bf16x8 bh = Pvt.hi44(16 * nn + l16, 16 * J0 + 4 * lg, 16 * J1 + 4 * lg);
            bf16x8 bl = bh;
            if constexpr (SIN) bl = Pvt.lo44(16 * nn + l16, 16 * J0 + 4 * lg, 16 * J1 + 4 * lg);
            acc[nn] = mma<true, SIN>(acc[nn], ah, al, bh, bl);
          }
        }
      }
#pragma unroll
      for (int nn = 0; nn < BV / 16; ++nn) {
        const int vv = vt * BV + 16 * nn + l16;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = 16 * I + 4 * lg + r;
          if (i < nval && vv < V) In<TIn>::st(o + ((size_t)(row0 + t0 + i) * H + hh) * V + vv, acc[nn][r]);
        }
      }
    }
    // ---------------- state update
#pragma unroll
    for (int i = 0; i < NHT; ++i) {
      const int t = wave + 4 * i, m = t / (BV / 16), nn = t % (BV / 16);
      f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kc = 0; kc < C / 32; ++kc) {
        const bf16x8 ah = Pkt.hi8(16 * m + l16, 32 * kc + 8 * lg);
        const bf16x8 al = Pkt.lo8(16 * m + l16, 32 * kc + 8 * lg);
        const bf16x8 bh = Pvt.hi8(16 * nn + l16, 32 * kc + 8 * lg);
        bf16x8 bl = bh;
        if constexpr (SIN) bl = Pvt.lo8(16 * nn + l16, 32 * kc + 8 * lg);
        d = mma<true, SIN>(d, ah, al, bh, bl);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int kr = 16 * m + 4 * lg + r;
        const float gam = sGam[kr], gmv = sGm[kr];
        hacc[i][r] = fast_exp2(gam) * hacc[i][r] + fast_exp2(gam - gmv) * d[r];
      }
    }
  }

  if (p.ht) {
#pragma unroll
    for (int i = 0; i < NHT; ++i) {
      const int t = wave + 4 * i, m = t / (BV / 16), nn = t % (BV / 16);
      const int vv = vt * BV + 16 * nn + l16;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int kr = 16 * m + 4 * lg + r;
        if (kr < K && vv < V) p.ht[((size_t)(n * H + hh) * K + kr) * V + vv] = hacc[i][r];
      }
    }
  }
}

template <typename TIn, int KP>
static hipError_t launch_fwd(const GlaFwdParams& p, hipStream_t s) {
  dim3 grid(p.NV * p.H * p.N);
  hipLaunchKernelGGL((gla_fwd_kernel<TIn, KP>), grid, dim3(256), 0, s, p);
  return hipGetLastError();
}

}  // namespace tops

using namespace tops;

extern "C" int tops_gla_chunk_fwd(const void* q, const void* k, const void* v, const float* g,
                                  const float* h0, void* o, float* ht, float* h_ckpt,
                                  const int32_t* cu_seqlens, const int32_t* chunk_offsets,
                                  int B, int T, int H, int K, int V, int N, int dtype,
                                  float scale, void* stream) {
  if (!q || !k || !v || !g || !o) return tops_set_error(TOPS_ERR_NULL, "gla_chunk_fwd: null tensor");
  if (B <= 0 || T <= 0 || H <= 0 || K <= 0 || V <= 0 || N <= 0)
    return tops_set_error(TOPS_ERR_SHAPE, "gla_chunk_fwd: non-positive dimension");
  if (K > 128 || (K % 8) || (V % 8))
    return tops_set_error(TOPS_ERR_SHAPE, "gla_chunk_fwd: need K <= 128, K % 8 == 0, V % 8 == 0");
  if (cu_seqlens && B != 1) return tops_set_error(TOPS_ERR_SHAPE, "gla_chunk_fwd: varlen needs B == 1");
  if (!cu_seqlens && N != B) return tops_set_error(TOPS_ERR_SHAPE, "gla_chunk_fwd: N must equal B");
  if (h_ckpt && cu_seqlens && !chunk_offsets)
    return tops_set_error(TOPS_ERR_NULL, "gla_chunk_fwd: varlen checkpoints need chunk_offsets");
  GlaFwdParams p{q, k, v, g, h0, o, ht, h_ckpt, cu_seqlens, chunk_offsets,
                 B, T, H, K, V, N, (V + 63) / 64, scale};
  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  const int kp = K <= 32 ? 32 : (K <= 64 ? 64 : 128);
  if (dtype == TOPS_BF16) {
    e = kp == 32 ? launch_fwd<uint16_t, 32>(p, s) : kp == 64 ? launch_fwd<uint16_t, 64>(p, s)
                                                            : launch_fwd<uint16_t, 128>(p, s);
  } else if (dtype == TOPS_F32) {
    e = kp == 32 ? launch_fwd<float, 32>(p, s) : kp == 64 ? launch_fwd<float, 64>(p, s)
                                                         : launch_fwd<float, 128>(p, s);
  } else {
    return tops_set_error(TOPS_ERR_DTYPE, "gla_chunk_fwd: dtype must be TOPS_F32 or TOPS_BF16");
  }
  if (e != hipSuccess) return tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
  return TOPS_OK;
}
