// GLA backward, chunk-parallel stage: dq, dk and the gate gradient dg for gfx950.
//
// Replaces the dq/dk/dg part of the reference's fused K4 (chunk_gla_bwd_fused_kernel,
// tops/ops/gla/chunk.py:1447-1581), following the oracle tops/cpu/ops/gla/chunk.py:357-466
// (chunk_gla_bwd_dqk_intra and chunk_gla_bwd_dqkg).
//
// One workgroup (4 wave64) per (chunk, head).  With G the in-chunk gate cumsum (log2
// units), Gamma = G[last], Gm = Gamma / 2, q~ = q 2^(G-Gm), k~ = k 2^(Gm-G), h_c the state
// before the chunk and dh_c the gradient w.r.t. the state after it:
//     dA  = scale tril(dO v^T)
//     X   = dA k~ + dO (scale 2^Gm h_c)^T            dq = 2^(G-Gm) X
//     W   = dA^T q~ + v (2^(Gamma-Gm) dh_c)^T         dk = 2^(Gm-G) W
//     dg  = revcumsum_t(q dq - k dk) + 2^Gamma sum_v(h_c dh_c) + sum_t k~ W_inter
// The last term is sum_t k dk_inter of the oracle (k dk_inter = k~ W_inter).
//
// Wave w owns token rows 16w..16w+15 of X and W.  The h_c / dh_c checkpoints are fp32
// [K][V] with V contiguous, which is already the MFMA B-operand layout for a contraction
// over V: each lane reads its 8 values straight from global memory (L2), scales and
// splits them into bf16 hi/lo, so no LDS holds a state.  K is processed in passes of 32
// (K = 128) or 64 channels so that the gated q~^T / k~^T planes, the v / dO planes and
// the fp32 epilogue tiles fit in < 64 KB of LDS and the registers stay under 256: two
// workgroups share a CU and overlap each other's loads with compute.
#include "gla_sweep.h"
#include "tops_common.h"

namespace tops {

template <typename TIn, int KP, int VP>
__global__ __launch_bounds__(256, 2) void gla_dqkg_kernel(DqkgParams p) {
  constexpr int C = kChunk;
  constexpr int NQ = KP / 4, NSEG = 256 / NQ, RPT = C / NSEG;   // [C][KP] staging
  constexpr int KH = KP == 64 ? 64 : 32;                        // channels per pass
  constexpr int NKH = KP / KH;
  constexpr int KB = KH / 16;
  constexpr int VC = VP / 32;
  constexpr bool SIN = !In<TIn>::kExactBf16;
  constexpr int NPL = SIN ? 2 : 1;
  constexpr int ES = sizeof(TIn);
  constexpr int LV = VP + 8, LT = C + 8, LX = KH + 4;
  constexpr int EP = 16 / ES;                  // elements per 16-byte piece of v / dO
  constexpr int NPC = VP / EP;                 // pieces per row
  constexpr int NPT = C * NPC / 256;           // pieces per thread
  constexpr int kPlanes = 2 * 2 * KH * LT * 2;            // q~^T, k~^T hi/lo (bytes)
  constexpr int kTiles = 2 * C * LX * 4;                  // X, W fp32 (bytes)
  constexpr int kRegion = kPlanes > kTiles ? kPlanes : kTiles;
  static_assert(RPT == 2 || RPT == 4 || RPT == 8, "KP must be 32, 64 or 128");
  static_assert(NPT >= 1 && C * NPC % 256 == 0, "VP must be 32, 64 or 128");
  typedef Words<TIn> Wd;

  __shared__ __attribute__((aligned(16))) uint16_t sV[NPL * C * LV];
  __shared__ __attribute__((aligned(16))) uint16_t sD[NPL * C * LV];
  __shared__ __attribute__((aligned(16))) unsigned char sR[kRegion];
  __shared__ __attribute__((aligned(16))) float sTot[NSEG * KP];
  __shared__ float sGm[KP];
  __shared__ float sGam[KP];
  __shared__ float sZk[4 * KH];
  __shared__ float sHdh[KH];

  const Plane Pv{sV, SIN ? sV + C * LV : sV, LV};
  const Plane Pd{sD, SIN ? sD + C * LV : sD, LV};
  uint16_t* rp = (uint16_t*)sR;
  const Plane Pqt{rp, rp + KH * LT, LT};
  const Plane Pkt{rp + 2 * KH * LT, rp + 3 * KH * LT, LT};
  float* sXf = (float*)sR;
  float* sWf = sXf + C * LX;

  const int tid = threadIdx.x, lane = tid & 63;
  const int W = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lg = lane >> 4;
  const int hh = blockIdx.x % p.H;
  const int gc = blockIdx.x / p.H;
  const int H = p.H, K = p.K, V = p.V;
  const float scale = p.scale;

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
  const long long rows_total = (long long)p.B * p.T;
  const size_t e0 = (size_t)(row0 + t0) * H + hh;
  const long long remr = (rows_total - (row0 + t0)) * (long long)H;
  const uint32_t rowK = (uint32_t)(H * K), rowV = (uint32_t)(H * V);

  // ---------------- phase 0: loads
  const int cq = tid % NQ, seg = tid / NQ;
  const int c0 = 4 * cq, r0 = seg * RPT;
  const bool colok = c0 < K;
  const uint32_t offQ = colok ? ((uint32_t)r0 * rowK + c0) * ES : kOOB;
  const uint32_t offG = colok ? ((uint32_t)r0 * rowK + c0) * 4u : kOOB;
  const rsrc_t Rq = make_rsrc((const TIn*)p.q + e0 * K, remr * K * ES);
  const rsrc_t Rk = make_rsrc((const TIn*)p.k + e0 * K, remr * K * ES);
  const rsrc_t Rg = make_rsrc(p.g + e0 * K, remr * K * 4);
  const rsrc_t Rv = make_rsrc((const TIn*)p.v + e0 * V, remr * V * ES);
  const rsrc_t Rd = make_rsrc((const TIn*)p.dout + e0 * V, remr * V * ES);
  typename Wd::W4 rq[RPT], rk[RPT];
  float G[RPT][4];
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const bool ok = r0 + i < nval;
    rq[i] = Wd::ld4(Rq, ok ? offQ : kOOB, i * rowK * ES);
    rk[i] = Wd::ld4(Rk, ok ? offQ : kOOB, i * rowK * ES);
    float x[4];
    unpack4(bld128(Rg, ok ? offG : kOOB, i * rowK * 4), x);
#pragma unroll
    for (int j = 0; j < 4; ++j) G[i][j] = x[j] * kLog2e + (i > 0 ? G[i - 1][j] : 0.f);
  }
  uint4 pv[NPT], pd[NPT];
#pragma unroll
  for (int i = 0; i < NPT; ++i) {
    const int pc = tid + 256 * i, row = pc / NPC, col = (pc % NPC) * EP;
    const uint32_t o = (row < nval && col < V) ? ((uint32_t)row * rowV + col) * ES : kOOB;
    pv[i] = bld128(Rv, o, 0);
    pd[i] = bld128(Rd, o, 0);
  }

  // ---------------- phase 1: gate cumsum across segments, v / dO planes
  *(float4*)(sTot + seg * KP + c0) = make_float4(G[RPT - 1][0], G[RPT - 1][1], G[RPT - 1][2], G[RPT - 1][3]);
#pragma unroll
  for (int i = 0; i < NPT; ++i) {
    const int pc = tid + 256 * i, row = pc / NPC, col = (pc % NPC) * EP;
    if constexpr (!SIN) {
      *(uint4*)(Pv.hi + row * LV + col) = pv[i];
      *(uint4*)(Pd.hi + row * LV + col) = pd[i];
    } else {
      float a[4], b[4];
      unpack4(pv[i], a);
      unpack4(pd[i], b);
      put_n<true, 4>(Pv, row, col, a);
      put_n<true, 4>(Pd, row, col, b);
    }
  }
  __syncthreads();
  float gm[4], gam[4];
  {
    float pre[4] = {0.f, 0.f, 0.f, 0.f};
    gam[0] = gam[1] = gam[2] = gam[3] = 0.f;
#pragma unroll
    for (int s = 0; s < NSEG; ++s) {
      const float4 t = *(const float4*)(sTot + s * KP + c0);
      if (s < seg) { pre[0] += t.x; pre[1] += t.y; pre[2] += t.z; pre[3] += t.w; }
      gam[0] += t.x; gam[1] += t.y; gam[2] += t.z; gam[3] += t.w;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      gm[j] = 0.5f * gam[j];
#pragma unroll
      for (int i = 0; i < RPT; ++i) G[i][j] += pre[j];
    }
  }
  if (seg == 0) {
    *(float4*)(sGm + c0) = make_float4(gm[0], gm[1], gm[2], gm[3]);
    *(float4*)(sGam + c0) = make_float4(gam[0], gam[1], gam[2], gam[3]);
  }

  // gated q~^T / k~^T planes of the channel half kh (threads owning those columns)
  auto stage = [&](int kh) {
    const int cl = c0 - kh * KH;
    if (cl >= 0 && cl < KH) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float qt[RPT], kt[RPT];
#pragma unroll
        for (int i = 0; i < RPT; ++i) {
          float qv[4], kv[4];
          unpack4(rq[i], qv);
          unpack4(rk[i], kv);
          qt[i] = qv[j] * fast_exp2(G[i][j] - gm[j]);
          kt[i] = kv[j] * fast_exp2(gm[j] - G[i][j]);
        }
        put_n<true, RPT>(Pqt, cl + j, r0, qt);
        put_n<true, RPT>(Pkt, cl + j, r0, kt);
      }
    }
  };
  stage(0);
  __syncthreads();

  const float* hsrc = p.hs + ((size_t)gc * H + hh) * K * V;
  const float* dsrc = p.dhs + ((size_t)gc * H + hh) * K * V;
  const rsrc_t Rh = make_rsrc(hsrc, (long long)K * V * 4);
  const rsrc_t Rdh = make_rsrc(dsrc, (long long)K * V * 4);
  const rsrc_t Rdq = make_rsrc((TIn*)p.dq + e0 * K, remr * K * ES);
  const rsrc_t Rdk = make_rsrc((TIn*)p.dk + e0 * K, remr * K * ES);
  const rsrc_t Rdg = make_rsrc(p.dg + e0 * K, remr * K * 4);

#pragma unroll 1
  for (int kh = 0; kh < NKH; ++kh) {
    if (kh > 0) {
      __syncthreads();  // previous half's epilogue is done with the region
      stage(kh);
      __syncthreads();
    }
    f32x4 X[KB], Wt[KB];
    float hd[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      X[kb] = f32x4{0.f, 0.f, 0.f, 0.f};
      Wt[kb] = f32x4{0.f, 0.f, 0.f, 0.f};
      hd[kb] = 0.f;
    }
    // ---- inter-chunk: X += dO (alpha h)^T, W += v (beta dh)^T, straight from the checkpoints
#pragma unroll
    for (int vc = 0; vc < VC; ++vc) {
      const bf16x8 doh = Pd.hi8(16 * W + l16, 32 * vc + 8 * lg);
      const bf16x8 vh = Pv.hi8(16 * W + l16, 32 * vc + 8 * lg);
      bf16x8 dol = doh, vl = vh;
      if constexpr (SIN) {
        dol = Pd.lo8(16 * W + l16, 32 * vc + 8 * lg);
        vl = Pv.lo8(16 * W + l16, 32 * vc + 8 * lg);
      }
      const int v0 = 32 * vc + 8 * lg;
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        const int kk = kh * KH + 16 * kb + l16;
        const uint32_t o = (kk < K && v0 < V) ? ((uint32_t)kk * V + v0) * 4u : kOOB;
        const uint4 h0 = bld128(Rh, o, 0), h1 = bld128(Rh, o, 16);
        const uint4 d0 = bld128(Rdh, o, 0), d1 = bld128(Rdh, o, 16);
        float hv[8], dv[8];
        unpack4(h0, hv);
        unpack4(h1, hv + 4);
        unpack4(d0, dv);
        unpack4(d1, dv + 4);
        if (W == 0) {
#pragma unroll
          for (int e = 0; e < 8; ++e) hd[kb] += hv[e] * dv[e];
        }
        const float al = scale * fast_exp2(sGm[kk]);
        const float be = fast_exp2(sGam[kk] - sGm[kk]);
        uint32_t hh_[4], hl_[4], dh_[4], dl_[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          split_bf16x2(al * hv[2 * e], al * hv[2 * e + 1], hh_[e], hl_[e]);
          split_bf16x2(be * dv[2 * e], be * dv[2 * e + 1], dh_[e], dl_[e]);
        }
        const bf16x8 Bh = __builtin_bit_cast(bf16x8, make_uint4(hh_[0], hh_[1], hh_[2], hh_[3]));
        const bf16x8 Bl = __builtin_bit_cast(bf16x8, make_uint4(hl_[0], hl_[1], hl_[2], hl_[3]));
        const bf16x8 Dh = __builtin_bit_cast(bf16x8, make_uint4(dh_[0], dh_[1], dh_[2], dh_[3]));
        const bf16x8 Dl = __builtin_bit_cast(bf16x8, make_uint4(dl_[0], dl_[1], dl_[2], dl_[3]));
        X[kb] = mma<SIN, true>(X[kb], doh, dol, Bh, Bl);
        Wt[kb] = mma<SIN, true>(Wt[kb], vh, vl, Dh, Dl);
      }
    }
    // ---- sum_t k~ W_inter for this wave's rows (before the intra part joins W)
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      const int cl = 16 * kb + l16, j0 = 16 * W + 4 * lg;
      const uint2 kh_ = *(const uint2*)(Pkt.hi + cl * LT + j0);
      const uint2 kl_ = *(const uint2*)(Pkt.lo + cl * LT + j0);
      float a[4], b[4];
      unpack4(kh_, a);
      unpack4(kl_, b);
      float z = 0.f;
#pragma unroll
      for (int r = 0; r < 4; ++r) z += (a[r] + b[r]) * Wt[kb][r];
      z += __shfl_xor(z, 16, 64);
      z += __shfl_xor(z, 32, 64);
      if (lg == 0) sZk[W * KH + cl] = z;
      if (W == 0) {
        float x = hd[kb];
        x += __shfl_xor(x, 16, 64);
        x += __shfl_xor(x, 32, 64);
        if (lg == 0) sHdh[cl] = x;
      }
    }
    uint2 dthh[4], dthl[4], dahh[4], dahl[4];
    // ---- dA tiles of this wave's rows (registers), recomputed per pass to keep them
      // out of the inter-chunk loop's register peak
    // dth[J], J <= W: lane holds dA[16W + l16][16J + 4lg + r]   (A-operand of dA k~)
    // dah[I], I >= W: lane holds dA[16I + 4lg + r][16W + l16]   (A-operand of dA^T q~)
  #pragma unroll
    for (int J = 0; J < 4; ++J) {
      dthh[J] = dthl[J] = dahh[J] = dahl[J] = make_uint2(0u, 0u);
      if (J <= W) {
        f32x4 t = {0.f, 0.f, 0.f, 0.f};
  #pragma unroll
        for (int vc = 0; vc < VC; ++vc) {
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
        for (int r = 0; r < 4; ++r) t[r] = (16 * J + 4 * lg + r <= i) ? t[r] * scale : 0.f;
        acc_to_bf16x4(t, dthh[J], dthl[J]);
      }
      if (J >= W) {
        f32x4 t = {0.f, 0.f, 0.f, 0.f};
  #pragma unroll
        for (int vc = 0; vc < VC; ++vc) {
          const bf16x8 ah = Pd.hi8(16 * J + l16, 32 * vc + 8 * lg);
          const bf16x8 bh = Pv.hi8(16 * W + l16, 32 * vc + 8 * lg);
          bf16x8 al = ah, bl = bh;
          if constexpr (SIN) {
            al = Pd.lo8(16 * J + l16, 32 * vc + 8 * lg);
            bl = Pv.lo8(16 * W + l16, 32 * vc + 8 * lg);
          }
          t = mma<SIN, SIN>(t, ah, al, bh, bl);
        }
        const int j = 16 * W + l16;
  #pragma unroll
        for (int r = 0; r < 4; ++r) t[r] = (j <= 16 * J + 4 * lg + r) ? t[r] * scale : 0.f;
        acc_to_bf16x4(t, dahh[J], dahl[J]);
      }
    }
    // ---- intra-chunk: X += dA k~, W += dA^T q~ (contraction over tokens)
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
      for (int Pp = 0; Pp < 2; ++Pp) {
        const int P0 = 2 * Pp, P1 = 2 * Pp + 1;
        if (P0 <= W) {
          X[kb] = mma<true, true>(X[kb], cat44(dthh[P0], dthh[P1]), cat44(dthl[P0], dthl[P1]),
                                  Pkt.hi44(16 * kb + l16, 16 * P0 + 4 * lg, 16 * P1 + 4 * lg),
                                  Pkt.lo44(16 * kb + l16, 16 * P0 + 4 * lg, 16 * P1 + 4 * lg));
        }
        if (P1 >= W) {
          Wt[kb] = mma<true, true>(Wt[kb], cat44(dahh[P0], dahh[P1]), cat44(dahl[P0], dahl[P1]),
                                   Pqt.hi44(16 * kb + l16, 16 * P0 + 4 * lg, 16 * P1 + 4 * lg),
                                   Pqt.lo44(16 * kb + l16, 16 * P0 + 4 * lg, 16 * P1 + 4 * lg));
        }
      }
    }
    __syncthreads();  // every wave is done reading the planes: the region takes the tiles
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 16 * W + 4 * lg + r, cl = 16 * kb + l16;
        sXf[row * LX + cl] = X[kb][r];
        sWf[row * LX + cl] = Wt[kb][r];
      }
    }
    __syncthreads();
    // ---- epilogue in the staging layout: dq, dk, and dg for this half's columns
    const int cl = c0 - kh * KH;
    const bool mine = cl >= 0 && cl < KH;
    float dgr[RPT][4];
    if (mine) {
#pragma unroll
      for (int i = 0; i < RPT; ++i) {
        const int r = r0 + i;
        const float4 x = *(const float4*)(sXf + r * LX + cl);
        const float4 w = *(const float4*)(sWf + r * LX + cl);
        const float xs[4] = {x.x, x.y, x.z, x.w}, ws[4] = {w.x, w.y, w.z, w.w};
        float qv[4], kv[4];
        unpack4(rq[i], qv);
        unpack4(rk[i], kv);
        f32x4 dqv, dkv;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          dqv[j] = fast_exp2(G[i][j] - gm[j]) * xs[j];
          dkv[j] = fast_exp2(gm[j] - G[i][j]) * ws[j];
          dgr[i][j] = qv[j] * dqv[j] - kv[j] * dkv[j];
        }
        const bool ok = r < nval;
        Wd::st4(Rdq, dqv, ok ? offQ : kOOB, i * rowK * ES);
        Wd::st4(Rdk, dkv, ok ? offQ : kOOB, i * rowK * ES);
      }
#pragma unroll
      for (int i = RPT - 2; i >= 0; --i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) dgr[i][j] += dgr[i + 1][j];
      }
      *(float4*)(sTot + seg * KP + c0) = make_float4(dgr[0][0], dgr[0][1], dgr[0][2], dgr[0][3]);
    }
    __syncthreads();
    if (mine) {
      float add[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        add[j] = fast_exp2(gam[j]) * sHdh[cl + j];
#pragma unroll
        for (int w = 0; w < 4; ++w) add[j] += sZk[w * KH + cl + j];
      }
#pragma unroll
      for (int s = 0; s < NSEG; ++s) {
        if (s > seg) {
          const float4 t = *(const float4*)(sTot + s * KP + c0);
          add[0] += t.x; add[1] += t.y; add[2] += t.z; add[3] += t.w;
        }
      }
#pragma unroll
      for (int i = 0; i < RPT; ++i) {
        const bool ok = r0 + i < nval;
        bst128(Rdg, make_uint4(__float_as_uint(dgr[i][0] + add[0]), __float_as_uint(dgr[i][1] + add[1]),
                               __float_as_uint(dgr[i][2] + add[2]), __float_as_uint(dgr[i][3] + add[3])),
               ok ? offG : kOOB, i * rowK * 4);
      }
    }
  }
}

template <typename TIn>
hipError_t launch_gla_dqkg(const DqkgParams& p, hipStream_t s) {
  const int kp = p.K <= 32 ? 32 : (p.K <= 64 ? 64 : 128);
  const int vp = p.V <= 32 ? 32 : (p.V <= 64 ? 64 : 128);
  dim3 grid(p.total * p.H), block(256);
#define TOPS_DQKG(KPV, VPV) \
  if (kp == KPV && vp == VPV) { hipLaunchKernelGGL((gla_dqkg_kernel<TIn, KPV, VPV>), grid, block, 0, s, p); return hipGetLastError(); }
  TOPS_DQKG(32, 32) TOPS_DQKG(32, 64) TOPS_DQKG(32, 128)
  TOPS_DQKG(64, 32) TOPS_DQKG(64, 64) TOPS_DQKG(64, 128)
  TOPS_DQKG(128, 32) TOPS_DQKG(128, 64) TOPS_DQKG(128, 128)
#undef TOPS_DQKG
  return hipErrorInvalidValue;
}

template hipError_t launch_gla_dqkg<uint16_t>(const DqkgParams&, hipStream_t);
template hipError_t launch_gla_dqkg<float>(const DqkgParams&, hipStream_t);

}  // namespace tops
