// KDA backward, WY stage, for gfx950: gradients that flow through u = T (beta v),
// w = T (beta 2^G k) and Akk.
//
// Replaces the WY part of the reference's fused K18 (_chunk_kda_bwd_wy_dqkg_fused_kernel,
// tops/ops/kda/chunk_bwd.py:19-141) and the Akk part of K17 (kda_intra_chunk_bwd_kernel,
// tops/ops/kda/chunk_intra.py:283-383), following the oracle
// tops/cpu/ops/kda/chunk_bwd.py:525-668 (wy_fast.py for the WY backward).
//
// One workgroup (4 wave64) per (chunk, head).  With dv_new the gradient w.r.t.
// v_new = u - w S (S the state before the chunk), the WY backward collapses to
//     P    = T^T dv_new                      (dL/d(beta v))
//     dbk  = -P S^T                          (dL/d(beta 2^G k))
//     dAkk = -P v_new^T, strictly lower      (since v_new = T (beta v - beta 2^G k S))
// and then
//     dv    = beta P
//     dbeta = sum_v v P + sum_d 2^G k dbk + sum_d k Y1
//     dk    = beta 2^G dbk + beta Y1 + Y2
//     dG    = beta 2^G k dbk + beta k Y1 - k Y2          (w.r.t. the natural-log cumsum)
// with Y1[i] = 2^(G_i - Gm) sum_j dAkk[i][j] k~_j (k~ = k 2^(Gm - G)) and
//      Y2[j] = 2^(Gm - G_j) sum_i beta_i dAkk[i][j] k^_i (k^ = k 2^(G - Gm)).
// dg_wy is the reverse in-chunk cumsum of dG.  The GLA-shaped terms (through o and the
// state update) are added by the dq / dk / dg kernel, which reads dk_wy and dg_wy.
//
// Wave R owns token block R (16 tokens).  P goes through LDS (bf16 hi/lo); the dAkk tiles
// stay in registers for the channel passes (32 channels each: gated k^T planes, gate
// cumsum).  The inputs T^T [C][C] and dv_new^T [V][C] are stored transposed per chunk,
// so MFMA operands load straight from global memory.
#include "kda.h"
#include "tops_common.h"

namespace tops {

__device__ __forceinline__ void load_split8(rsrc_t r, uint32_t off, bf16x8& h, bf16x8& l) {
  float a[4], b[4];
  unpack4(bld128(r, off, 0), a);
  unpack4(bld128(r, off == kOOB ? kOOB : off + 16u, 0), b);
  uint32_t hh[4], ll[4];
  split_bf16x2(a[0], a[1], hh[0], ll[0]);
  split_bf16x2(a[2], a[3], hh[1], ll[1]);
  split_bf16x2(b[0], b[1], hh[2], ll[2]);
  split_bf16x2(b[2], b[3], hh[3], ll[3]);
  h = __builtin_bit_cast(bf16x8, make_uint4(hh[0], hh[1], hh[2], hh[3]));
  l = __builtin_bit_cast(bf16x8, make_uint4(ll[0], ll[1], ll[2], ll[3]));
}

template <typename TIn, int KP, int VP>
__global__ __launch_bounds__(256, 2) void kda_wy_kernel(KdaWyParams p) {
  constexpr int C = kChunk;
  constexpr int KH = 32;                 // channels per pass
  constexpr int NPS = KP / KH;
  constexpr int VC = VP / 32;
  constexpr int NVB = VP / 16;           // 16-wide V blocks
  constexpr int ES = sizeof(TIn);
  constexpr int LP = VP + 8, LT = C + 8, LG = KH + 4;
  static_assert(KP % KH == 0 && VP % 32 == 0, "KP, VP must be 32, 64 or 128");
  typedef Words<TIn> Wd;

  __shared__ __attribute__((aligned(16))) uint16_t sP[2 * C * LP];
  __shared__ __attribute__((aligned(16))) uint16_t sK1t[2 * KH * LT];
  __shared__ __attribute__((aligned(16))) uint16_t sK2t[2 * KH * LT];
  __shared__ __attribute__((aligned(16))) float sG[C * LG];
  __shared__ __attribute__((aligned(16))) float sTot[8 * KH];
  __shared__ __attribute__((aligned(16))) float sGm[KH];
  __shared__ __attribute__((aligned(16))) float sBlk[2 * 16];     // per channel half: tokens 32..63 total
  __shared__ float sBeta[C];
  __shared__ float sDbv[4 * C];         // per wave: sum_v v P over its V blocks
  __shared__ float sDbk[2 * C];         // per channel half: sum_d (2^G k dbk + k Y1)

  const Plane PP{sP, sP + C * LP, LP};
  const Plane PK1t{sK1t, sK1t + KH * LT, LT};
  const Plane PK2t{sK2t, sK2t + KH * LT, LT};

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kb = wave & 1, tp = wave >> 1;   // channel half of a pass, token-block pair
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
  const rsrc_t Rvn = make_rsrc_rows(p.vnew, e0, nrows, V);
  const rsrc_t Rb = make_rsrc_rows(p.beta, e0, nrows, 1);
  const rsrc_t Rtt = make_rsrc(p.tt + ((size_t)gc * H + hh) * C * C, (long long)C * C * 4);
  const rsrc_t Rdvt = make_rsrc(p.dvnt + ((size_t)gc * H + hh) * V * C, (long long)V * C * 4);
  const rsrc_t Rh = make_rsrc(p.hs + ((size_t)gc * H + hh) * K * V, (long long)K * V * 4);

  if (tid < C) sBeta[tid] = __uint_as_float(bld32(Rb, tid < nval ? (uint32_t)tid * H * 4u : kOOB, 0));
  __syncthreads();  // beta visible

  // ---------------- P = T^T dv_new: wave w takes the V blocks vb = w, w + 4, ..; tile (vb, I)
  // computed transposed, lane holds P[16I + l16][16vb + 4lg + r].  Every global operand of
  // the phase (dv_new^T and T^T fragments, v rows) is requested before the first product.
  {
    constexpr int NVW = (NVB + 3) / 4;          // V blocks per wave
    const rsrc_t Rdv = make_rsrc_rows((const TIn*)p.dv, e0, nrows, V);
    uint4 draw[NVW][2][2], traw[4][2][2];
    typename Wd::W4 vraw[NVW][4];
#pragma unroll
    for (int u = 0; u < NVW; ++u) {
      const int vb = wave + 4 * u;
      const int v = 16 * vb + l16;
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        const uint32_t o = (vb < NVB && v < V) ? ((uint32_t)v * C + 32 * kc + 8 * lg) * 4u : kOOB;
        draw[u][kc][0] = bld128(Rdvt, o, 0);
        draw[u][kc][1] = bld128(Rdvt, o == kOOB ? kOOB : o + 16u, 0);
      }
    }
#pragma unroll
    for (int I = 0; I < 4; ++I) {
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        if (kc == 1 || I < 2) {                 // T[i'][i] = 0 for i' < i
          const uint32_t o = ((uint32_t)(16 * I + l16) * C + 32 * kc + 8 * lg) * 4u;
          traw[I][kc][0] = bld128(Rtt, o, 0);
          traw[I][kc][1] = bld128(Rtt, o + 16u, 0);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < NVW; ++u) {
#pragma unroll
      for (int I = 0; I < 4; ++I) {
        const int vb = wave + 4 * u, i = 16 * I + l16, col = 16 * vb + 4 * lg;
        vraw[u][I] = Wd::ld4(Rv, (vb < NVB && i < nval && col < V) ? ((uint32_t)i * rowV + col) * ES : kOOB, 0);
      }
    }
    auto split16 = [](const uint4 (&r)[2], bf16x8& h, bf16x8& l) {
      float a[4], b[4];
      unpack4(r[0], a);
      unpack4(r[1], b);
      uint32_t hh[4], ll[4];
      split_bf16x2(a[0], a[1], hh[0], ll[0]);
      split_bf16x2(a[2], a[3], hh[1], ll[1]);
      split_bf16x2(b[0], b[1], hh[2], ll[2]);
      split_bf16x2(b[2], b[3], hh[3], ll[3]);
      h = __builtin_bit_cast(bf16x8, make_uint4(hh[0], hh[1], hh[2], hh[3]));
      l = __builtin_bit_cast(bf16x8, make_uint4(ll[0], ll[1], ll[2], ll[3]));
    };
    bf16x8 th[4][2], tl[4][2];
#pragma unroll
    for (int I = 0; I < 4; ++I) {
#pragma unroll
      for (int kc = 0; kc < 2; ++kc)
        if (kc == 1 || I < 2) split16(traw[I][kc], th[I][kc], tl[I][kc]);
    }
    float dbv[4] = {0.f, 0.f, 0.f, 0.f};        // per token block I: sum_v v P (this lane's v's)
#pragma unroll
    for (int u = 0; u < NVW; ++u) {
      const int vb = wave + 4 * u;
      if (vb < NVB) {
        bf16x8 ah[2], al[2];
#pragma unroll
        for (int kc = 0; kc < 2; ++kc) split16(draw[u][kc], ah[kc], al[kc]);
#pragma unroll
        for (int I = 0; I < 4; ++I) {
          const int i = 16 * I + l16;
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int kc = 0; kc < 2; ++kc)
            if (kc == 1 || I < 2) acc = mma<true, true>(acc, ah[kc], al[kc], th[I][kc], tl[I][kc]);
          const float x[4] = {acc[0], acc[1], acc[2], acc[3]};
          put_n<true, 4>(PP, i, 16 * vb + 4 * lg, x);
          const int col = 16 * vb + 4 * lg;
          const uint32_t off = (i < nval && col < V) ? ((uint32_t)i * rowV + col) * ES : kOOB;
          float vv[4];
          unpack4(vraw[u][I], vv);
#pragma unroll
          for (int r = 0; r < 4; ++r) dbv[I] += vv[r] * acc[r];
          const float bi = sBeta[i];
          Wd::st4(Rdv, f32x4{bi * acc[0], bi * acc[1], bi * acc[2], bi * acc[3]}, off, 0);
        }
      }
    }
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      float x = dbv[I];
      x += __shfl_xor(x, 16, 64);
      x += __shfl_xor(x, 32, 64);
      if (lg == 0) sDbv[wave * C + 16 * I + l16] = x;
    }
  }
  __syncthreads();  // P plane visible

  // ---------------- dAkk tiles (registers, all passes) for the token blocks t = 2tp + a
  // dar[a][J] (J <= t): lane holds dAkk[16t + l16][16J + 4lg + r]          (A operand, rows i)
  // dac[a][I] (I >= t): lane holds beta_i dAkk[16I + 4lg + r][16t + l16]   (A operand, rows j)
  uint2 darh[2][4], darl[2][4], dach[2][4], dacl[2][4];
  {
    // v_new rows of the wave's two token blocks, requested together; the lower half of the
    // chunk (blocks 0, 1) is handed to the upper waves through LDS (the pass planes' space,
    // unused until the channel passes), so no wave reads a row block from HBM twice
    uint4 oraw[2][VC][2];
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      const int j = 16 * (2 * tp + a) + l16;
#pragma unroll
      for (int vc = 0; vc < VC; ++vc) {
        const int v0 = 32 * vc + 8 * lg;
        const uint32_t o = (j < nval && v0 < V) ? ((uint32_t)j * rowV + v0) * 4u : kOOB;
        oraw[a][vc][0] = bld128(Rvn, o, 0);
        oraw[a][vc][1] = bld128(Rvn, o == kOOB ? kOOB : o + 16u, 0);
      }
    }
    bf16x8 vth[2][VC], vtl[2][VC];
#pragma unroll
    for (int a = 0; a < 2; ++a) {
#pragma unroll
      for (int vc = 0; vc < VC; ++vc) {
        float x[4], y[4];
        unpack4(oraw[a][vc][0], x);
        unpack4(oraw[a][vc][1], y);
        uint32_t hh[4], ll[4];
        split_bf16x2(x[0], x[1], hh[0], ll[0]);
        split_bf16x2(x[2], x[3], hh[1], ll[1]);
        split_bf16x2(y[0], y[1], hh[2], ll[2]);
        split_bf16x2(y[2], y[3], hh[3], ll[3]);
        vth[a][vc] = __builtin_bit_cast(bf16x8, make_uint4(hh[0], hh[1], hh[2], hh[3]));
        vtl[a][vc] = __builtin_bit_cast(bf16x8, make_uint4(ll[0], ll[1], ll[2], ll[3]));
      }
    }
    static_assert(32 * LP * 2 <= 2 * KH * LT * 2, "rows 0..31 must fit the pass planes");
    const Plane PL{sK1t, sK2t, LP};             // v_new rows 0..31, hi / lo
    if (tp == 0 && kb == 0) {
#pragma unroll
      for (int a = 0; a < 2; ++a) {
#pragma unroll
        for (int vc = 0; vc < VC; ++vc) {
          *(bf16x8*)(PL.hi + (16 * a + l16) * LP + 32 * vc + 8 * lg) = vth[a][vc];
          *(bf16x8*)(PL.lo + (16 * a + l16) * LP + 32 * vc + 8 * lg) = vtl[a][vc];
        }
      }
    }
    __syncthreads();  // rows 0..31 visible
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      const int t = 2 * tp + a;
      bf16x8 pth[VC], ptl[VC];
#pragma unroll
      for (int vc = 0; vc < VC; ++vc) {
        pth[vc] = PP.hi8(16 * t + l16, 32 * vc + 8 * lg);
        ptl[vc] = PP.lo8(16 * t + l16, 32 * vc + 8 * lg);
      }
#pragma unroll
      for (int J = 0; J < 4; ++J) {
        darh[a][J] = darl[a][J] = dach[a][J] = dacl[a][J] = make_uint2(0u, 0u);
        if (J <= t) {
          f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int vc = 0; vc < VC; ++vc) {
            bf16x8 ah, al;
            if (J == t) { ah = vth[a][vc]; al = vtl[a][vc]; }
            else if (J == 2 * tp) { ah = vth[0][vc]; al = vtl[0][vc]; }
            else { ah = PL.hi8(16 * J + l16, 32 * vc + 8 * lg); al = PL.lo8(16 * J + l16, 32 * vc + 8 * lg); }
            s = mma<true, true>(s, ah, al, pth[vc], ptl[vc]);
          }
          // s = sum_v vn[j][v] P[i][v] at (j = 16J + 4lg + r, i = 16t + l16)
          const int i = 16 * t + l16;
#pragma unroll
          for (int r = 0; r < 4; ++r) s[r] = (i > 16 * J + 4 * lg + r) ? -s[r] : 0.f;
          acc_to_bf16x4(s, darh[a][J], darl[a][J]);
        }
        if (J >= t) {
          f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int vc = 0; vc < VC; ++vc)
            s = mma<true, true>(s, PP.hi8(16 * J + l16, 32 * vc + 8 * lg), PP.lo8(16 * J + l16, 32 * vc + 8 * lg),
                                vth[a][vc], vtl[a][vc]);
          // s = sum_v P[i][v] vn[j][v] at (i = 16J + 4lg + r, j = 16t + l16)
          const int j = 16 * t + l16;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int i = 16 * J + 4 * lg + r;
            s[r] = i > j ? -sBeta[i] * s[r] : 0.f;
          }
          acc_to_bf16x4(s, dach[a][J], dacl[a][J]);
        }
      }
    }
  }

  // ---------------- channel passes: wave (kb, tp) -> channels cb + 16kb.., tokens of blocks 2tp, 2tp+1
  const rsrc_t Rdk = make_rsrc_rows(p.dk_wy, e0, nrows, K);
  const rsrc_t Rdg = make_rsrc_rows(p.dg_wy, e0, nrows, K);
  const int ch = tid & 31, sg = tid >> 5;
  float dbk_acc[2][4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};   // per (a, r): sum over channels
#pragma unroll 1
  for (int ps = 0; ps < NPS; ++ps) {
    const int cb = ps * KH;
    const int kl = 16 * kb + l16;        // channel in the pass of this lane's result column
    const int kk = cb + kl;
    // this pass's S rows kk (B operand of dbk), issued before the staging
    uint4 sraw[VC][2];
#pragma unroll
    for (int vc = 0; vc < VC; ++vc) {
      const int v0 = 32 * vc + 8 * lg;
      const uint32_t o = (kk < K && v0 < V) ? ((uint32_t)kk * V + v0) * 4u : kOOB;
      sraw[vc][0] = bld128(Rh, o, 0);
      sraw[vc][1] = bld128(Rh, o == kOOB ? kOOB : o + 16u, 0);
    }
    // ---- staging: thread = (channel ch, rows 8sg..8sg+7)
    {
      const int kc = cb + ch;
      float G[8], kv[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int r = 8 * sg + i;
        const bool ok = kc < K && r < nval;
        const uint32_t off = (uint32_t)r * rowK + kc;
        if constexpr (ES == 4) {
          kv[i] = __uint_as_float(bld32(Rk, ok ? off * 4u : kOOB, 0));
        } else {
          const uint32_t wd = bld32(Rk, ok ? (off & ~1u) * 2u : kOOB, 0);
          kv[i] = (off & 1u) ? __uint_as_float(wd & 0xffff0000u) : __uint_as_float(wd << 16);
        }
        const float x = __uint_as_float(bld32(Rg, ok ? off * 4u : kOOB, 0));
        G[i] = x * kLog2e + (i > 0 ? G[i - 1] : 0.f);
      }
      sTot[sg * KH + ch] = G[7];          // sTot is last read before the previous pass's planes barrier
      __syncthreads();
      float pre = 0.f, gam = 0.f;
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const float t = sTot[s * KH + ch];
        if (s < sg) pre += t;
        gam += t;
      }
      const float gmv = 0.5f * gam;
      if (sg == 0) sGm[ch] = gmv;
      float k1[8], k2[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        G[i] += pre;
        sG[(8 * sg + i) * LG + ch] = G[i];
        k1[i] = kv[i] * fast_exp2(G[i] - gmv);
        k2[i] = kv[i] * fast_exp2(gmv - G[i]);
      }
      put_n<true, 8>(PK1t, ch, 8 * sg, k1);
      put_n<true, 8>(PK2t, ch, 8 * sg, k2);
    }
    __syncthreads();  // pass planes, sG, sGm visible

    bf16x8 bh[VC], bl[VC];              // S rows kk, split once for both token blocks
#pragma unroll
    for (int vc = 0; vc < VC; ++vc) {
      float a[4], b[4];
      unpack4(sraw[vc][0], a);
      unpack4(sraw[vc][1], b);
      uint32_t h4[4], l4[4];
      split_bf16x2(a[0], a[1], h4[0], l4[0]);
      split_bf16x2(a[2], a[3], h4[1], l4[1]);
      split_bf16x2(b[0], b[1], h4[2], l4[2]);
      split_bf16x2(b[2], b[3], h4[3], l4[3]);
      bh[vc] = __builtin_bit_cast(bf16x8, make_uint4(h4[0], h4[1], h4[2], h4[3]));
      bl[vc] = __builtin_bit_cast(bf16x8, make_uint4(l4[0], l4[1], l4[2], l4[3]));
    }
    const float gmv = sGm[kl];
    float dgr[2][4], dkr[2][4];
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      const int t = 2 * tp + a;
      // dbk: -sum_v P[j][v] S[kk][v]
      f32x4 db = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int vc = 0; vc < VC; ++vc)
        db = mma<true, true>(db, PP.hi8(16 * t + l16, 32 * vc + 8 * lg), PP.lo8(16 * t + l16, 32 * vc + 8 * lg),
                             bh[vc], bl[vc]);
      // Y1 (rows i of block t) and Y2 (rows j of block t), contraction over tokens
      f32x4 y1 = {0.f, 0.f, 0.f, 0.f}, y2 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int Pp = 0; Pp < 2; ++Pp) {
        const int P0 = 2 * Pp, P1 = 2 * Pp + 1;
        if (P0 <= t)
          y1 = mma<true, true>(y1, cat44(darh[a][P0], darh[a][P1]), cat44(darl[a][P0], darl[a][P1]),
                               PK2t.hi44(kl, 16 * P0 + 4 * lg, 16 * P1 + 4 * lg),
                               PK2t.lo44(kl, 16 * P0 + 4 * lg, 16 * P1 + 4 * lg));
        if (P1 >= t)
          y2 = mma<true, true>(y2, cat44(dach[a][P0], dach[a][P1]), cat44(dacl[a][P0], dacl[a][P1]),
                               PK1t.hi44(kl, 16 * P0 + 4 * lg, 16 * P1 + 4 * lg),
                               PK1t.lo44(kl, 16 * P0 + 4 * lg, 16 * P1 + 4 * lg));
      }
      // epilogue: lane holds (token 16t + 4lg + r, channel kk)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int tok = 16 * t + 4 * lg + r;
        const bool ok = kk < K && tok < nval;
        const uint32_t off = (uint32_t)tok * rowK + kk;
        float kv;
        if constexpr (ES == 4) {
          kv = __uint_as_float(bld32(Rk, ok ? off * 4u : kOOB, 0));
        } else {
          const uint32_t wd = bld32(Rk, ok ? (off & ~1u) * 2u : kOOB, 0);
          kv = (off & 1u) ? __uint_as_float(wd & 0xffff0000u) : __uint_as_float(wd << 16);
        }
        const float Gt = sG[tok * LG + kl];
        const float e = fast_exp2(Gt);
        const float b = sBeta[tok];
        const float dbkv = -db[r];
        const float Y1 = y1[r] * fast_exp2(Gt - gmv);
        const float Y2 = y2[r] * fast_exp2(gmv - Gt);
        dkr[a][r] = b * e * dbkv + b * Y1 + Y2;
        dgr[a][r] = b * e * kv * dbkv + b * kv * Y1 - kv * Y2;
        dbk_acc[a][r] += e * kv * dbkv + kv * Y1;
      }
    }
    // reverse in-chunk cumsum of dG over this wave's 32 tokens (in-lane, lane groups, block
    // 2tp+1 into 2tp), then tokens 32..63 into the first token pair through LDS
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      dgr[a][2] += dgr[a][3];
      dgr[a][1] += dgr[a][2];
      dgr[a][0] += dgr[a][1];
      const float tot = dgr[a][0];
      const float t1 = __shfl(tot, l16 + 16, 64);
      const float t2 = __shfl(tot, l16 + 32, 64);
      const float t3 = __shfl(tot, l16 + 48, 64);
      const float add = (lg < 1 ? t1 : 0.f) + (lg < 2 ? t2 : 0.f) + (lg < 3 ? t3 : 0.f);
#pragma unroll
      for (int r = 0; r < 4; ++r) dgr[a][r] += add;
    }
    {
      const float blk1 = __shfl(dgr[1][0], l16, 64);       // total of block 2tp + 1
#pragma unroll
      for (int r = 0; r < 4; ++r) dgr[0][r] += blk1;
    }
    if (tp == 1 && lg == 0) sBlk[kb * 16 + l16] = dgr[0][0];   // total of tokens 32..63
    __syncthreads();  // block totals visible
    const float add = tp == 0 ? sBlk[kb * 16 + l16] : 0.f;
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      const int t = 2 * tp + a;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int tok = 16 * t + 4 * lg + r;
        const uint32_t off = (kk < K && tok < nval) ? ((uint32_t)tok * rowK + kk) * 4u : kOOB;
        bst32(Rdg, __float_as_uint(dgr[a][r] + add), off, 0);
        bst32(Rdk, __float_as_uint(dkr[a][r]), off, 0);
      }
    }
  }

  // ---------------- dbeta: channel sums (16 lanes, two channel halves), plus sum_v v P
#pragma unroll
  for (int a = 0; a < 2; ++a) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) dbk_acc[a][r] += __shfl_xor(dbk_acc[a][r], o, 64);
    }
  }
  if (l16 == 0) {
#pragma unroll
    for (int a = 0; a < 2; ++a) {
#pragma unroll
      for (int r = 0; r < 4; ++r) sDbk[kb * C + 16 * (2 * tp + a) + 4 * lg + r] = dbk_acc[a][r];
    }
  }
  __syncthreads();
  if (tid < C) {
    const float x = sDbk[tid] + sDbk[C + tid] + sDbv[tid] + sDbv[C + tid] + sDbv[2 * C + tid] + sDbv[3 * C + tid];
    const rsrc_t Rdb = make_rsrc_rows(p.dbeta, e0, nrows, 1);
    bst32(Rdb, __float_as_uint(x), tid < nval ? (uint32_t)tid * H * 4u : kOOB, 0);
  }
}

template <typename TIn>
hipError_t launch_kda_wy(const KdaWyParams& p, hipStream_t s) {
  const int kp = p.K <= 32 ? 32 : (p.K <= 64 ? 64 : 128);
  const int vp = p.V <= 32 ? 32 : (p.V <= 64 ? 64 : 128);
  dim3 grid(p.total * p.H), block(256);
#define TOPS_KWY(KPV, VPV) \
  if (kp == KPV && vp == VPV) { hipLaunchKernelGGL((kda_wy_kernel<TIn, KPV, VPV>), grid, block, 0, s, p); return hipGetLastError(); }
  TOPS_KWY(32, 32) TOPS_KWY(32, 64) TOPS_KWY(32, 128)
  TOPS_KWY(64, 32) TOPS_KWY(64, 64) TOPS_KWY(64, 128)
  TOPS_KWY(128, 32) TOPS_KWY(128, 64) TOPS_KWY(128, 128)
#undef TOPS_KWY
  return hipErrorInvalidValue;
}

template hipError_t launch_kda_wy<uint16_t>(const KdaWyParams&, hipStream_t);
template hipError_t launch_kda_wy<float>(const KdaWyParams&, hipStream_t);

}  // namespace tops
