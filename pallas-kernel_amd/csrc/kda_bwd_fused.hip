// KDA backward, chunk-parallel stage for gfx950: the WY backward and dq / dk / dg in one
// workgroup per (chunk, head), for bf16 inputs.
//
// The same arithmetic as the pair kda_wy_kernel (kda_wy.hip: P = T^T dv_new, dv, dbeta and
// the WY parts of dk and of the gate gradient) + gla_dqkg_kernel<bf16, fp32 v> (gla_dqkg.hip:
// dq, dk, dg of the GLA-shaped terms with v := v_new), which replace the reference's
// chunk_kda_bwd stages K17-K20 (tops/ops/kda/chunk_bwd.py:19-141, 655-832; oracle
// tops/cpu/ops/kda/chunk_bwd.py:525-668).  Here:
//   * 8 waves: waves 0-3 (group A) run the dq / dk / dg passes of 32 channels, waves 4-7
//     (group B) the WY passes over the same channels, on shared LDS planes: v_new (bf16
//     hi / lo), dO, the pass's q~ / k~ / k^ (k~ = k 2^(Gm - G), k^ = k 2^(G - Gm)) and its
//     gate cumsum, all staged by group A (B reads no q / k / g rows of its own);
//   * the WY parts of dk and of the gate gradient go from group B to group A through an
//     LDS exchange per pass, not through two [B,T,H,K] fp32 tensors in HBM, and are added
//     before A's reverse token cumsum (the cumsum is linear);
//   * each pass's state checkpoint rows are read by both groups in the same pass (the
//     second read hits L2), and v_new is read once.
// Group B computes its products with the operands exchanged, so its results sit in group
// A's result layout: lane holds (token 16 t + l16, channels 4 lg + r of a 16-channel block).
// Both groups run the same barrier sequence.
#include <type_traits>

#include "kda.h"
#include "tops_common.h"

namespace tops {

// C16: fp16 checkpoints (KdaBwdParams::ckpt16), 8 values per 16-byte load, scaled on the way
template <int KP, int VP, bool C16>
__global__ __launch_bounds__(512, 1) void kda_bwd_fused_kernel(KdaBwdParams p) {
  constexpr int C = kChunk;
  constexpr int KH = 32;                 // channels per pass
  constexpr int NPS = KP / KH;
  constexpr int VC = VP / 32;
  constexpr int NVB = VP / 16;           // 16-wide V blocks
  constexpr int LV = VP + 8, LT = C + 8, LG = KH + 4, LP = VP + 8, LX = KH + 4;
  constexpr int NPC = VP / 8;            // 16-byte pieces of a dO row (bf16)
  constexpr int NPT = C * NPC / 256;
  constexpr int NPCV = VP / 4;           // 16-byte pieces of a v_new row (fp32)
  constexpr int NPTV = C * NPCV / 256;
  static_assert(KP % KH == 0 && VP % 32 == 0 && NPT >= 1 && NPTV >= 1, "KP, VP: 32, 64 or 128");
  typedef Words<uint16_t> Wd;

  __shared__ __attribute__((aligned(16))) uint16_t sV[2 * C * LV];     // v_new hi / lo
  __shared__ __attribute__((aligned(16))) uint16_t sD[C * LV];         // dO
  __shared__ __attribute__((aligned(16))) uint16_t sQT[2 * KH * LT];   // q~^T of the pass
  __shared__ __attribute__((aligned(16))) uint16_t sKT[2 * KH * LT];   // k~^T = k 2^(Gm - G)
  __shared__ __attribute__((aligned(16))) uint16_t sK1[2 * KH * LT];   // k 2^(G - Gm) (WY)
  __shared__ __attribute__((aligned(16))) uint16_t sP[2 * C * LP];     // P = T^T dv_new
  __shared__ __attribute__((aligned(16))) float sG[C * LG];            // gate cumsum of the pass
  // exchange of the WY parts of dk and dG (per pass); before the passes it holds dAkk (fp32)
  __shared__ __attribute__((aligned(16))) float sX[2 * C * LX];
  __shared__ __attribute__((aligned(16))) float sTot[8 * KH];
  __shared__ __attribute__((aligned(16))) float sGm[KH];
  __shared__ __attribute__((aligned(16))) float sGam[KH];
  __shared__ __attribute__((aligned(16))) float sZk[2 * KH];
  __shared__ __attribute__((aligned(16))) float sHdh[KH];
  __shared__ __attribute__((aligned(16))) float sBlk[KH];
  __shared__ float sBeta[C];
  __shared__ float sDbv[4 * C];          // per B wave: sum_v v P over its V blocks
  __shared__ float sDbk[2 * C];          // per channel block: sum_d (2^G k dbk + k Y1)

  float* const sXk = sX;                 // exchange: WY dk
  float* const sXg = sX + C * LX;        // exchange: WY dG
  constexpr int LM = C + 4;
  float* const sM = sX;                  // dAkk[i][j], row i (before the passes)
  static_assert(C * LM <= 2 * C * LX, "dAkk fits the exchange planes");
  const Plane Pv{sV, sV + C * LV, LV};
  const Plane Pd{sD, sD, LV};
  const Plane Pqt{sQT, sQT + KH * LT, LT};
  const Plane Pkt{sKT, sKT + KH * LT, LT};
  const Plane Pk1{sK1, sK1 + KH * LT, LT};
  const Plane PP{sP, sP + C * LP, LP};

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool grpB = wave >= 4;           // wave-uniform
  const int lw = wave & 3;               // wave within the group
  const int tq = tid & 255;              // thread within the group
  const int kb = lw & 1, rh = lw >> 1;   // channel block of the pass, token-block pair
  const int l16 = lane & 15, lg = lane >> 4;
  const int hh = blockIdx.x % p.H;
  const int gc = blockIdx.x / p.H;
  const int H = p.H, K = p.K, V = p.V;
  const float scale = p.scale;

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
  const long long nrows = (long long)p.B * p.T * H;
  const uint32_t rowK = (uint32_t)(H * K), rowV = (uint32_t)(H * V);
  const rsrc_t Rq = make_rsrc_rows((const uint16_t*)p.q, e0, nrows, K);
  const rsrc_t Rk = make_rsrc_rows((const uint16_t*)p.k, e0, nrows, K);
  const rsrc_t Rg = make_rsrc_rows(p.g, e0, nrows, K);
  const long long KVB = (long long)K * V * (C16 ? 2 : 4);
  const size_t so = ((size_t)gc * H + hh) * K * V;
  const rsrc_t Rh = C16 ? make_rsrc((const uint16_t*)p.hs + so, KVB) : make_rsrc(p.hs + so, KVB);
  // C16: the factors of this chunk's two 64-column tiles (h and dh)
  float hsc[2] = {1.f, 1.f}, dhsc[2] = {1.f, 1.f};
  if constexpr (C16) {
    const int nv = cdiv(V, 64);
    const size_t fo = ((size_t)gc * H + hh) * nv;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      if (t < nv) {
        hsc[t] = p.hs_scale[fo + t];
        dhsc[t] = p.dhs_scale[fo + t];
      }
    }
  }

  // ---------------- group A's staging registers: thread = (channel ch, rows 8 sg .. 8 sg + 7)
  const int ch = tq & 31, sg = tq >> 5;
  const uint32_t hsh = (ch & 1) ? 0u : 16u;
  auto elem = [&](uint32_t w) { return __uint_as_float((w << hsh) & 0xffff0000u); };
  uint32_t rq[8], rk[8];
  float rg[8];
  auto load_pass = [&](int ps) {
    const int kc = ps * KH + ch;
    const bool ok = kc < K;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = 8 * sg + i;
      const bool v_ = ok && r < nval;
      const uint32_t off = (uint32_t)r * rowK + kc;
      rq[i] = bld32(Rq, v_ ? (off & ~1u) * 2u : kOOB, 0);
      rk[i] = bld32(Rk, v_ ? (off & ~1u) * 2u : kOOB, 0);
      rg[i] = __uint_as_float(bld32(Rg, v_ ? off * 4u : kOOB, 0));
    }
  };
  // a lane's 8 values of state row kk = 32 ps + 16 kb + l16, v = 32 vc + 8 lg + 0..7
  const int kl = 16 * kb + l16;
  auto load_state = [&](const rsrc_t& R, uint4 (&raw)[VC][2], int ps) {
    const int kk = ps * KH + kl;
#pragma unroll
    for (int vc = 0; vc < VC; ++vc) {
      const int v0 = 32 * vc + 8 * lg;
      const uint32_t o = (kk < K && v0 < V) ? ((uint32_t)kk * V + v0) * (C16 ? 2u : 4u) : kOOB;
      raw[vc][0] = bld128(R, o, 0);
      if constexpr (!C16) raw[vc][1] = bld128(R, o, 16);
    }
  };
  // the lane's 8 state values of value block vc (scaled back for fp16 checkpoints)
  auto state8 = [&](const uint4 (&raw)[VC][2], int vc, const float* sc, float* x) {
    if constexpr (C16) {
      unpack8_f16(raw[vc][0], x);
      const float f = sc[(32 * vc + 8 * lg) >> 6];
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] *= f;
    } else {
      unpack4(raw[vc][0], x);
      unpack4(raw[vc][1], x + 4);
    }
  };

  // ================================================================ the two groups
  // Each group runs its whole flow in its own function (runA / runB below), so that no value
  // of one group is live across the other group's code.  Both run the barriers P1, P2, P3, then
  // S1 .. S4 per channel pass, then E1.
  // A: dA tiles (registers, all passes).  dth[a][J] (row block 2rh + a, J <= it): lane holds
  // dA[16(2rh+a) + l16][16J + 4lg + r];  dah[a][J] (col block 2rh + a, J >= it): lane holds
  // dA[16J + 4lg + r][16(2rh+a) + l16].
  // B: dAkk tiles (registers, all passes).  dar[a][J] (J <= t): lane holds
  // dAkk[16t + l16][16J + 4lg + r];  dac[a][J] (J >= t): beta_i dAkk[16J + 4lg + r][16t + l16]
  constexpr int NVW = (NVB + 3) / 4;     // V blocks per B wave
  // ================================================================ channel passes
  const rsrc_t Rdh = C16 ? make_rsrc((const uint16_t*)p.dhs + so, KVB) : make_rsrc(p.dhs + so, KVB);
  const rsrc_t Rdq = make_rsrc_rows((uint16_t*)p.dq, e0, nrows, K);
  const rsrc_t Rdk = make_rsrc_rows((uint16_t*)p.dk, e0, nrows, K);
  const rsrc_t Rdg = make_rsrc_rows(p.dg, e0, nrows, K);
  // dAkk[i][j] = -sum_v P[i][v] v_new[j][v] for i > j (else 0), the 10 blocks (I >= J) of
  // 16 x 16 computed once each, by waves w and w + 8 of the workgroup, into sM
  auto dakk_blocks = [&]() {
#pragma unroll
    for (int rep_ = 0; rep_ < 2; ++rep_) {
      const int b = wave + 8 * rep_;
      if (b < 10) {
        const int I = b < 1 ? 0 : (b < 3 ? 1 : (b < 6 ? 2 : 3));
        const int J = b - I * (I + 1) / 2;
        f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int vc = 0; vc < VC; ++vc)
          s = mma<true, true>(s, PP.hi8(16 * I + l16, 32 * vc + 8 * lg), PP.lo8(16 * I + l16, 32 * vc + 8 * lg),
                              Pv.hi8(16 * J + l16, 32 * vc + 8 * lg), Pv.lo8(16 * J + l16, 32 * vc + 8 * lg));
        // lane holds (i = 16 I + 4 lg + r, j = 16 J + l16)
        const int j = 16 * J + l16;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = 16 * I + 4 * lg + r;
          sM[i * LM + j] = i > j ? -s[r] : 0.f;
        }
      }
    }
  };
  // ---------------- group A: dq / dk / dg
  auto runA = [&](auto RHc) {
  constexpr int rh = decltype(RHc)::value;   // token-block pair, a constant per instance
  uint2 dthh[2][4], dthl[2][4], dahh[2][4], dahl[2][4];
    // A: v_new (fp32, split into hi / lo) and dO planes ([C][V], V contiguous)
    const rsrc_t Rvn = make_rsrc_rows(p.vnew, e0, nrows, V);
    const rsrc_t Rd = make_rsrc_rows((const uint16_t*)p.dout, e0, nrows, V);
    uint4 pv[NPTV], pd[NPT];
#pragma unroll
    for (int i = 0; i < NPTV; ++i) {
      const int pc = tq + 256 * i, row = pc / NPCV, col = (pc % NPCV) * 4;
      pv[i] = bld128(Rvn, (row < nval && col < V) ? ((uint32_t)row * rowV + col) * 4u : kOOB, 0);
    }
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      const int pc = tq + 256 * i, row = pc / NPC, col = (pc % NPC) * 8;
      pd[i] = bld128(Rd, (row < nval && col < V) ? ((uint32_t)row * rowV + col) * 2u : kOOB, 0);
    }
#pragma unroll
    for (int i = 0; i < NPTV; ++i) {
      const int pc = tq + 256 * i, row = pc / NPCV, col = (pc % NPCV) * 4;
      float a[4];
      unpack4(pv[i], a);
      put_n<true, 4>(Pv, row, col, a);
    }
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      const int pc = tq + 256 * i, row = pc / NPC, col = (pc % NPC) * 8;
      *(uint4*)(Pd.hi + row * LV + col) = pd[i];
    }
    load_pass(0);
    __syncthreads();  // P1: v_new / dO planes and beta visible
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      const int B2 = 2 * rh + a;
#pragma unroll
      for (int J = 0; J < 4; ++J) {
        dthh[a][J] = dthl[a][J] = dahh[a][J] = dahl[a][J] = make_uint2(0u, 0u);
        if (J <= B2) {
          f32x4 t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int vc = 0; vc < VC; ++vc)
            t = mma<true, false>(t, Pv.hi8(16 * J + l16, 32 * vc + 8 * lg), Pv.lo8(16 * J + l16, 32 * vc + 8 * lg),
                                 Pd.hi8(16 * B2 + l16, 32 * vc + 8 * lg), Pd.hi8(16 * B2 + l16, 32 * vc + 8 * lg));
          const int i = 16 * B2 + l16;
#pragma unroll
          for (int r = 0; r < 4; ++r) t[r] = (16 * J + 4 * lg + r <= i) ? t[r] * scale : 0.f;
          acc_to_bf16x4(t, dthh[a][J], dthl[a][J]);
        }
        if (J >= B2) {
          f32x4 t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int vc = 0; vc < VC; ++vc)
            t = mma<false, true>(t, Pd.hi8(16 * J + l16, 32 * vc + 8 * lg), Pd.hi8(16 * J + l16, 32 * vc + 8 * lg),
                                 Pv.hi8(16 * B2 + l16, 32 * vc + 8 * lg), Pv.lo8(16 * B2 + l16, 32 * vc + 8 * lg));
          const int j = 16 * B2 + l16;
#pragma unroll
          for (int r = 0; r < 4; ++r) t[r] = (j <= 16 * J + 4 * lg + r) ? t[r] * scale : 0.f;
          acc_to_bf16x4(t, dahh[a][J], dahl[a][J]);
        }
      }
    }
    __syncthreads();  // P2: P plane visible
    dakk_blocks();
    __syncthreads();  // P3: dAkk visible
  
  uint4 hraw[VC][2], draw[VC][2];
#pragma unroll 1
  for (int ps = 0; ps < NPS; ++ps) {
    const int cb = ps * KH;
    load_state(Rh, hraw, ps);              // h rows of the inter products
    // ---- gate cumsum of the pass (thread: channel ch, rows 8sg..8sg+7); A publishes the
    // segment totals, both groups read them
    float G[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) G[i] = rg[i] * kLog2e + (i > 0 ? G[i - 1] : 0.f);
    sTot[sg * KH + ch] = G[7];
    __syncthreads();  // S1: segment totals visible
    float pre = 0.f, gam = 0.f;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const float t = sTot[s * KH + ch];
      if (s < sg) pre += t;
      gam += t;
    }
    const float gmv = 0.5f * gam;
    const int cl = 16 * kb + 4 * lg;       // first channel of the lane's result (in pass)
    const int kc = cb + cl;
    const bool chok = kc < K;
    {
      if (sg == 0) {
        sGm[ch] = gmv;
        sGam[ch] = gam;
      }
      float qt[8], kt[8], k1[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        G[i] += pre;
        sG[(8 * sg + i) * LG + ch] = G[i];
        const float e = fast_exp2(G[i] - gmv);
        qt[i] = elem(rq[i]) * e;
        k1[i] = elem(rk[i]) * e;
        kt[i] = elem(rk[i]) * fast_exp2(gmv - G[i]);
      }
      put_n<true, 8>(Pqt, ch, 8 * sg, qt);
      put_n<true, 8>(Pkt, ch, 8 * sg, kt);
      put_n<true, 8>(Pk1, ch, 8 * sg, k1);
      load_state(Rdh, draw, ps);
      __syncthreads();  // S2: planes, gate cumsum, Gm, Gamma visible
      float dkv[2][4], dgr[2][4];
      // ---- A: inter-chunk X^T += (alpha h) dO^T (the h rows were requested first)
      const float al = scale * fast_exp2(sGm[kl]);
      const float be = fast_exp2(sGam[kl] - sGm[kl]);
      f32x4 X[2], Wt[2], Wq[2];
      X[0] = X[1] = Wt[0] = Wt[1] = Wq[0] = Wq[1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int vc = 0; vc < VC; ++vc) {
        const int v0 = 32 * vc + 8 * lg;
        float hv[8];
        state8(hraw, vc, hsc, hv);
        uint32_t ah_[4], al_[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) split_bf16x2(al * hv[2 * e], al * hv[2 * e + 1], ah_[e], al_[e]);
        const bf16x8 Ah = __builtin_bit_cast(bf16x8, make_uint4(ah_[0], ah_[1], ah_[2], ah_[3]));
        const bf16x8 Al = __builtin_bit_cast(bf16x8, make_uint4(al_[0], al_[1], al_[2], al_[3]));
#pragma unroll
        for (int a = 0; a < 2; ++a) {
          const bf16x8 doh = Pd.hi8(16 * (2 * rh + a) + l16, v0);
          X[a] = mma<true, false>(X[a], Ah, Al, doh, doh);
        }
      }
      // ---- intra-chunk: X^T += k~^T dA^T, Wq^T = q~^T dA (LDS operands only: they cover the
      // wait for the dh rows)
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        const int B2 = 2 * rh + a;
#pragma unroll
        for (int Pp = 0; Pp < 2; ++Pp) {
          const int P0 = 2 * Pp, P1 = 2 * Pp + 1;
          if (P0 <= B2) {
            X[a] = mma<true, true>(X[a], Pkt.hi44(kl, 16 * P0 + 4 * lg, 16 * P1 + 4 * lg),
                                   Pkt.lo44(kl, 16 * P0 + 4 * lg, 16 * P1 + 4 * lg),
                                   cat44(dthh[a][P0], dthh[a][P1]), cat44(dthl[a][P0], dthl[a][P1]));
          }
          if (P1 >= B2) {
            Wq[a] = mma<true, true>(Wq[a], Pqt.hi44(kl, 16 * P0 + 4 * lg, 16 * P1 + 4 * lg),
                                    Pqt.lo44(kl, 16 * P0 + 4 * lg, 16 * P1 + 4 * lg),
                                    cat44(dahh[a][P0], dahh[a][P1]), cat44(dahl[a][P0], dahl[a][P1]));
          }
        }
      }
      // ---- inter-chunk W^T = (beta dh) v_new^T, and sum_v h dh (token-half-0 waves)
      float hd = 0.f;
#pragma unroll
      for (int vc = 0; vc < VC; ++vc) {
        const int v0 = 32 * vc + 8 * lg;
        float hv[8], dv[8];
        state8(hraw, vc, hsc, hv);
        state8(draw, vc, dhsc, dv);
        if (rh == 0) {
#pragma unroll
          for (int e = 0; e < 8; ++e) hd += hv[e] * dv[e];
        }
        uint32_t bh_[4], bl_[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) split_bf16x2(be * dv[2 * e], be * dv[2 * e + 1], bh_[e], bl_[e]);
        const bf16x8 Dh = __builtin_bit_cast(bf16x8, make_uint4(bh_[0], bh_[1], bh_[2], bh_[3]));
        const bf16x8 Dl = __builtin_bit_cast(bf16x8, make_uint4(bl_[0], bl_[1], bl_[2], bl_[3]));
#pragma unroll
        for (int a = 0; a < 2; ++a) {
          const int tr = 16 * (2 * rh + a) + l16;
          Wt[a] = mma<true, true>(Wt[a], Dh, Dl, Pv.hi8(tr, v0), Pv.lo8(tr, v0));
        }
      }
      // the next pass's q / k / g rows, requested once the state rows have been consumed
      if (ps + 1 < NPS) load_pass(ps + 1);
      // ---- sum_t k~ W_inter (this wave's tokens) and sum_v h dh (token-half-0 waves)
      {
        float z[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int a = 0; a < 2; ++a) {
          const int j = 16 * (2 * rh + a) + l16;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int cr = 16 * kb + 4 * lg + r;
            const float kv = bf16_to_f32(Pkt.hi[cr * LT + j]) + bf16_to_f32(Pkt.lo[cr * LT + j]);
            z[r] += kv * Wt[a][r];
          }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) z[r] = row16_sum(z[r]);
        if (l16 == 0) {
#pragma unroll
          for (int r = 0; r < 4; ++r) sZk[rh * KH + 16 * kb + 4 * lg + r] = z[r];
        }
        if (rh == 0) {
          hd += __shfl_xor(hd, 16, 64);
          hd += __shfl_xor(hd, 32, 64);
          if (lg == 0) sHdh[kl] = hd;
        }
      }
#pragma unroll
      for (int a = 0; a < 2; ++a) {
#pragma unroll
        for (int r = 0; r < 4; ++r) Wt[a][r] += Wq[a][r];
      }
      // ---- epilogue, part 1: lane holds (token 16(2rh+a) + l16, channels cb + cl + r)
      const float4 gm4 = *(const float4*)(sGm + cl);
      const float gmr[4] = {gm4.x, gm4.y, gm4.z, gm4.w};
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        const int tok = 16 * (2 * rh + a) + l16;
        const bool ok = chok && tok < nval;
        const uint32_t off = (uint32_t)tok * rowK + kc;
        const float4 g4 = *(const float4*)(sG + tok * LG + cl);
        const float gr[4] = {g4.x, g4.y, g4.z, g4.w};
        f32x4 dqv;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          dqv[r] = fast_exp2(gr[r] - gmr[r]) * X[a][r];
          dkv[a][r] = fast_exp2(gmr[r] - gr[r]) * Wt[a][r];
          const int pi = (cl + r) * LT + tok;
          const float qt = bf16_to_f32(Pqt.hi[pi]) + bf16_to_f32(Pqt.lo[pi]);
          const float kt = bf16_to_f32(Pkt.hi[pi]) + bf16_to_f32(Pkt.lo[pi]);
          dgr[a][r] = qt * X[a][r] - kt * Wt[a][r];
        }
        Wd::st4(Rdq, dqv, ok ? off * 2u : kOOB, 0);
      }
      __syncthreads();  // S3: the WY parts of the pass visible
      // ---- epilogue part 2: add the WY parts, store dk, reverse token cumsum of dg
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        const int tok = 16 * (2 * rh + a) + l16;
        const bool ok = chok && tok < nval;
        const uint32_t off = (uint32_t)tok * rowK + kc;
        const float4 xk = *(const float4*)(sXk + tok * LX + cl);
        const float4 xg = *(const float4*)(sXg + tok * LX + cl);
        f32x4 dk4 = {dkv[a][0] + xk.x, dkv[a][1] + xk.y, dkv[a][2] + xk.z, dkv[a][3] + xk.w};
        dgr[a][0] += xg.x; dgr[a][1] += xg.y; dgr[a][2] += xg.z; dgr[a][3] += xg.w;
        Wd::st4(Rdk, dk4, ok ? off * 2u : kOOB, 0);
      }
      // reverse cumsum over tokens: 16-lane suffix sums, block a=1's total into a=0, half 1
      // into half 0 (through sBlk)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float t1 = row16_sum(dgr[1][r]);
        dgr[0][r] = row16_suffix_sum(dgr[0][r]) + t1;
        dgr[1][r] = row16_suffix_sum(dgr[1][r]);
      }
      if (rh == 1 && l16 == 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r) sBlk[cl + r] = dgr[0][r];   // total of tokens 32..63
      }
      __syncthreads();  // S4: sZk, sHdh, sBlk visible
      float add[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        add[r] = fast_exp2(sGam[cl + r]) * sHdh[cl + r] + sZk[cl + r] + sZk[KH + cl + r];
        if (rh == 0) add[r] += sBlk[cl + r];
      }
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        const int tok = 16 * (2 * rh + a) + l16;
        const bool ok = chok && tok < nval;
        const uint32_t off = (uint32_t)tok * rowK + kc;
        bst128(Rdg, make_uint4(__float_as_uint(dgr[a][0] + add[0]), __float_as_uint(dgr[a][1] + add[1]),
                               __float_as_uint(dgr[a][2] + add[2]), __float_as_uint(dgr[a][3] + add[3])),
               ok ? off * 4u : kOOB, 0);
      }
    }
  }
  __syncthreads();  // E1
  };

  // ---------------- group B: the WY backward
  auto runB = [&](auto RHc) {
  constexpr int rh = decltype(RHc)::value;
  uint2 darh[2][4], darl[2][4], dach[2][4], dacl[2][4];
    // B: the P phase's global operands (dv_new^T and T^T fragments, v rows), requested first
    uint4 pdraw[NVW][2][2], ptraw[4][2][2];
    Wd::W4 pvraw[NVW][4];
    const rsrc_t Rtt = make_rsrc(p.tt + ((size_t)gc * H + hh) * C * C, (long long)C * C * 4);
    const rsrc_t Rdvt = make_rsrc(p.dvnt + ((size_t)gc * H + hh) * V * C, (long long)V * C * 4);
    const rsrc_t Rb = make_rsrc_rows(p.beta, e0, nrows, 1);
    const rsrc_t Rv = make_rsrc_rows((const uint16_t*)p.v, e0, nrows, V);
    const uint32_t braw = tq < C ? bld32(Rb, tq < nval ? (uint32_t)tq * H * 4u : kOOB, 0) : 0u;
#pragma unroll
    for (int u = 0; u < NVW; ++u) {
      const int vb = lw + 4 * u;
      const int v = 16 * vb + l16;
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        const uint32_t o = (vb < NVB && v < V) ? ((uint32_t)v * C + 32 * kc + 8 * lg) * 4u : kOOB;
        pdraw[u][kc][0] = bld128(Rdvt, o, 0);
        pdraw[u][kc][1] = bld128(Rdvt, o == kOOB ? kOOB : o + 16u, 0);
      }
#pragma unroll
      for (int I = 0; I < 4; ++I) {
        const int i = 16 * I + l16, col = 16 * vb + 4 * lg;
        pvraw[u][I] = Wd::ld4(Rv, (vb < NVB && i < nval && col < V) ? ((uint32_t)i * rowV + col) * 2u : kOOB, 0);
      }
    }
#pragma unroll
    for (int I = 0; I < 4; ++I) {
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        ptraw[I][kc][0] = ptraw[I][kc][1] = make_uint4(0u, 0u, 0u, 0u);
        if (kc == 1 || I < 2) {                 // T[i'][i] = 0 for i' < i
          const uint32_t o = ((uint32_t)(16 * I + l16) * C + 32 * kc + 8 * lg) * 4u;
          ptraw[I][kc][0] = bld128(Rtt, o, 0);
          ptraw[I][kc][1] = bld128(Rtt, o + 16u, 0);
        }
      }
    }
    if (tq < C) sBeta[tq] = __uint_as_float(braw);
    __syncthreads();  // P1: v_new / dO planes and beta visible
    {
    // B: P = T^T dv_new, tiles (vb, I) computed transposed: lane holds P[16I + l16][16vb + 4lg + r]
    const rsrc_t Rdv = make_rsrc_rows((uint16_t*)p.dv, e0, nrows, V);
    auto split16 = [](const uint4 (&r)[2], bf16x8& h, bf16x8& l) {
      float a[4], b[4];
      unpack4(r[0], a);
      unpack4(r[1], b);
      uint32_t hh4[4], ll4[4];
      split_bf16x2(a[0], a[1], hh4[0], ll4[0]);
      split_bf16x2(a[2], a[3], hh4[1], ll4[1]);
      split_bf16x2(b[0], b[1], hh4[2], ll4[2]);
      split_bf16x2(b[2], b[3], hh4[3], ll4[3]);
      h = __builtin_bit_cast(bf16x8, make_uint4(hh4[0], hh4[1], hh4[2], hh4[3]));
      l = __builtin_bit_cast(bf16x8, make_uint4(ll4[0], ll4[1], ll4[2], ll4[3]));
    };
    bf16x8 th[4][2], tl[4][2];
#pragma unroll
    for (int I = 0; I < 4; ++I) {
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) split16(ptraw[I][kc], th[I][kc], tl[I][kc]);
    }
    float dbv[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < NVW; ++u) {
      const int vb = lw + 4 * u;
      if (vb < NVB) {
        bf16x8 ah[2], al[2];
#pragma unroll
        for (int kc = 0; kc < 2; ++kc) split16(pdraw[u][kc], ah[kc], al[kc]);
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
          const uint32_t off = (i < nval && col < V) ? ((uint32_t)i * rowV + col) * 2u : kOOB;
          float vv[4];
          unpack4(pvraw[u][I], vv);
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
      if (lg == 0) sDbv[lw * C + 16 * I + l16] = x;
    }
    }
    __syncthreads();  // P2: P plane visible
    dakk_blocks();
    __syncthreads();  // P3: dAkk visible
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      const int t = 2 * rh + a;
#pragma unroll
      for (int J = 0; J < 4; ++J) {
        darh[a][J] = darl[a][J] = dach[a][J] = dacl[a][J] = make_uint2(0u, 0u);
        if (J <= t) {          // dAkk[16t + l16][16J + 4lg + r]
          const float4 m = *(const float4*)(sM + (16 * t + l16) * LM + 16 * J + 4 * lg);
          acc_to_bf16x4(f32x4{m.x, m.y, m.z, m.w}, darh[a][J], darl[a][J]);
        }
        if (J >= t) {          // beta_i dAkk[i = 16J + 4lg + r][16t + l16]
          f32x4 x;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int i = 16 * J + 4 * lg + r;
            x[r] = sBeta[i] * sM[i * LM + 16 * t + l16];
          }
          acc_to_bf16x4(x, dach[a][J], dacl[a][J]);
        }
      }
    }

  uint4 hraw[VC][2];
  float dbk_acc[2] = {0.f, 0.f};  // per token: sum over channels of 2^G k dbk + k Y1
#pragma unroll 1
  for (int ps = 0; ps < NPS; ++ps) {
    const int cb = ps * KH;
    load_state(Rh, hraw, ps);              // S rows of dbk
    // k of the epilogue's (token, 4 channels), requested with the state rows
    Wd::W4 kvraw[2];
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      const int tok = 16 * (2 * rh + a) + l16, kq = cb + 16 * kb + 4 * lg;
      kvraw[a] = Wd::ld4(Rk, (kq < K && tok < nval) ? ((uint32_t)tok * rowK + kq) * 2u : kOOB, 0);
    }
    __syncthreads();  // S1
    const int cl = 16 * kb + 4 * lg;       // first channel of the lane's result (in pass)
    {
      __syncthreads();  // S2: group A's planes (k~, k^), gate cumsum and Gm visible
      // ---- B: dbk' = S P^T, Y1' = k~^T dAkk^T, Y2' = k^^T (beta dAkk), all transposed:
      // lane holds (channel cb + cl + r, token 16t + l16)
      bf16x8 sh[VC], sl[VC];
#pragma unroll
      for (int vc = 0; vc < VC; ++vc) {
        float a4[8];
        state8(hraw, vc, hsc, a4);
        const float* b4 = a4 + 4;
        uint32_t h4[4], l4[4];
        split_bf16x2(a4[0], a4[1], h4[0], l4[0]);
        split_bf16x2(a4[2], a4[3], h4[1], l4[1]);
        split_bf16x2(b4[0], b4[1], h4[2], l4[2]);
        split_bf16x2(b4[2], b4[3], h4[3], l4[3]);
        sh[vc] = __builtin_bit_cast(bf16x8, make_uint4(h4[0], h4[1], h4[2], h4[3]));
        sl[vc] = __builtin_bit_cast(bf16x8, make_uint4(l4[0], l4[1], l4[2], l4[3]));
      }
      const float4 gm4 = *(const float4*)(sGm + cl);
      const float gmr[4] = {gm4.x, gm4.y, gm4.z, gm4.w};
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        const int t = 2 * rh + a;
        f32x4 db = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int vc = 0; vc < VC; ++vc)
          db = mma<true, true>(db, sh[vc], sl[vc], PP.hi8(16 * t + l16, 32 * vc + 8 * lg),
                               PP.lo8(16 * t + l16, 32 * vc + 8 * lg));
        f32x4 y1 = {0.f, 0.f, 0.f, 0.f}, y2 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int Pp = 0; Pp < 2; ++Pp) {
          const int P0 = 2 * Pp, P1 = 2 * Pp + 1;
          if (P0 <= t)
            y1 = mma<true, true>(y1, Pkt.hi44(kl, 16 * P0 + 4 * lg, 16 * P1 + 4 * lg),
                                 Pkt.lo44(kl, 16 * P0 + 4 * lg, 16 * P1 + 4 * lg),
                                 cat44(darh[a][P0], darh[a][P1]), cat44(darl[a][P0], darl[a][P1]));
          if (P1 >= t)
            y2 = mma<true, true>(y2, Pk1.hi44(kl, 16 * P0 + 4 * lg, 16 * P1 + 4 * lg),
                                 Pk1.lo44(kl, 16 * P0 + 4 * lg, 16 * P1 + 4 * lg),
                                 cat44(dach[a][P0], dach[a][P1]), cat44(dacl[a][P0], dacl[a][P1]));
        }
        const int tok = 16 * t + l16;
        float kv[4];
        unpack4(kvraw[a], kv);
        const float4 g4 = *(const float4*)(sG + tok * LG + cl);
        const float gt[4] = {g4.x, g4.y, g4.z, g4.w};
        const float b = sBeta[tok];
        float xk[4], xg[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float e = fast_exp2(gt[r]);
          const float dbkv = -db[r];
          const float Y1 = y1[r] * fast_exp2(gt[r] - gmr[r]);
          const float Y2 = y2[r] * fast_exp2(gmr[r] - gt[r]);
          xk[r] = b * e * dbkv + b * Y1 + Y2;
          xg[r] = b * e * kv[r] * dbkv + b * kv[r] * Y1 - kv[r] * Y2;
          dbk_acc[a] += e * kv[r] * dbkv + kv[r] * Y1;
        }
        *(float4*)(sXk + tok * LX + cl) = make_float4(xk[0], xk[1], xk[2], xk[3]);
        *(float4*)(sXg + tok * LX + cl) = make_float4(xg[0], xg[1], xg[2], xg[3]);
      }
      __syncthreads();  // S3
      __syncthreads();  // S4
        }
  }
  // ================================================================ dbeta (group B)
  {
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      float x = dbk_acc[a];
      x += __shfl_xor(x, 16, 64);
      x += __shfl_xor(x, 32, 64);
      if (lg == 0) sDbk[kb * C + 16 * (2 * rh + a) + l16] = x;
    }
  }
  __syncthreads();  // E1
  if (tq < C) {
    const float x = sDbk[tq] + sDbk[C + tq] + sDbv[tq] + sDbv[C + tq] + sDbv[2 * C + tq] + sDbv[3 * C + tq];
    const rsrc_t Rdb = make_rsrc_rows(p.dbeta, e0, nrows, 1);
    bst32(Rdb, __float_as_uint(x), tq < nval ? (uint32_t)tq * H * 4u : kOOB, 0);
  }
  };

  // one instance per token-block pair: the dA / dAkk tiles a wave never uses take no registers
  typedef std::integral_constant<int, 0> RH0;
  typedef std::integral_constant<int, 1> RH1;
  if (grpB) {
    if (rh == 0) runB(RH0{});
    else runB(RH1{});
  } else {
    if (rh == 0) runA(RH0{});
    else runA(RH1{});
  }
}

hipError_t launch_kda_bwd_fused(const KdaBwdParams& p, hipStream_t s) {
  const int kp = p.K <= 32 ? 32 : (p.K <= 64 ? 64 : 128);
  const int vp = p.V <= 32 ? 32 : (p.V <= 64 ? 64 : 128);
  dim3 grid(p.total * p.H), block(512);
#define TOPS_KBF(KPV, VPV) \
  if (kp == KPV && vp == VPV) { \
    if (p.ckpt16) hipLaunchKernelGGL((kda_bwd_fused_kernel<KPV, VPV, true>), grid, block, 0, s, p); \
    else hipLaunchKernelGGL((kda_bwd_fused_kernel<KPV, VPV, false>), grid, block, 0, s, p); \
    return hipGetLastError(); }
  TOPS_KBF(32, 32) TOPS_KBF(32, 64) TOPS_KBF(32, 128)
  TOPS_KBF(64, 32) TOPS_KBF(64, 64) TOPS_KBF(64, 128)
  TOPS_KBF(128, 32) TOPS_KBF(128, 64) TOPS_KBF(128, 128)
#undef TOPS_KBF
  return hipErrorInvalidValue;
}

}  // namespace tops
