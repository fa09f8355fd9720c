// GLA backward, chunk-parallel stage: dq, dk and the gate gradient dg for gfx950.
//
// Replaces the dq/dk/dg part of the reference's fused K4 (chunk_gla_bwd_fused_kernel,
// tops/ops/gla/chunk.py:1447-1581), following the oracle tops/cpu/ops/gla/chunk.py:357-466
// (chunk_gla_bwd_dqk_intra and chunk_gla_bwd_dqkg).
//
// One workgroup (4 wave64) per (chunk, head).  With G the in-chunk gate cumsum (log2
// units), Gamma = G[last], Gm = Gamma / 2, q~ = q 2^(G-Gm), k~ = k 2^(Gm-G), h_c the state
// before the chunk and dh_c the gradient w.r.t. the state after it, computed transposed
// (channel-major) so every result tile holds 4 consecutive channels of one token:
//     dA    = scale tril(dO v^T)
//     X^T   = (scale 2^Gm h_c) dO^T + k~^T dA^T           dq = 2^(G-Gm) X
//     W^T   = (2^(Gamma-Gm) dh_c) v^T + q~^T dA            dk = 2^(Gm-G) W
//     dg    = revcumsum_t(q dq - k dk) + 2^Gamma sum_v(h_c dh_c) + sum_t k~ W_inter
// The last term is sum_t k dk_inter of the oracle (k dk_inter = k~ W_inter).
//
// Channels are processed in passes of 32.  Wave w owns channel block (w & 1) of the
// pass and token blocks 2(w >> 1), 2(w >> 1) + 1.  The fp32 [K][V] checkpoints have V
// contiguous, the MFMA A-operand layout for a contraction over V, so each wave reads
// its 16 channels straight from global memory (L2) and splits them into bf16 hi/lo
// once.  The dA tiles (scale tril(dO v^T), bf16 hi/lo) are computed once per
// workgroup and stay in registers across passes.  The epilogue works in the MFMA
// result layout: the reverse token cumsum of dg is a 16-lane shuffle scan plus a
// cross-wave block total.  LDS holds the v / dO planes, the pass's gated q~^T / k~^T
// planes and its fp32 gate cumsum: < 70 KB, so two workgroups share a CU.
//
// RG (bf16, one gate per token: simple GLA's g [B,T,H] or g_gamma [H]): the gate cumsum G_t
// is the same for every channel, computed once per chunk, and 2^(G - Gm) factors out of q~
// and k~ per token: the intra products take exact q / k planes (no lo half) against dA
// tiles that carry the token factors (dA 2^(Gm - G_j) for dq, 2^(G_i - Gm) dA for dk), and
// dq, dk take their token's factor in the epilogue.
//
// PAIR (bf16 inputs, interleaved checkpoints): one workgroup of 8 waves takes the chunk
// pair (2i, 2i + 1), four waves per chunk, each half with its own LDS.  The buffer holds
// h_(2i) and dh_(2i+1) only; the missing states come from the partner's planes on MFMA,
//     dh_(2i)  = 2^Gamma' dh_(2i+1) + scale 2^Gm' (q~'^T dO')      (' = chunk 2i + 1)
//     h_(2i+1) = 2^Gamma h_(2i) + 2^(Gamma-Gm) (k~^T v)             (chunk 2i)
// the updates of the two sweeps, with dO' / v read transposed from the row-major planes
// (ds_read_b64_tr_b16).  That halves the checkpoint bytes written and read.  The results
// are [V-tile][channel] accumulator tiles, so every state row a lane holds is the runs
// v = 32vc + 4lg + 0..3 and 32vc + 16 + 4lg + 0..3: the contraction over v of the
// inter-chunk products takes dO / v in the same order.
#include <type_traits>

#include "gla_sweep.h"
#include "tops_common.h"

namespace tops {

// GK: the per-channel gate mode only (kGateK: GLA and KDA), compiled without gate-mode
// branches; !GK serves the per-token and constant gates chosen at run time.
// C16: the checkpoints are fp16 with one power-of-two factor per 64-column tile
// (SweepParams::ckpt16), read as 8 values per 16-byte load and scaled on the way.
template <typename TIn, typename TV, int KP, int VP, bool GK, bool PAIR, bool RG = false,
          bool C16 = false>
__global__ __launch_bounds__(PAIR ? 512 : 256, 2) void gla_dqkg_kernel(DqkgParams p) {
  constexpr int C = kChunk;
  constexpr int NG = PAIR ? 2 : 1;             // chunks per workgroup
  constexpr int KH = 32;                       // channels per pass
  constexpr int NPS = KP / KH;                 // passes
  constexpr int VC = VP / 32;
  constexpr bool SIN = !In<TIn>::kExactBf16;
  constexpr bool SINV = !In<TV>::kExactBf16;
  // fp16 inputs: split like fp32 ones, loaded as 2-byte elements like bf16 ones
  constexpr bool F16 = std::is_same<TIn, _Float16>::value;
  constexpr bool F16V = std::is_same<TV, _Float16>::value;
  constexpr int NPL = SIN ? 2 : 1;
  constexpr int NPLV = SINV ? 2 : 1;
  constexpr int ES = sizeof(TIn);
  constexpr int ESV = sizeof(TV);
  constexpr int LV = VP + 8, LT = C + 8, LG = KH + 4;
  constexpr int EP = 16 / ES;                  // elements per 16-byte piece of dO
  constexpr int NPC = VP / EP;                 // pieces per row
  constexpr int NPT = C * NPC / 256;           // pieces per thread
  constexpr int EPV = 16 / ESV;                // the same for v
  constexpr int NPCV = VP / EPV;
  constexpr int NPTV = C * NPCV / 256;
  static_assert(NPT >= 1 && C * NPC % 256 == 0, "VP must be 32, 64 or 128");
  static_assert(NPTV >= 1 && C * NPCV % 256 == 0, "VP must be 32, 64 or 128");
  static_assert(KP % KH == 0, "KP must be 32, 64 or 128");
  static_assert(!PAIR || (!SIN && !SINV), "the paired layout takes bf16 inputs");
  static_assert(!RG || (!GK && !PAIR && !SIN && !SINV), "RG: bf16, per-token gates, unpaired");
  static_assert(!C16 || !PAIR, "fp16 checkpoints: the unpaired layout");
  typedef Words<TIn> Wd;

  constexpr int ZV = NPLV * C * LV, ZD = NPL * C * LV, ZT = (RG ? 1 : 2) * KH * LT;
  __shared__ __attribute__((aligned(16))) uint16_t sV[NG * ZV];
  __shared__ __attribute__((aligned(16))) uint16_t sD[NG * ZD];
  __shared__ __attribute__((aligned(16))) uint16_t sQT[NG * ZT];
  __shared__ __attribute__((aligned(16))) uint16_t sKT[NG * ZT];
  __shared__ __attribute__((aligned(16))) float sG[RG ? 1 : NG * C * LG];  // gate cumsum of the pass
  __shared__ __attribute__((aligned(16))) float sRG[RG ? C : 1];          // RG: token gate cumsum
  __shared__ __attribute__((aligned(16))) float sTot[NG * 8 * KH];
  __shared__ __attribute__((aligned(16))) float sGm[NG * KH];
  __shared__ __attribute__((aligned(16))) float sGam[NG * KH];
  __shared__ __attribute__((aligned(16))) float sZk[NG * 2 * KH];
  __shared__ __attribute__((aligned(16))) float sHdh[NG * KH];
  __shared__ __attribute__((aligned(16))) float sBlk[NG * KH];
  // kGateS: per channel-block token sums (the fp32-v instantiation serves only kGateK, and
  // dropping this keeps it under 80 KB of LDS: two workgroups per CU)
  constexpr bool kScalarGate = std::is_same<TIn, TV>::value;
  __shared__ __attribute__((aligned(16))) float sDgS[kScalarGate ? NG * 2 * C : 1];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // The chunk of the pair is a compile-time index (GRP), so that every LDS address of the
  // body folds to an immediate offset; the two halves run the same barriers in the same order.
  // The token half (rh) is one too: the dA tiles a wave never uses then take no registers.
  auto run = [&](auto grp_tag, auto rh_tag) {
  constexpr int grp = decltype(grp_tag)::value;
  constexpr int rh = decltype(rh_tag)::value;  // token half
  const int tq = PAIR ? tid & 255 : tid;       // thread index within the chunk's four waves
  const int kb = wave & 1;                     // channel block of the pass
  const int l16 = lane & 15, lg = lane >> 4;
  const int hh = blockIdx.x % p.H;
  const int gc = PAIR ? 2 * (blockIdx.x / p.H) + grp : blockIdx.x / p.H;
  const int H = p.H, K = p.K, V = p.V;
  // row lengths of the channel- and value-indexed tensors (slices of wider heads)
  const int LDK = p.ldk > 0 ? p.ldk : K, LDV = p.ldv > 0 ? p.ldv : V;
  const float scale = p.scale;

  // this chunk's LDS (the partner's, for PAIR, at index pg)
  constexpr int pg = PAIR ? 1 - grp : 0;
  const Plane Pv{sV + grp * ZV, SINV ? sV + grp * ZV + C * LV : sV + grp * ZV, LV};
  const Plane Pd{sD + grp * ZD, SIN ? sD + grp * ZD + C * LV : sD + grp * ZD, LV};
  const Plane Pqt{sQT + grp * ZT, sQT + grp * ZT + (RG ? 0 : KH * LT), LT};
  const Plane Pkt{sKT + grp * ZT, sKT + grp * ZT + (RG ? 0 : KH * LT), LT};
  float* const gG = sG + (RG ? 0 : grp * C * LG);
  float* const gTot = sTot + grp * 8 * KH;
  float* const gGm = sGm + grp * KH;
  float* const gGam = sGam + grp * KH;
  float* const gZk = sZk + grp * 2 * KH;
  float* const gHdh = sHdh + grp * KH;
  float* const gBlk = sBlk + grp * KH;
  float* const gDgS = sDgS + (kScalarGate ? grp * 2 * C : 0);

  auto seq_of = [&](int x) { return p.cu_seqlens ? p.chunk_map[x] : x / cdiv(p.T, C); };
  // PAIR: the second chunk of the last pair may not exist (odd total): its waves take part
  // in the barriers with every access masked (nval = 0, empty state ranges)
  const bool present = !PAIR || gc < p.total;
  int n = 0, c = 0, L = 0, row0 = 0;
  if (present) {
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
  }
  // both chunks of the pair in one sequence: each recomputes its missing state from the other
  bool linked = false;
  if constexpr (PAIR) {
    const int c0 = 2 * (blockIdx.x / p.H);
    linked = c0 + 1 < p.total && seq_of(c0) == seq_of(c0 + 1);
  }
  const int t0 = c * C;
  const int nval = present ? min(C, L - t0) : 0;
  const size_t e0 = (size_t)(row0 + t0) * H + hh;
  const uint32_t rowK = (uint32_t)(H * LDK), rowV = (uint32_t)(H * LDV);
  // chunk-bounded resources (chunk_rsrc): the tokens past nval are out of range, so the
  // row loads and stores below carry no token mask
  const rsrc_t Rq = chunk_rsrc((const TIn*)p.q, e0, nval, (int)rowK, LDK);
  const rsrc_t Rk = chunk_rsrc((const TIn*)p.k, e0, nval, (int)rowK, LDK);
  const int gmode = GK ? kGateK : p.gate_mode;
  const rsrc_t Rg = gmode == kGateK ? chunk_rsrc(p.g, e0, nval, (int)rowK, LDK)
                                    : chunk_rsrc(p.g, e0, nval, H, 1);
  const float gam_h = gmode == kGateGamma ? p.g[hh] : 0.f;
  // kGateGammaK: this thread's constant of every pass (channel ps * KH + ch), read up front
  // through a range that is empty in the other modes.  The load is issued on every path: a
  // vector load inside the pass loop taken only in some modes would make the compiler's
  // waits for the prefetched rows conservative in all of them.
  float gck[NPS];
  if constexpr (!GK) {
    const rsrc_t Rgc = make_rsrc(gmode == kGateGammaK ? p.g + (size_t)hh * LDK : nullptr,
                                 gmode == kGateGammaK ? (long long)K * 4 : 0);
#pragma unroll
    for (int ps = 0; ps < NPS; ++ps) {
      const int c = ps * KH + (tq & 31);
      gck[ps] = __uint_as_float(bld32(Rgc, c < K ? (uint32_t)c * 4u : kOOB, 0));
    }
  }

  // ---------------- v / dO planes ([C][V], V contiguous)
  {
    const rsrc_t Rv = chunk_rsrc((const TV*)p.v, e0, nval, (int)rowV, LDV);
    const rsrc_t Rd = chunk_rsrc((const TIn*)p.dout, e0, nval, (int)rowV, LDV);
    uint4 pv[NPTV], pd[NPT];
#pragma unroll
    for (int i = 0; i < NPTV; ++i) {
      const int pc = tq + 256 * i, row = pc / NPCV, col = (pc % NPCV) * EPV;
      pv[i] = bld128(Rv, col < V ? ((uint32_t)row * rowV + col) * ESV : kOOB, 0);
    }
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      const int pc = tq + 256 * i, row = pc / NPC, col = (pc % NPC) * EP;
      pd[i] = bld128(Rd, col < V ? ((uint32_t)row * rowV + col) * ES : kOOB, 0);
    }
#pragma unroll
    for (int i = 0; i < NPTV; ++i) {
      const int pc = tq + 256 * i, row = pc / NPCV, col = (pc % NPCV) * EPV;
      if constexpr (!SINV) {
        *(uint4*)(Pv.hi + row * LV + col) = pv[i];
      } else if constexpr (F16V) {
        float a[8];
        unpack8_f16(pv[i], a);
        put_n<true, 8>(Pv, row, col, a);
      } else {
        float a[4];
        unpack4(pv[i], a);
        put_n<true, 4>(Pv, row, col, a);
      }
    }
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      const int pc = tq + 256 * i, row = pc / NPC, col = (pc % NPC) * EP;
      if constexpr (!SIN) {
        *(uint4*)(Pd.hi + row * LV + col) = pd[i];
      } else if constexpr (F16) {
        float b[8];
        unpack8_f16(pd[i], b);
        put_n<true, 8>(Pd, row, col, b);
      } else {
        float b[4];
        unpack4(pd[i], b);
        put_n<true, 4>(Pd, row, col, b);
      }
    }
  }

  // ---------------- RG: the token gate cumsum (log2 units) of the chunk, by the first wave
  if constexpr (RG) {
    if (tq < C) {
      float x = 0.f;
      if (gmode == kGateS) x = __uint_as_float(bld32(Rg, (uint32_t)tq * H * 4u, 0));
      else x = tq < nval ? gam_h : 0.f;
      x *= kLog2e;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const float y = __shfl_up(x, d, 64);
        if (lane >= d) x += y;
      }
      sRG[tq] = x;
    }
  }

  // ---------------- staging of a pass: thread = (channel ch, 8-row segment sg)
  const int ch = tq & 31, sg = tq >> 5;
  // raw words of the next pass's rows: fp32 elements, or (bf16) the aligned 32-bit word
  // holding the element, whose half is the same for every row and pass (row strides H*K
  // and pass offsets 32 are even: the half is ch's parity).  The element is taken out where
  // it is used, so that the prefetch is not waited for at its issue.
  uint32_t rq[8], rk[8];
  float rg[8];
  const uint32_t hsh = (ch & 1) ? 0u : 16u;
  auto elem = [&](uint32_t w) {
    if constexpr (F16) return f16_to_f32(hsh ? w : (w >> 16));
    else if constexpr (SIN) return __uint_as_float(w);
    else return __uint_as_float((w << hsh) & 0xffff0000u);
  };
  // gate element (row r, channel kc): per-channel [.., K], per-token [.., 1], or none (gamma)
  const bool gk_mode = GK || gmode == kGateK;
  const uint32_t gstr = gk_mode ? rowK * 4u : (uint32_t)H * 4u;
  const bool gload = !RG && (GK || gmode == kGateK || gmode == kGateS);   // the constant gates
                                                                         // (and RG) load nothing
  auto load_pass = [&](int ps) {
    const int kc = ps * KH + ch;
    const bool ok = kc < K;
    const uint32_t gcol = gk_mode ? (uint32_t)kc * 4u : 0u;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = 8 * sg + i;
      const bool v_ = ok;                 // rows past nval: out of the chunk's range
      const uint32_t off = (uint32_t)r * rowK + kc;
      if constexpr (SIN && !F16) {
        rq[i] = bld32(Rq, v_ ? off * 4u : kOOB, 0);
        rk[i] = bld32(Rk, v_ ? off * 4u : kOOB, 0);
      } else {
        rq[i] = bld32(Rq, v_ ? (off & ~1u) * 2u : kOOB, 0);
        rk[i] = bld32(Rk, v_ ? (off & ~1u) * 2u : kOOB, 0);
      }
      // one unconditional load whatever the gate mode (gamma loads nothing: out of range)
      if constexpr (RG) rg[i] = 0.f;
      else rg[i] = __uint_as_float(bld32(Rg, (v_ && gload) ? (uint32_t)r * gstr + gcol : kOOB, 0));
    }
  };
  load_pass(0);

  // ---------------- dA tiles (registers, all passes)
  // dth[a][J] (row block B = 2rh + a, J <= B): lane holds dA[16B + l16][16J + 4lg + r]
  // dah[a][I] (col block B = 2rh + a, I >= B): lane holds dA[16I + 4lg + r][16B + l16]
  __syncthreads();  // v / dO planes (and the RG token cumsum) visible
  // RG: Gamma and Gm of the chunk (rows past the sequence add nothing)
  const float rgam = RG ? sRG[C - 1] : 0.f, rgm = 0.5f * rgam;
  uint2 dthh[2][4], dthl[2][4], dahh[2][4], dahl[2][4];
#pragma unroll
  for (int a = 0; a < 2; ++a) {
    const int B2 = 2 * rh + a;
#pragma unroll
    for (int J = 0; J < 4; ++J) {
      dthh[a][J] = dthl[a][J] = dahh[a][J] = dahl[a][J] = make_uint2(0u, 0u);
      if (J <= B2) {
        f32x4 t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int vc = 0; vc < VC; ++vc) {
          const bf16x8 ah = Pv.hi8(16 * J + l16, 32 * vc + 8 * lg);
          const bf16x8 bh = Pd.hi8(16 * B2 + l16, 32 * vc + 8 * lg);
          bf16x8 al = ah, bl = bh;
          if constexpr (SINV) al = Pv.lo8(16 * J + l16, 32 * vc + 8 * lg);
          if constexpr (SIN) bl = Pd.lo8(16 * B2 + l16, 32 * vc + 8 * lg);
          t = mma<SINV, SIN>(t, ah, al, bh, bl);
        }
        const int i = 16 * B2 + l16;
#pragma unroll
        for (int r = 0; r < 4; ++r) t[r] = (16 * J + 4 * lg + r <= i) ? t[r] * scale : 0.f;
        if constexpr (RG) {
#pragma unroll
          for (int r = 0; r < 4; ++r) t[r] *= fast_exp2(rgm - sRG[16 * J + 4 * lg + r]);
        }
        acc_to_bf16x4(t, dthh[a][J], dthl[a][J]);
      }
      if (J >= B2) {
        f32x4 t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int vc = 0; vc < VC; ++vc) {
          const bf16x8 ah = Pd.hi8(16 * J + l16, 32 * vc + 8 * lg);
          const bf16x8 bh = Pv.hi8(16 * B2 + l16, 32 * vc + 8 * lg);
          bf16x8 al = ah, bl = bh;
          if constexpr (SIN) al = Pd.lo8(16 * J + l16, 32 * vc + 8 * lg);
          if constexpr (SINV) bl = Pv.lo8(16 * B2 + l16, 32 * vc + 8 * lg);
          t = mma<SIN, SINV>(t, ah, al, bh, bl);
        }
        const int j = 16 * B2 + l16;
#pragma unroll
        for (int r = 0; r < 4; ++r) t[r] = (j <= 16 * J + 4 * lg + r) ? t[r] * scale : 0.f;
        if constexpr (RG) {
#pragma unroll
          for (int r = 0; r < 4; ++r) t[r] *= fast_exp2(sRG[16 * J + 4 * lg + r] - rgm);
        }
        acc_to_bf16x4(t, dahh[a][J], dahl[a][J]);
      }
    }
  }

  // the state rows: h_c and dh_c, or for PAIR this chunk's checkpoint and the partner's
  // (linked) or the sequence's h0 / dht (not linked; NULL reads as zero)
  const long long KVB = (long long)K * LDV * 4;
  auto slot = [&](const float* b, int x) { return b + ((size_t)x * H + hh) * LDK * LDV; };
  rsrc_t Rh, Rdh;
  if constexpr (PAIR) {
    const float* other = nullptr;
    if (linked) other = slot(p.hs, grp == 0 ? gc + 1 : gc - 1);
    else if (present) {
      const float* b = grp == 0 ? p.dht : p.h0;
      other = b ? b + ((size_t)n * H + hh) * LDK * LDV : nullptr;
    }
    const rsrc_t Ro = make_rsrc(present ? slot(p.hs, gc) : nullptr, present ? KVB : 0);
    const rsrc_t Rx = make_rsrc(other, other ? KVB : 0);
    Rh = grp == 0 ? Ro : Rx;
    Rdh = grp == 0 ? Rx : Ro;
  } else {
    if constexpr (C16) {
      const size_t o = ((size_t)gc * H + hh) * LDK * LDV;
      Rh = make_rsrc((const uint16_t*)p.hs + o, (long long)K * LDV * 2);
      Rdh = make_rsrc((const uint16_t*)p.dhs + o, (long long)K * LDV * 2);
    } else {
      Rh = make_rsrc(slot(p.hs, gc), KVB);
      Rdh = make_rsrc(slot(p.dhs, gc), KVB);
    }
  }
  // C16: the factors of this chunk's two 64-column tiles (h and dh)
  float hsc[2] = {1.f, 1.f}, dhsc[2] = {1.f, 1.f};
  if constexpr (C16) {
    const int nv = cdiv(V, 64);
    const size_t so = ((size_t)gc * H + hh) * nv;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      if (t < nv) {
        hsc[t] = p.hs_scale[so + t];
        dhsc[t] = p.dhs_scale[so + t];
      }
    }
  }
  // the lane's 8 state values of value block vc as stored (fp16 checkpoints: before their
  // tile factor, which tfac gives; the 8 values v0 .. v0 + 7 lie in 64-column tile vc / 2)
  auto state8 = [&](const uint4 (&raw)[VC][2], int vc, float* x) {
    if constexpr (C16) {
      unpack8_f16(raw[vc][0], x);
    } else {
      unpack4(raw[vc][0], x);
      unpack4(raw[vc][1], x + 4);
    }
  };
  auto tfac = [&](const float* sc, int vc) { return C16 ? sc[vc >> 1] : 1.f; };
  const rsrc_t Rdq = chunk_rsrc((const TIn*)p.dq, e0, nval, (int)rowK, LDK);
  const rsrc_t Rdk = chunk_rsrc((const TIn*)p.dk, e0, nval, (int)rowK, LDK);
  // C16 calls take no slices and no WY parts (the launcher checks): their instance compiles
  // without those paths, and without the resources below
  constexpr bool kSlices = !C16;
  const rsrc_t Rdka = chunk_rsrc(kSlices ? p.dk_add : nullptr, e0, nval, (int)rowK, LDK);
  const rsrc_t Rdga = chunk_rsrc(kSlices ? p.dg_add : nullptr, e0, nval, (int)rowK, LDK);
  const rsrc_t Rdg = gmode == kGateS ? chunk_rsrc(p.dg, e0, nval, H, 1)
                                     : chunk_rsrc(gmode == kGateGamma ? nullptr : p.dg, e0, nval,
                                                  (int)rowK, LDK);
  // value slices: fp32 sums of dq / dk over the slices (acc_mode 1..3)
  const rsrc_t Rdq32 = chunk_rsrc(kSlices ? p.dq32 : nullptr, e0, nval, (int)rowK, LDK);
  const rsrc_t Rdk32 = chunk_rsrc(kSlices ? p.dk32 : nullptr, e0, nval, (int)rowK, LDK);
  if (kScalarGate && tq < 2 * C) gDgS[tq] = 0.f;

  // ---- the h / dh rows of a pass: a lane's 8 values of state row kk = 32 ps + 16 kb + l16,
  // v = v0 .. v0 + 7, or (PAIR) the runs v0 .. v0 + 3 and v0 + 16 .. v0 + 19 of the
  // accumulator-tile order.  h is requested at the start of the pass, so that its latency
  // overlaps the staging, dh just before the planes barrier.
  const int kl = 16 * kb + l16;            // channel of this lane's A-operand row (in pass)
  uint4 hraw[VC][2], draw[VC][2];
  auto load_state = [&](const rsrc_t& R, uint4 (&raw)[VC][2], int ps) {
    const int kk = ps * KH + kl;
    auto vrun = [&](int vc, int j) {
      const int v0 = PAIR ? 32 * vc + 16 * j + 4 * lg : 32 * vc + 8 * lg;
      return (kk < K && v0 < V) ? ((uint32_t)kk * LDV + v0) * (C16 ? 2u : 4u) : kOOB;
    };
#pragma unroll
    for (int vc = 0; vc < VC; ++vc) {
      if constexpr (PAIR) {
        raw[vc][0] = bld128(R, vrun(vc, 0), 0);
        raw[vc][1] = bld128(R, vrun(vc, 1), 0);
      } else if constexpr (C16) {
        raw[vc][0] = bld128(R, vrun(vc, 0), 0);
      } else {
        const uint32_t o = vrun(vc, 0);
        raw[vc][0] = bld128(R, o, 0);
        raw[vc][1] = bld128(R, o, 16);
      }
    }
  };

#pragma unroll 1
  for (int ps = 0; ps < NPS; ++ps) {
    const int cb = ps * KH;
    load_state(Rh, hraw, ps);
    constexpr bool kEarlyAdd = !kScalarGate;
    uint4 kadd[2], gadd[2];
    // ---- gate cumsum of the pass (thread: channel ch, rows 8sg..8sg+7); the constant gates
    // (g_gamma [H] or [H, K]) give every valid row the same value
    if constexpr (RG) {
      // exact q / k planes (hi only); the token factors live in the dA tiles and the epilogue
      float qt[8], kt[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        qt[i] = elem(rq[i]);
        kt[i] = elem(rk[i]);
      }
      put_n<false, 8>(Pqt, ch, 8 * sg, qt);
      put_n<false, 8>(Pkt, ch, 8 * sg, kt);
    } else {
    float gconst = gam_h;
    if constexpr (!GK) {
      if (gmode == kGateGammaK) gconst = gck[ps];
    }
    float G[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float x = rg[i];
      if constexpr (!GK) {
        if (!gload) x = (cb + ch < K && 8 * sg + i < nval) ? gconst : 0.f;
      }
      G[i] = x * kLog2e + (i > 0 ? G[i - 1] : 0.f);
    }
    // (no barrier before this write: sTot is last read before the previous pass's planes
    // barrier, and everything read after its final barrier is rewritten only after the next one)
    gTot[sg * KH + ch] = G[7];
    __syncthreads();
    float pre = 0.f, gam = 0.f;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const float t = gTot[s * KH + ch];
      if (s < sg) pre += t;
      gam += t;
    }
    const float gmv = 0.5f * gam;
    if (sg == 0) {
      gGm[ch] = gmv;
      gGam[ch] = gam;
    }
    {
      float qt[8], kt[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        G[i] += pre;
        gG[(8 * sg + i) * LG + ch] = G[i];
        qt[i] = elem(rq[i]) * fast_exp2(G[i] - gmv);
        kt[i] = elem(rk[i]) * fast_exp2(gmv - G[i]);
      }
      put_n<true, 8>(Pqt, ch, 8 * sg, qt);
      put_n<true, 8>(Pkt, ch, 8 * sg, kt);
    }
    }  // !RG
    // the next pass's q / k / g rows (PAIR: after the state rebuild, which needs the registers)
    if (!PAIR && ps + 1 < NPS) load_pass(ps + 1);
    // this pass's dh rows, in flight across the barrier
    load_state(Rdh, draw, ps);
    __syncthreads();  // planes, sG, sGm, sGam visible

    // ---- PAIR: the missing state from the partner chunk (see the header), accumulated onto
    // the partner-side state it starts from (scaled by 2^Gamma' / f, then the sum by f)
    if constexpr (PAIR) {
      auto rebuild = [&](uint4 (&xr)[VC][2], const uint16_t* zplane, const uint16_t* yplane,
                         float pre_s, float post_s) {
        const Plane Pz{(uint16_t*)zplane, (uint16_t*)zplane + KH * LT, LT};
        f32x4 acc[2 * VC];
#pragma unroll
        for (int vc = 0; vc < VC; ++vc)
#pragma unroll
          for (int j = 0; j < 2; ++j) acc[2 * vc + j] = __builtin_bit_cast(f32x4, xr[vc][j]) * pre_s;
        bf16x8 bh[2], bl[2];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          bh[ks] = Pz.hi8(kl, 32 * ks + 8 * lg);
          bl[ks] = Pz.lo8(kl, 32 * ks + 8 * lg);
        }
#pragma unroll
        for (int t = 0; t < 2 * VC; ++t) {
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) {
            const bf16x8 a = tr_read8(yplane, LV, 32 * ks, 16 * t, lane);
            acc[t] = mma<false, true>(acc[t], a, a, bh[ks], bl[ks]);
          }
        }
#pragma unroll
        for (int vc = 0; vc < VC; ++vc)
#pragma unroll
          for (int j = 0; j < 2; ++j) xr[vc][j] = __builtin_bit_cast(uint4, acc[2 * vc + j] * post_s);
      };
      if (linked) {
        const float pgam = sGam[pg * KH + kl], pgm = sGm[pg * KH + kl];
        if (grp == 0) {
          // dh_c = 2^Gamma' dh' + scale 2^Gm' (q~'^T dO')
          rebuild(draw, sQT + pg * ZT, sD + pg * ZD, fast_exp2(pgam - pgm) / scale,
                  scale * fast_exp2(pgm));
        } else {
          // h_c = 2^Gamma h'' + 2^(Gamma-Gm) (k~''^T v'')   (Gamma - Gm = Gm)
          rebuild(hraw, sKT + pg * ZT, sV + pg * ZV, fast_exp2(pgm), fast_exp2(pgam - pgm));
        }
      }
      if (ps + 1 < NPS) load_pass(ps + 1);
    }

    // ---- inter-chunk X^T += (alpha h) dO^T first: the h rows were requested a phase before
    // the dh rows
    const float al = scale * fast_exp2(RG ? rgm : gGm[kl]);
    const float be = fast_exp2(RG ? rgam - rgm : gGam[kl] - gGm[kl]);
    f32x4 X[2], Wt[2], Wq[2];
    X[0] = X[1] = Wt[0] = Wt[1] = Wq[0] = Wq[1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int vc = 0; vc < VC; ++vc) {
      const int v0 = 32 * vc + 8 * lg;
      float hv[8];
      state8(hraw, vc, hv);
      const float alt = al * tfac(hsc, vc);
      uint32_t ah_[4], al_[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) split_bf16x2(alt * hv[2 * e], alt * hv[2 * e + 1], ah_[e], al_[e]);
      const bf16x8 Ah = __builtin_bit_cast(bf16x8, make_uint4(ah_[0], ah_[1], ah_[2], ah_[3]));
      const bf16x8 Al = __builtin_bit_cast(bf16x8, make_uint4(al_[0], al_[1], al_[2], al_[3]));
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        const int B2 = 2 * rh + a;
        const int tr = 16 * B2 + l16;
        const bf16x8 doh = PAIR ? Pd.hi44(tr, 32 * vc + 4 * lg, 32 * vc + 16 + 4 * lg) : Pd.hi8(tr, v0);
        bf16x8 dol = doh;
        if constexpr (SIN) dol = Pd.lo8(16 * B2 + l16, v0);
        X[a] = mma<true, SIN>(X[a], Ah, Al, doh, dol);
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
          X[a] = mma<!RG, true>(X[a], Pkt.hi44(kl, 16 * P0 + 4 * lg, 16 * P1 + 4 * lg),
                                 Pkt.lo44(kl, 16 * P0 + 4 * lg, 16 * P1 + 4 * lg),
                                 cat44(dthh[a][P0], dthh[a][P1]), cat44(dthl[a][P0], dthl[a][P1]));
        }
        if (P1 >= B2) {
          Wq[a] = mma<!RG, true>(Wq[a], Pqt.hi44(kl, 16 * P0 + 4 * lg, 16 * P1 + 4 * lg),
                                  Pqt.lo44(kl, 16 * P0 + 4 * lg, 16 * P1 + 4 * lg),
                                  cat44(dahh[a][P0], dahh[a][P1]), cat44(dahl[a][P0], dahl[a][P1]));
        }
      }
    }
    // ---- inter-chunk W^T = (beta dh) v^T, and sum_v h dh (token-half-0 waves)
    float hd = 0.f;
#pragma unroll
    for (int vc = 0; vc < VC; ++vc) {
      const int v0 = 32 * vc + 8 * lg;
      float hv[8], dv[8];
      state8(hraw, vc, hv);
      state8(draw, vc, dv);
      if (rh == 0) {
        if constexpr (C16) {
          float s = 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) s += hv[e] * dv[e];
          hd += s * (hsc[vc >> 1] * dhsc[vc >> 1]);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) hd += hv[e] * dv[e];
        }
      }
      const float bet = be * tfac(dhsc, vc);
      uint32_t bh_[4], bl_[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) split_bf16x2(bet * dv[2 * e], bet * dv[2 * e + 1], bh_[e], bl_[e]);
      const bf16x8 Dh = __builtin_bit_cast(bf16x8, make_uint4(bh_[0], bh_[1], bh_[2], bh_[3]));
      const bf16x8 Dl = __builtin_bit_cast(bf16x8, make_uint4(bl_[0], bl_[1], bl_[2], bl_[3]));
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        const int B2 = 2 * rh + a;
        const int tr = 16 * B2 + l16;
        const bf16x8 vh = PAIR ? Pv.hi44(tr, 32 * vc + 4 * lg, 32 * vc + 16 + 4 * lg) : Pv.hi8(tr, v0);
        bf16x8 vl = vh;
        if constexpr (SINV) vl = Pv.lo8(16 * B2 + l16, v0);
        Wt[a] = mma<true, SINV>(Wt[a], Dh, Dl, vh, vl);
      }
    }
    // ---- the pass's WY parts of dk / dg (fp32-v instantiation only, the one the KDA
    // backward uses): requested once the inter-chunk products have freed their registers,
    // added in the epilogue
    if constexpr (kEarlyAdd) {
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        const int tok = 16 * (2 * rh + a) + l16;
        const int kc = cb + 16 * kb + 4 * lg;
        const uint32_t o = kc < K ? ((uint32_t)tok * rowK + kc) * 4u : kOOB;
        kadd[a] = bld128(Rdka, o, 0);
        gadd[a] = bld128(Rdga, o, 0);
      }
    }
    // ---- sum_t k~ W_inter (this wave's tokens) and sum_v h dh (token-half-0 waves)
    {
      float z[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        const int j = 16 * (2 * rh + a) + l16;
        const float fk = RG ? fast_exp2(rgm - sRG[j]) : 1.f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int cr = 16 * kb + 4 * lg + r;
          const float kv = RG ? bf16_to_f32(Pkt.hi[cr * LT + j]) * fk
                              : bf16_to_f32(Pkt.hi[cr * LT + j]) + bf16_to_f32(Pkt.lo[cr * LT + j]);
          z[r] += kv * Wt[a][r];
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) z[r] = row16_sum(z[r]);
      if (l16 == 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r) gZk[rh * KH + 16 * kb + 4 * lg + r] = z[r];
      }
      if (rh == 0) {
        hd += lane_xor16(hd, lane);
        hd += lane_xor32(hd, lane);
        if (lg == 0) gHdh[kl] = hd;
      }
    }
#pragma unroll
    for (int a = 0; a < 2; ++a) {
#pragma unroll
      for (int r = 0; r < 4; ++r) Wt[a][r] += Wq[a][r];
    }
    // ---- epilogue in the result layout: lane holds (token 16(2rh+a) + l16,
    //      channels cb + 16kb + 4lg + r), r = 0..3
    const int cl = 16 * kb + 4 * lg;       // first channel of the lane (in pass)
    const int kc = cb + cl;
    const bool chok = kc < K;
    float gmr[4] = {rgm, rgm, rgm, rgm};
    if constexpr (!RG) {
      const float4 gm4 = *(const float4*)(gGm + cl);
      gmr[0] = gm4.x; gmr[1] = gm4.y; gmr[2] = gm4.z; gmr[3] = gm4.w;
    }
    float dgr[2][4];
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      const int tok = 16 * (2 * rh + a) + l16;
      const bool ok = chok;                 // tokens past nval: out of the chunk's range
      const uint32_t off = (uint32_t)tok * rowK + kc;
      float gr[4];
      if constexpr (RG) {
        gr[0] = gr[1] = gr[2] = gr[3] = sRG[tok];
      } else {
        const float4 g4 = *(const float4*)(gG + tok * LG + cl);
        gr[0] = g4.x; gr[1] = g4.y; gr[2] = g4.z; gr[3] = g4.w;
      }
      // fp32 inputs re-read q, k (exact); bf16 inputs use q dq - k dk = q~ X - k~ W with
      // q~ / k~ read back from the pass planes (hi + lo: 2^-17 relative, far below bf16)
      float qv[4], kv[4];
      if constexpr (SIN) {
        unpack4(Wd::ld4(Rq, ok ? off * ES : kOOB, 0), qv);
        unpack4(Wd::ld4(Rk, ok ? off * ES : kOOB, 0), kv);
      }
      f32x4 dqv, dkv;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        dqv[r] = fast_exp2(gr[r] - gmr[r]) * X[a][r];
        dkv[r] = fast_exp2(gmr[r] - gr[r]) * Wt[a][r];
        if constexpr (SIN) {
          dgr[a][r] = qv[r] * dqv[r] - kv[r] * dkv[r];
        } else {
          const int pi = (cl + r) * LT + tok;
          if constexpr (RG) {
            // q dq - k dk with exact q, k
            dgr[a][r] = bf16_to_f32(Pqt.hi[pi]) * dqv[r] - bf16_to_f32(Pkt.hi[pi]) * dkv[r];
          } else {
            const float qt = bf16_to_f32(Pqt.hi[pi]) + bf16_to_f32(Pqt.lo[pi]);
            const float kt = bf16_to_f32(Pkt.hi[pi]) + bf16_to_f32(Pkt.lo[pi]);
            dgr[a][r] = qt * X[a][r] - kt * Wt[a][r];
          }
        }
      }
      if (kEarlyAdd || (kSlices && p.dk_add)) {
        float ka[4];
        if constexpr (kEarlyAdd) unpack4(kadd[a], ka);
        else unpack4(bld128(Rdka, ok ? off * 4u : kOOB, 0), ka);
#pragma unroll
        for (int r = 0; r < 4; ++r) dkv[r] += ka[r];
      }
      if (!kSlices || p.acc_mode == 0) {
        Wd::st4(Rdq, dqv, ok ? off * ES : kOOB, 0);
        Wd::st4(Rdk, dkv, ok ? off * ES : kOOB, 0);
      } else {
        acc_slice_t<TIn>(Rdq, Rdq32, dqv, ok ? off * 4u : kOOB, ok ? off * ES : kOOB, 0, p.acc_mode);
        acc_slice_t<TIn>(Rdk, Rdk32, dkv, ok ? off * 4u : kOOB, ok ? off * ES : kOOB, 0, p.acc_mode);
      }
    }
    // reverse cumsum over tokens: 16-lane suffix sums, block a=1's total into a=0, half 1
    // into half 0 (through gBlk)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float t1 = row16_sum(dgr[1][r]);
      dgr[0][r] = row16_suffix_sum(dgr[0][r]) + t1;
      dgr[1][r] = row16_suffix_sum(dgr[1][r]);
    }
    if (rh == 1 && l16 == 0) {
#pragma unroll
      for (int r = 0; r < 4; ++r) gBlk[cl + r] = dgr[0][r];   // total of tokens 32..63
    }
    __syncthreads();  // sZk, sHdh, sBlk visible
    float add[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      add[r] = fast_exp2(RG ? rgam : gGam[cl + r]) * gHdh[cl + r] + gZk[cl + r] + gZk[KH + cl + r];
      if (rh == 0) add[r] += gBlk[cl + r];
    }
    if (GK || gmode == kGateK || (gmode == kGateGammaK && p.dg)) {
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        const int tok = 16 * (2 * rh + a) + l16;
        const bool ok = chok;               // tokens past nval: out of the chunk's range
        const uint32_t off = (uint32_t)tok * rowK + kc;
        float ga[4] = {0.f, 0.f, 0.f, 0.f};
        if constexpr (kEarlyAdd) unpack4(gadd[a], ga);
        else if (kSlices && p.dg_add) unpack4(bld128(Rdga, ok ? off * 4u : kOOB, 0), ga);
        else if (kSlices && p.dg_accum) unpack4(bld128(Rdg, ok ? off * 4u : kOOB, 0), ga);   // earlier slices
        bst128(Rdg, make_uint4(__float_as_uint(dgr[a][0] + add[0] + ga[0]), __float_as_uint(dgr[a][1] + add[1] + ga[1]),
                               __float_as_uint(dgr[a][2] + add[2] + ga[2]), __float_as_uint(dgr[a][3] + add[3] + ga[3])),
               ok ? off * 4u : kOOB, 0);
      }
    } else if (kScalarGate && gmode == kGateS) {
      // one gate per token: sum the per-channel gradients over this wave's 16 channels
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        float x = 0.f;
        if (chok) {
#pragma unroll
          for (int r = 0; r < 4; ++r) x += dgr[a][r] + add[r];
        }
        x += __shfl_xor(x, 16, 64);
        x += __shfl_xor(x, 32, 64);
        if (lg == 0) gDgS[kb * C + 16 * (2 * rh + a) + l16] += x;
      }
    }
  }
  if (kScalarGate && gmode == kGateS && p.dg) {
    __syncthreads();
    if (tq < C) {
      float x = gDgS[tq] + gDgS[C + tq];
      const uint32_t o = (uint32_t)tq * H * 4u;   // tokens past nval: out of Rdg's range
      if (kSlices && p.dg_accum) x += __uint_as_float(bld32(Rdg, o, 0));   // earlier slices
      bst32(Rdg, __float_as_uint(x), o, 0);
    }
  }
  };
  typedef std::integral_constant<int, 0> I0;
  typedef std::integral_constant<int, 1> I1;
  const bool r1 = (wave >> 1) & 1;
  if (PAIR && (wave >> 2)) {
    if (r1) run(I1{}, I1{});
    else run(I1{}, I0{});
  } else {
    if (r1) run(I0{}, I1{});
    else run(I0{}, I0{});
  }
}

template <typename TIn, typename TV>
hipError_t launch_gla_dqkg(const DqkgParams& p, hipStream_t s) {
  const int kp = p.K <= 32 ? 32 : (p.K <= 64 ? 64 : 128);
  const int vp = p.V <= 32 ? 32 : (p.V <= 64 ? 64 : 128);
  dim3 grid(p.total * p.H), block(256);
  // the fp32-v instantiation (the KDA backward) serves only the per-channel gate
  constexpr bool kAllModes = std::is_same<TIn, TV>::value;
  constexpr bool kPairs = kAllModes && std::is_same<TIn, uint16_t>::value;
  const bool gk = !kAllModes || p.gate_mode == kGateK;
  if (p.paired && !kPairs) return hipErrorInvalidValue;
  const dim3 pgrid(((p.total + 1) / 2) * p.H), pblock(512);
  // fp16 checkpoints: bf16, per-channel gates or one gate per token (RG), no pairs or slices
  const bool rg_mode = !gk && (p.gate_mode == kGateS || p.gate_mode == kGateGamma);
  if (p.ckpt16 && (!kPairs || !(gk || rg_mode) || p.paired || p.acc_mode || p.dg_accum ||
                   p.dk_add || p.dg_add || p.ldk || p.ldv))
    return hipErrorInvalidValue;
#define TOPS_DQKG(KPV, VPV)                                                                   \
  if (kp == KPV && vp == VPV) {                                                               \
    if constexpr (kPairs) {                                                                   \
      if (p.ckpt16) {                                                                         \
        if (gk) hipLaunchKernelGGL((gla_dqkg_kernel<TIn, TV, KPV, VPV, true, false, false, true>), grid, block, 0, s, p); \
        else hipLaunchKernelGGL((gla_dqkg_kernel<TIn, TV, KPV, VPV, false, false, true, true>), grid, block, 0, s, p); \
        return hipGetLastError();                                                             \
      }                                                                                       \
      if (p.paired) {                                                                         \
        if (gk) hipLaunchKernelGGL((gla_dqkg_kernel<TIn, TV, KPV, VPV, true, true>), pgrid, pblock, 0, s, p); \
        else hipLaunchKernelGGL((gla_dqkg_kernel<TIn, TV, KPV, VPV, false, true>), pgrid, pblock, 0, s, p); \
        return hipGetLastError();                                                             \
      }                                                                                       \
    }                                                                                         \
    if constexpr (kPairs) {                                                                   \
      if (!gk && (p.gate_mode == kGateS || p.gate_mode == kGateGamma)) {                      \
        hipLaunchKernelGGL((gla_dqkg_kernel<TIn, TV, KPV, VPV, false, false, true>), grid, block, 0, s, p); \
        return hipGetLastError();                                                             \
      }                                                                                       \
    }                                                                                         \
    if (gk) hipLaunchKernelGGL((gla_dqkg_kernel<TIn, TV, KPV, VPV, true, false>), grid, block, 0, s, p); \
    else if constexpr (kAllModes)                                                             \
      hipLaunchKernelGGL((gla_dqkg_kernel<TIn, TV, KPV, VPV, false, false>), grid, block, 0, s, p); \
    return hipGetLastError();                                                                 \
  }
  TOPS_DQKG(32, 32) TOPS_DQKG(32, 64) TOPS_DQKG(32, 128)
  TOPS_DQKG(64, 32) TOPS_DQKG(64, 64) TOPS_DQKG(64, 128)
  TOPS_DQKG(128, 32) TOPS_DQKG(128, 64) TOPS_DQKG(128, 128)
#undef TOPS_DQKG
  return hipErrorInvalidValue;
}

template hipError_t launch_gla_dqkg<uint16_t, uint16_t>(const DqkgParams&, hipStream_t);
template hipError_t launch_gla_dqkg<_Float16, _Float16>(const DqkgParams&, hipStream_t);
template hipError_t launch_gla_dqkg<float, float>(const DqkgParams&, hipStream_t);
template hipError_t launch_gla_dqkg<uint16_t, float>(const DqkgParams&, hipStream_t);

}  // namespace tops
