// Fused recurrent GLA for gfx950: the per-token recurrence, forward and backward.
//
// Replaces the reference's K5 _fused_recurrent_gla_fwd_kernel
// (tops/ops/gla/fused_recurrent.py:140-372), K6 _fused_recurrent_gla_bwd_kernel (:496-750)
// and _compute_gate_grads (:800-878), following the oracle
// tops/cpu/ops/gla/fused_recurrent.py:51-358:
//     h_t = h_{t-1} * exp(gk_t)[:, None] * exp(gv_t)[None, :] + k_t v_t^T
//     o_t = h_t^T (scale q_t)
// over t = bos..eos-1, or eos-1..bos with `reverse`, per sequence (varlen) and head.
//
// One workgroup (4 wave64) owns one (sequence, head, 32-wide V tile).  Thread (grp, col)
// holds state rows grp*RG .. grp*RG + RG - 1 of column col in registers (RG = KP / 8).
// Tokens are processed in blocks of 16: the block's q (pre-scaled), k, exp(gk), v and
// exp(gv) are staged in LDS (the next block is prefetched into registers meanwhile), every
// thread advances its rows token by token reading broadcast LDS values, and the
// reductions over K (o, dv) are done once per block through LDS.  Reductions over V
// within the tile (dq, dk) use a 32-lane reduce-scatter; the V tiles' partial sums are
// added by the finishing kernel, which also forms the gate gradients as suffix sums.
#include <stdio.h>

#include "tops_common.h"
#include "tops_hip.h"

namespace tops {

struct FrParams {
  const void* q;
  const void* k;
  const void* v;
  const float* gk;      // [B,T,H,K] or NULL
  const float* gv;      // [B,T,H,V] or NULL
  const float* s0;      // h0 (forward / replay) [N,H,K,V] or NULL
  const float* dht;     // [N,H,K,V] or NULL (backward)
  const void* dout;     // dO [B,T,H,V] (backward)
  void* o;              // o [B,T,H,V] in the input dtype (forward)
  float* o32;           // o in fp32 (forward, optional)
  float* s_fin;         // ht (forward) / dh0 (backward) or NULL
  float* h_fin;         // final state of the replay (backward) [N,H,K,V]
  float* dq_part;       // [NV, B*T*H*K] fp32 (backward)
  float* dk_part;       // [NV, B*T*H*K] fp32 (backward)
  void* dv;             // [B,T,H,V] (backward)
  float* dv32;          // fp32 copy of dv for the gv gradient, or NULL (backward)
  const int* cu_seqlens;
  int B, T, H, K, V, N, NV;
  float scale;
  int reverse;
  const float* beta = nullptr;   // KDA decode: the delta-rule rate [B,T,H]
  // decode with the output norm (NORM instance): y = RMSNorm(o) * nw * silu(ng) over V
  const void* ng = nullptr;      // output gate [B,T,H,V] in the input dtype, or NULL
  const float* nw = nullptr;     // norm weight [V], or NULL
  float neps = 0.f;
  float ninv = 0.f;              // 1 / V
  // decode with the layer's ShortConvolutions fused into the token staging (CONV instance):
  // q, k, v are then the projections before the convolutions; per input (0 q, 1 k, 2 v) the
  // weights [D,W] fp32, bias [D] or NULL, cache [N,D,W] fp32 in (NULL: zeros) and out (NULL:
  // not kept; may alias the input cache), D = H*K or H*V
  const float* cw[3] = {nullptr, nullptr, nullptr};
  const float* cb[3] = {nullptr, nullptr, nullptr};
  const float* cci[3] = {nullptr, nullptr, nullptr};
  float* cco[3] = {nullptr, nullptr, nullptr};
  int cW = 0;                    // taps
  int cact = 0;                  // 1: SiLU after the convolution
  int y32 = 0;                   // 1: the output is fp32 (whatever the input dtype)
};

constexpr int kFrBV = 32;   // V tile
constexpr int kFrTB = 16;   // tokens per block

__device__ __forceinline__ float ld_elem(const uint16_t* p, size_t i) { return bf16_to_f32(p[i]); }
__device__ __forceinline__ float ld_elem(const float* p, size_t i) { return p[i]; }
__device__ __forceinline__ void st_elem(uint16_t* p, size_t i, float x) { p[i] = f32_to_bf16(x); }
__device__ __forceinline__ void st_elem(float* p, size_t i, float x) { p[i] = x; }
// 4 consecutive elements at p + i (i a multiple of 4: 8- / 16-byte aligned)
__device__ __forceinline__ float4 ld4(const uint16_t* p, size_t i) {
  const uint2 w = *(const uint2*)(p + i);
  return make_float4(__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xffff0000u),
                     __uint_as_float(w.y << 16), __uint_as_float(w.y & 0xffff0000u));
}
__device__ __forceinline__ float4 ld4(const float* p, size_t i) { return *(const float4*)(p + i); }
__device__ __forceinline__ void st4(uint16_t* p, size_t i, float4 x) {
  *(uint2*)(p + i) = make_uint2((uint32_t)f32_to_bf16(x.x) | ((uint32_t)f32_to_bf16(x.y) << 16),
                                (uint32_t)f32_to_bf16(x.z) | ((uint32_t)f32_to_bf16(x.w) << 16));
}
__device__ __forceinline__ void st4(float* p, size_t i, float4 x) { *(float4*)(p + i) = x; }

// Sum of v[0..NR-1] over the 32 lanes of a half-wave, reduce-scattered (v is clobbered):
// returns the total of row `row` (lanes 2j and 2j+1 of the half-wave get row j for
// NR = 16; lanes 4j..4j+3 for NR = 8; lanes 8j..8j+7 for NR = 4).  NR in {4, 8, 16}.
template <int NR>
__device__ __forceinline__ float rs32(float (&v)[NR], int lane32, int& row) {
  int n = NR, base = 0;
#pragma unroll
  for (int off = 16; off >= 1; off >>= 1) {
    if (n > 1) {
      const int h = n / 2;
      const bool upper = (lane32 & off) != 0;
#pragma unroll
      for (int i = 0; i < NR / 2; ++i) {
        if (i < h) {
          const float mine = upper ? v[i + h] : v[i];
          const float other = upper ? v[i] : v[i + h];
          v[i] = mine + __shfl_xor(other, off, 64);
        }
      }
      if (upper) base += h;
      n = h;
    } else {
      v[0] += __shfl_xor(v[0], off, 64);
    }
  }
  row = base;
  return v[0];
}

template <typename TIn, int KP, bool BWD>
__global__ __launch_bounds__(256) void fr_kernel(FrParams p) {
  constexpr int BV = kFrBV, TB = kFrTB, RG = KP / 8;
  constexpr int NE = TB * KP / 256;   // staged [TB][KP] elements per thread
  __shared__ __attribute__((aligned(16))) float sq[TB][KP];
  __shared__ __attribute__((aligned(16))) float sk[TB][KP];
  __shared__ __attribute__((aligned(16))) float sd[TB][KP];
  __shared__ float sv[TB][BV];
  __shared__ float sgv[TB][BV];
  __shared__ float sdo[TB][BV];
  __shared__ float sred[8][TB][BV];
  __shared__ __attribute__((aligned(16))) float sdqk[TB][KP];

  const int tid = threadIdx.x;
  const int col = tid & 31, grp = tid >> 5, lane32 = tid & 31;
  const int r0 = grp * RG;
  const int wg = blockIdx.x;
  const int vt = wg % p.NV;
  const int hh = (wg / p.NV) % p.H;
  const int n = wg / (p.NV * p.H);
  const int H = p.H, K = p.K, V = p.V;
  const int vc = vt * BV + col;
  const bool colok = vc < V;

  int bos, L;
  if (p.cu_seqlens) {
    bos = p.cu_seqlens[n];
    L = p.cu_seqlens[n + 1] - bos;
  } else {
    bos = n * p.T;
    L = p.T;
  }
  const int nblk = cdiv(L, TB);
  const TIn* q = (const TIn*)p.q;
  const TIn* kk = (const TIn*)p.k;
  const TIn* v = (const TIn*)p.v;
  const TIn* dout = (const TIn*)p.dout;
  const size_t sbase = ((size_t)n * H + hh) * K * V;

  // time index of the j-th token of block b in processing order
  auto tok = [&](int b, int j) { return p.reverse ? bos + L - 1 - (b * TB + j) : bos + b * TB + j; };

  // ---- raw block registers (prefetch)
  float rq[NE], rk[NE], rg[NE], rv[2], rgv[2], rdo[2];
  auto load_block = [&](int b) {
#pragma unroll
    for (int i = 0; i < NE; ++i) {
      const int e = tid + 256 * i, j = e / KP, row = e % KP;
      const bool ok = (b * TB + j < L) && row < K;
      const size_t off = ((size_t)(ok ? tok(b, j) : bos) * H + hh) * K + (ok ? row : 0);
      rq[i] = ok ? ld_elem(q, off) : 0.f;
      rk[i] = ok ? ld_elem(kk, off) : 0.f;
      rg[i] = (ok && p.gk) ? p.gk[off] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int e = tid + 256 * i, j = e / BV, c = e % BV, vv = vt * BV + c;
      const bool ok = (b * TB + j < L) && vv < V;
      const size_t off = ((size_t)(ok ? tok(b, j) : bos) * H + hh) * V + (ok ? vv : 0);
      rv[i] = ok ? ld_elem(v, off) : 0.f;
      rgv[i] = (ok && p.gv) ? p.gv[off] : 0.f;
      if constexpr (BWD) rdo[i] = ok ? ld_elem(dout, off) : 0.f;
    }
  };
  auto stage_block = [&]() {
#pragma unroll
    for (int i = 0; i < NE; ++i) {
      const int e = tid + 256 * i, j = e / KP, row = e % KP;
      sq[j][row] = rq[i] * p.scale;
      sk[j][row] = rk[i];
      sd[j][row] = fast_exp2(rg[i] * kLog2e);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int e = tid + 256 * i, j = e / BV, c = e % BV;
      sv[j][c] = rv[i];
      sgv[j][c] = fast_exp2(rgv[i] * kLog2e);
      if constexpr (BWD) sdo[j][c] = rdo[i];
    }
  };

  // ================= forward (or the backward's replay pass)
  float h[RG];
#pragma unroll
  for (int r = 0; r < RG; ++r) {
    const int kr = r0 + r;
    h[r] = (p.s0 && kr < K && colok) ? p.s0[sbase + (size_t)kr * V + vc] : 0.f;
  }
  load_block(0);
  for (int b = 0; b < nblk; ++b) {
    stage_block();
    __syncthreads();
    if (b + 1 < nblk) load_block(b + 1);
#pragma unroll
    for (int j = 0; j < TB; ++j) {
      const float vj = sv[j][col], gvj = sgv[j][col];
      float acc = 0.f;
      float pr[RG];
#pragma unroll
      for (int r4 = 0; r4 < RG; r4 += 4) {
        const float4 d4 = *(const float4*)&sd[j][r0 + r4];
        const float4 k4 = *(const float4*)&sk[j][r0 + r4];
        const float4 q4 = *(const float4*)&sq[j][r0 + r4];
        const float dd[4] = {d4.x, d4.y, d4.z, d4.w}, ks[4] = {k4.x, k4.y, k4.z, k4.w};
        const float qs[4] = {q4.x, q4.y, q4.z, q4.w};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          h[r4 + u] = h[r4 + u] * (dd[u] * gvj) + ks[u] * vj;
          acc += h[r4 + u] * qs[u];
        }
      }
      if constexpr (BWD) {
        // dq_t[k] = scale sum_v h_t[k][v] dO_t[v] over this tile's columns
        const float dj = sdo[j][col] * p.scale;
#pragma unroll
        for (int r = 0; r < RG; ++r) pr[r] = h[r] * dj;
        int row;
        const float s = rs32<RG>(pr, lane32, row);
        if ((lane32 & ((32 / RG) - 1)) == 0) sdqk[j][r0 + row] = s;
      } else {
        sred[grp][j][col] = acc;
      }
    }
    __syncthreads();
    if constexpr (!BWD) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int e = tid + 256 * i, j = e / BV, c = e % BV, vv = vt * BV + c;
        float s = 0.f;
#pragma unroll
        for (int g = 0; g < 8; ++g) s += sred[g][j][c];
        if (b * TB + j < L && vv < V) {
          const size_t off = ((size_t)tok(b, j) * H + hh) * V + vv;
          st_elem((TIn*)p.o, off, s);
          if (p.o32) p.o32[off] = s;
        }
      }
    } else {
      // dq partial of this V tile
#pragma unroll
      for (int i = 0; i < NE; ++i) {
        const int e = tid + 256 * i, j = e / KP, row = e % KP;
        if (b * TB + j < L && row < K)
          p.dq_part[(size_t)vt * ((size_t)p.B * p.T * H * K) + ((size_t)tok(b, j) * H + hh) * K + row] = sdqk[j][row];
      }
    }
    __syncthreads();
  }
  if (!BWD && p.s_fin) {
#pragma unroll
    for (int r = 0; r < RG; ++r) {
      const int kr = r0 + r;
      if (kr < K && colok) p.s_fin[sbase + (size_t)kr * V + vc] = h[r];
    }
  }
  if constexpr (BWD) {
    if (p.h_fin) {
#pragma unroll
      for (int r = 0; r < RG; ++r) {
        const int kr = r0 + r;
        if (kr < K && colok) p.h_fin[sbase + (size_t)kr * V + vc] = h[r];
      }
    }
    // ================= backward: reverse of the processing order
    float dh[RG];
#pragma unroll
    for (int r = 0; r < RG; ++r) {
      const int kr = r0 + r;
      dh[r] = (p.dht && kr < K && colok) ? p.dht[sbase + (size_t)kr * V + vc] : 0.f;
    }
    load_block(nblk - 1);
    for (int b = nblk - 1; b >= 0; --b) {
      stage_block();
      __syncthreads();
      if (b > 0) load_block(b - 1);
#pragma unroll 2
      for (int jj = 0; jj < TB; ++jj) {
        const int j = TB - 1 - jj;
        const float vj = sv[j][col], gvj = sgv[j][col], dj = sdo[j][col];
        float acc = 0.f, pr[RG];
#pragma unroll
        for (int r4 = 0; r4 < RG; r4 += 4) {
          const float4 k4 = *(const float4*)&sk[j][r0 + r4];
          const float4 q4 = *(const float4*)&sq[j][r0 + r4];
          const float ks[4] = {k4.x, k4.y, k4.z, k4.w}, qs[4] = {q4.x, q4.y, q4.z, q4.w};
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            dh[r4 + u] += qs[u] * dj;                 // dh += (scale q) dO^T
            pr[r4 + u] = dh[r4 + u] * vj;             // dk_t = dh v_t
            acc += dh[r4 + u] * ks[u];                // dv_t = dh^T k_t
          }
        }
        int row;
        const float s = rs32<RG>(pr, lane32, row);
        if ((lane32 & ((32 / RG) - 1)) == 0) sdqk[j][r0 + row] = s;
        sred[grp][j][col] = acc;
#pragma unroll
        for (int r4 = 0; r4 < RG; r4 += 4) {
          const float4 d4 = *(const float4*)&sd[j][r0 + r4];
          const float dd[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
          for (int u = 0; u < 4; ++u) dh[r4 + u] *= dd[u] * gvj;
        }
      }
      __syncthreads();
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int e = tid + 256 * i, j = e / BV, c = e % BV, vv = vt * BV + c;
        float s = 0.f;
#pragma unroll
        for (int g = 0; g < 8; ++g) s += sred[g][j][c];
        if (b * TB + j < L && vv < V) {
          const size_t off = ((size_t)tok(b, j) * H + hh) * V + vv;
          st_elem((TIn*)p.dv, off, s);
          if (p.dv32) p.dv32[off] = s;
        }
      }
#pragma unroll
      for (int i = 0; i < NE; ++i) {
        const int e = tid + 256 * i, j = e / KP, row = e % KP;
        if (b * TB + j < L && row < K)
          p.dk_part[(size_t)vt * ((size_t)p.B * p.T * H * K) + ((size_t)tok(b, j) * H + hh) * K + row] = sdqk[j][row];
      }
      __syncthreads();
    }
    if (p.s_fin) {
#pragma unroll
      for (int r = 0; r < RG; ++r) {
        const int kr = r0 + r;
        if (kr < K && colok) p.s_fin[sbase + (size_t)kr * V + vc] = dh[r];
      }
    }
  }
}

// Finishing kernel of the backward: one workgroup per (sequence, head).  Threads
// 0..K-1 sum the V-tile partials of dq and dk (written in the input dtype) and form
// dgk_t = sum over later-processed tokens s >= t of (q dq - k dk)_s + sum_v(h_T dht);
// threads 128..128+V-1 form dgv_t = sum_{s >= t} (o dO - v dv)_s + sum_k(h_T dht).
struct FrFinishParams {
  const void* q;
  const void* k;
  const void* v;
  const float* o32;
  const void* dout;
  const float* dv32;
  const float* dht;
  const float* h_fin;
  const float* dq_part;
  const float* dk_part;
  void* dq;
  void* dk;
  float* dgk;
  float* dgv;
  const int* cu_seqlens;
  int B, T, H, K, V, N, NV;
  int reverse;
};

template <typename TIn>
__global__ __launch_bounds__(256) void fr_finish_kernel(FrFinishParams p) {
  const int tid = threadIdx.x;
  const int hh = blockIdx.x % p.H, n = blockIdx.x / p.H;
  const int H = p.H, K = p.K, V = p.V;
  int bos, L;
  if (p.cu_seqlens) {
    bos = p.cu_seqlens[n];
    L = p.cu_seqlens[n + 1] - bos;
  } else {
    bos = n * p.T;
    L = p.T;
  }
  const size_t sbase = ((size_t)n * H + hh) * K * V;
  const size_t plane = (size_t)p.B * p.T * H * K;
  if (tid < 128) {
    const int kr = tid;
    if (kr >= K) return;
    float bnd = 0.f;
    if (p.dgk && p.dht) {
      for (int vv = 0; vv < V; ++vv) bnd += p.h_fin[sbase + (size_t)kr * V + vv] * p.dht[sbase + (size_t)kr * V + vv];
    }
    float run = 0.f;
    for (int s = L - 1; s >= 0; --s) {          // s: position in processing order
      const int t = p.reverse ? bos + L - 1 - s : bos + s;
      const size_t off = ((size_t)t * H + hh) * K + kr;
      float dq = 0.f, dk = 0.f;
      for (int i = 0; i < p.NV; ++i) {
        dq += p.dq_part[i * plane + off];
        dk += p.dk_part[i * plane + off];
      }
      st_elem((TIn*)p.dq, off, dq);
      st_elem((TIn*)p.dk, off, dk);
      if (p.dgk) {
        run += ld_elem((const TIn*)p.q, off) * dq - ld_elem((const TIn*)p.k, off) * dk;
        p.dgk[off] = run + bnd;
      }
    }
  } else {
    if (!p.dgv) return;
    for (int vv = tid - 128; vv < V; vv += 128) {
    float bnd = 0.f;
    if (p.dht) {
      for (int kr = 0; kr < K; ++kr) bnd += p.h_fin[sbase + (size_t)kr * V + vv] * p.dht[sbase + (size_t)kr * V + vv];
    }
    float run = 0.f;
    for (int s = L - 1; s >= 0; --s) {
      const int t = p.reverse ? bos + L - 1 - s : bos + s;
      const size_t off = ((size_t)t * H + hh) * V + vv;
      run += p.o32[off] * ld_elem((const TIn*)p.dout, off) - ld_elem((const TIn*)p.v, off) * p.dv32[off];
      p.dgv[off] = run + bnd;
    }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Short sequences (decode steps): one wave per (sequence, head, 32-column tile) with the state
// slice in registers.  Lane (kr, cq) = (lane % 8, lane / 8) holds rows RL kr .. RL kr + RL - 1
// (RL = KP / 8) and columns 4 cq .. 4 cq + 3 of the tile, so each state load or store of a wave
// covers whole 128-byte rows of the tile and no two waves share a line (one wave's tile never
// straddles the L2s of two XCDs).  Tokens are staged DT at a time into LDS with coalesced
// loads (q scaled, the gates as decay factors exp(g), one exponential per element), so their
// latency is paid once per block; o_t[v] is reduced over the 8 row groups with three DPP steps
// inside a 16-lane row.  With a few tokens the launch is bound by the state read and write
// (h0 in, ht out).
constexpr int kFrDecodeT = 4;    // longest sequence the fixed-length entry sends here

// sum over the 8 lanes l .. l | 7 (bits 0-2 of the lane index), in every one of them
__device__ __forceinline__ float oct_sum(float x) {
  x += dpp_row<0xB1>(x);   // quad_perm [1,0,3,2]
  x += dpp_row<0x4E>(x);   // quad_perm [2,3,0,1]
  x += dpp_row<0x141>(x);  // row_half_mirror: lane i <- 7 - i within each 8 lanes
  return x;
}

// DELTA: the KDA delta rule instead of the GLA update (tops/cpu/ops/kda/naive.py:10-118):
// S <- diag(exp g_t) S;  S <- S + beta_t k_t (v_t - S^T k_t)^T;  o_t = S^T (scale q_t), with a
// second 8-lane reduction for S^T k_t before the update.
// NORM: the output norm of the GLA layer fused as the epilogue (V <= 128, so the workgroup
// holds the whole head_v_dim row of every token): y_t = o_t / sqrt(mean_v o_t^2 + eps) * w *
// silu(g_t) (tops/modules/fused_norm_gate.py:6-37; without g: RMSNorm, layernorm.py:6-35).
// Each wave leaves its 32 columns of o_t in LDS, in the v block it has just read (a wave
// reads its own columns of v_t before it writes the same columns of o_t, and no other wave
// touches them), so the kernel keeps the plain instance's LDS size and with it the compiler's
// occupancy target; after the block's closing barrier a thread takes 4 columns of one token,
// the 32 lanes of a half-wave sum a token's squares, and the stores of y are coalesced.  o_t
// stays in fp32 on the way (the unfused route rounds it to the input dtype first).
template <typename TIn, int KP, bool DELTA, bool NORM, bool CONV = false>
__device__ __forceinline__ void fr_decode_body(const FrParams& p) {
  constexpr int RL = KP / 8;            // rows per lane
  constexpr int DT = 8;                 // tokens per staged block
  constexpr int WV = 4;                 // waves (32-column tiles) per workgroup
  __shared__ float sB[DT];              // beta (DELTA)
  __shared__ __attribute__((aligned(16))) float sQ[DT][KP];
  __shared__ __attribute__((aligned(16))) float sK[DT][KP];
  __shared__ __attribute__((aligned(16))) float sD[DT][KP];    // exp(gk)
  __shared__ __attribute__((aligned(16))) float sV[DT][32 * WV];
  __shared__ __attribute__((aligned(16))) float sDV[DT][32 * WV];   // exp(gv)
  float (*sO)[32 * WV] = sV;            // NORM: o_t of the block, over the consumed v
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kr = lane & 7, cq = lane >> 3;
  const int H = p.H, K = p.K, V = p.V;
  const int NT = (V + 31) / 32, NG = (NT + WV - 1) / WV;
  const int tg = blockIdx.x % NG;       // the workgroup's group of WV tiles (the same tokens)
  const int tile = WV * tg + wave;      // this wave's tile; waves past the last one only stage
  const bool live = tile < NT;
  const int hh = (blockIdx.x / NG) % H;
  const int n = blockIdx.x / (NG * H);
  int bos, L;
  if (p.cu_seqlens) {
    bos = p.cu_seqlens[n];
    L = p.cu_seqlens[n + 1] - bos;
  } else {
    bos = n * p.T;
    L = p.T;
  }
  const int r0 = RL * kr, c0 = 32 * tile + 4 * cq;
  // K % 4 == 0: each quad of rows is wholly in or out
  bool qok[RL / 4];
#pragma unroll
  for (int m = 0; m < RL / 4; ++m) qok[m] = r0 + 4 * m < K;
  bool cok[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) cok[c] = c0 + c < V;
  const bool vec = (V % 4) == 0 && cok[3];
  if (!live) {
#pragma unroll
    for (int c = 0; c < 4; ++c) cok[c] = false;
  }
  const size_t sbase = ((size_t)n * H + hh) * K * V;
  const TIn* q = (const TIn*)p.q;
  const TIn* kk = (const TIn*)p.k;
  const TIn* v = (const TIn*)p.v;
  auto tok = [&](int j) { return p.reverse ? bos + L - 1 - j : bos + j; };
  // CONV: the convolution of input x (weights wt, bias, cache cin) for channel d (column c of
  // head hh, row width DW) at position jj of the sequence: the causal W-tap window over the
  // projections, positions before the sequence read from the conv cache (position -1 = its
  // newest entry, W - 1)
  // (the taps are unrolled to the largest W, 8, so that every load of a window issues before
  // the first is used)
  auto conv_in = [&](const TIn* x, const float* wt, const float* bias, const float* cin, int D,
                     int d, int DW, int c, int jj) __attribute__((always_inline)) {
    const int W = p.cW;
    const float* w = wt + (size_t)d * W;
    const float* cache = cin ? cin + ((size_t)n * D + d) * W : nullptr;
    float wv[8], xv[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int pos = jj - (W - 1) + t;
      wv[t] = t < W ? w[t] : 0.f;
      xv[t] = t >= W ? 0.f
                     : (pos >= 0 ? ld_elem(x, ((size_t)(bos + pos) * H + hh) * DW + c)
                                 : (cache ? cache[W + pos] : 0.f));
    }
    float acc = bias ? bias[d] : 0.f;
#pragma unroll
    for (int t = 0; t < 8; ++t) acc += wv[t] * xv[t];
    return p.cact ? acc * sigm(acc) : acc;
  };

  float S[RL][4];
#pragma unroll
  for (int i = 0; i < RL; ++i) {
    const bool rok = qok[i / 4];
    const size_t o = sbase + (size_t)(r0 + i) * V + c0;
    if (p.s0 && rok && vec && live) {
      const float4 x = *(const float4*)(p.s0 + o);
      S[i][0] = x.x; S[i][1] = x.y; S[i][2] = x.z; S[i][3] = x.w;
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c) S[i][c] = (p.s0 && rok && cok[c]) ? p.s0[o + c] : 0.f;
    }
  }
  // CONV: the rolled conv caches, one thread per channel: entry t of channel d is the input at
  // position L - W + t (before the sequence: the old cache entry W + pos); written after the
  // last block (below).  One call per input with its own pointers: selecting among the
  // parameter block's pointers by a run-time index would put the whole block in private memory.
  auto roll = [&](const TIn* x, const float* cache, float* out, int DW) __attribute__((always_inline)) {
    if (!out) return;
    const int W = p.cW, D = H * DW;
    for (int c = tid; c < DW; c += 256) {
      const int d = hh * DW + c;
      const size_t cbase = ((size_t)n * D + d) * W;
      for (int t = 0; t < W; ++t) {
        const int pos = L - W + t;
        float val;
        if (pos >= 0) val = ld_elem(x, ((size_t)(bos + pos) * H + hh) * DW + c);
        else val = cache ? cache[cbase + W + pos] : 0.f;
        out[cbase + t] = val;
      }
    }
  };
  auto store_state = [&]() {
    if (!p.s_fin || !live) return;
    // opaque copies: the addresses are formed here, not hoisted into the block loop
    int rr = r0, cc = c0;
    asm volatile("" : "+v"(rr), "+v"(cc));
#pragma unroll
    for (int i = 0; i < RL; ++i) {
      if (!qok[i / 4]) continue;
      const size_t o = sbase + (size_t)(rr + i) * V + cc;
      if (vec) {
        *(float4*)(p.s_fin + o) = make_float4(S[i][0], S[i][1], S[i][2], S[i][3]);
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c)
          if (cok[c]) p.s_fin[o + c] = S[i][c];
      }
    }
  };
  for (int b0 = 0; b0 < L; b0 += DT) {
    const int nb = min(DT, L - b0);
    // ---- stage tokens b0 .. b0 + nb - 1 for the workgroup's tiles: element e = tid + 256 u of
    // the [DT][KP] / [DT][32 WV] blocks
    // CONV: an opaque copy of the lane index, so that the window's addresses are formed here
    // rather than hoisted out of the block loop and carried through the token loop
    int stid = tid;
    if constexpr (CONV) asm volatile("" : "+v"(stid));
#pragma unroll 2
    for (int u = 0; u < DT * KP / 256; ++u) {
      const int e = stid + 256 * u, j = e / KP, r = e % KP;
      const bool ok = j < nb && r < K;
      const size_t o = ok ? ((size_t)tok(b0 + j) * H + hh) * K + r : 0;
      if constexpr (CONV) {
        sQ[j][r] = ok ? conv_in(q, p.cw[0], p.cb[0], p.cci[0], H * K, hh * K + r, K, r, b0 + j) *
                            p.scale
                      : 0.f;
        sK[j][r] = ok ? conv_in(kk, p.cw[1], p.cb[1], p.cci[1], H * K, hh * K + r, K, r, b0 + j)
                      : 0.f;
      } else {
        sQ[j][r] = ok ? ld_elem(q, o) * p.scale : 0.f;
        sK[j][r] = ok ? ld_elem(kk, o) : 0.f;
      }
      sD[j][r] = (ok && p.gk) ? fast_exp2(p.gk[o] * kLog2e) : 1.f;
    }
#pragma unroll
    for (int u = 0; u < DT * 32 * WV / 256; ++u) {
      const int e = stid + 256 * u, j = e / (32 * WV), c = e % (32 * WV), col = 32 * WV * tg + c;
      const bool ok = j < nb && col < V;
      const size_t o = ok ? ((size_t)tok(b0 + j) * H + hh) * V + col : 0;
      if constexpr (CONV)
        sV[j][c] = ok ? conv_in(v, p.cw[2], p.cb[2], p.cci[2], H * V, hh * V + col, V, col, b0 + j)
                      : 0.f;
      else sV[j][c] = ok ? ld_elem(v, o) : 0.f;
      sDV[j][c] = (ok && p.gv) ? fast_exp2(p.gv[o] * kLog2e) : 1.f;
    }
    if constexpr (DELTA) {
      if (tid < DT) sB[tid] = tid < nb ? p.beta[(size_t)tok(b0 + tid) * H + hh] : 0.f;
    }
    __syncthreads();
    for (int j = 0; j < nb; ++j) {
      const float4 v4 = *(const float4*)&sV[j][32 * wave + 4 * cq];
      const float4 d4 = *(const float4*)&sDV[j][32 * wave + 4 * cq];
      const float vv[4] = {v4.x, v4.y, v4.z, v4.w}, dv[4] = {d4.x, d4.y, d4.z, d4.w};
      float acc[4] = {0.f, 0.f, 0.f, 0.f};
      if constexpr (DELTA) {
        // decay, then S^T k over the lane's rows, reduced over the 8 row groups
        float pr[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i4 = 0; i4 < RL; i4 += 4) {
          const float4 k4 = *(const float4*)&sK[j][r0 + i4];
          const float4 g4 = *(const float4*)&sD[j][r0 + i4];
          const float ks[4] = {k4.x, k4.y, k4.z, k4.w}, ds[4] = {g4.x, g4.y, g4.z, g4.w};
#pragma unroll
          for (int u = 0; u < 4; ++u) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
              S[i4 + u][c] *= ds[u];
              pr[c] += ks[u] * S[i4 + u][c];
            }
          }
        }
        const float b = sB[j];
        float du[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) du[c] = b * (vv[c] - oct_sum(pr[c]));
#pragma unroll
        for (int i4 = 0; i4 < RL; i4 += 4) {
          const float4 q4 = *(const float4*)&sQ[j][r0 + i4];
          const float4 k4 = *(const float4*)&sK[j][r0 + i4];
          const float qs[4] = {q4.x, q4.y, q4.z, q4.w}, ks[4] = {k4.x, k4.y, k4.z, k4.w};
#pragma unroll
          for (int u = 0; u < 4; ++u) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
              S[i4 + u][c] += ks[u] * du[c];
              acc[c] += S[i4 + u][c] * qs[u];
            }
          }
        }
      } else {
#pragma unroll
      for (int i4 = 0; i4 < RL; i4 += 4) {
        const float4 q4 = *(const float4*)&sQ[j][r0 + i4];
        const float4 k4 = *(const float4*)&sK[j][r0 + i4];
        const float4 g4 = *(const float4*)&sD[j][r0 + i4];
        const float qs[4] = {q4.x, q4.y, q4.z, q4.w}, ks[4] = {k4.x, k4.y, k4.z, k4.w};
        const float ds[4] = {g4.x, g4.y, g4.z, g4.w};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            S[i4 + u][c] = S[i4 + u][c] * (ds[u] * dv[c]) + ks[u] * vv[c];
            acc[c] += S[i4 + u][c] * qs[u];
          }
        }
      }
      }  // DELTA
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[c] = oct_sum(acc[c]);
      if constexpr (NORM) {
        if (kr == 0 && live)
          *(float4*)&sO[j][32 * wave + 4 * cq] = make_float4(acc[0], acc[1], acc[2], acc[3]);
      } else if (kr == 0) {
        const size_t ov = ((size_t)tok(b0 + j) * H + hh) * V + c0;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          if (cok[c]) {
            st_elem((TIn*)p.o, ov + c, acc[c]);
            if (p.o32) p.o32[ov + c] = acc[c];
          }
        }
      }
    }
    __syncthreads();   // the block's tokens are consumed before the next block is staged
    if constexpr (NORM) {
      if (b0 + DT >= L) store_state();   // the state is final: its stores go out first
      // Thread tid < 128: token j = tid / 16 of the block, columns 8 (tid % 16) .. + 7; the 16
      // threads of a token are one DPP row, which sums the token's squares on the VALU.
      // Columns past V (never written, or zero) are left out of the sum.
      // the lane index is made opaque here, so that the epilogue's addresses are computed
      // here rather than hoisted out of the block loop and carried through the token loop
      int et = tid;
      asm volatile("" : "+v"(et));
      if (et < 16 * DT) {
        const int j = et >> 4, c8 = 8 * (et & 15);
        const float4 oa = *(const float4*)&sO[j][c8], ob4 = *(const float4*)&sO[j][c8 + 4];
        const float ov[8] = {oa.x, oa.y, oa.z, oa.w, ob4.x, ob4.y, ob4.z, ob4.w};
        float ss = 0.f;
#pragma unroll
        for (int c = 0; c < 8; ++c) ss += c8 + c < V ? ov[c] * ov[c] : 0.f;
        ss = row16_sum(ss);
        if (j < nb) {
          const float r = 1.f / sqrtf(ss * p.ninv + p.neps);
          const size_t ob = ((size_t)tok(b0 + j) * H + hh) * V;
          const TIn* gate = (const TIn*)p.ng;
#pragma unroll
          for (int h4 = 0; h4 < 8; h4 += 4) {
            const int c4 = c8 + h4;
            if (c4 >= V) continue;
            if ((V & 3) == 0) {   // whole quads: one load of gate and weight, one store
              float y[4] = {ov[h4] * r, ov[h4 + 1] * r, ov[h4 + 2] * r, ov[h4 + 3] * r};
              if (p.nw) {
                const float4 w4 = *(const float4*)(p.nw + c4);
                y[0] *= w4.x; y[1] *= w4.y; y[2] *= w4.z; y[3] *= w4.w;
              }
              if (gate) {
                const float4 g4 = ld4(gate, ob + c4);
                const float gt[4] = {g4.x, g4.y, g4.z, g4.w};
#pragma unroll
                for (int c = 0; c < 4; ++c) y[c] *= gt[c] * sigm(gt[c]);
              }
              if (CONV && p.y32) st4((float*)p.o, ob + c4, make_float4(y[0], y[1], y[2], y[3]));
              else st4((TIn*)p.o, ob + c4, make_float4(y[0], y[1], y[2], y[3]));
            } else {
#pragma unroll
              for (int c = 0; c < 4; ++c) {
                if (c4 + c >= V) continue;
                float y = ov[h4 + c] * r;
                if (p.nw) y *= p.nw[c4 + c];
                if (gate) {
                  const float gt = ld_elem(gate, ob + c4 + c);
                  y *= gt * sigm(gt);
                }
                if (CONV && p.y32) st_elem((float*)p.o, ob + c4 + c, y);
                else st_elem((TIn*)p.o, ob + c4 + c, y);
              }
            }
          }
        }
      }
      if (b0 + DT < L) __syncthreads();   // sO is the next block's v: read before restaged
    }
  }
  // NORM stores the final state before its last epilogue (below, inside the block loop);
  // a sequence with no tokens passes h0 through here
  if (!(NORM && L > 0)) store_state();
  // CONV: the rolled caches, now that every block's staging has read the old entries (so an
  // output may alias its input cache)
  if constexpr (CONV) {
    roll(q, p.cci[0], p.cco[0], K);
    roll(kk, p.cci[1], p.cco[1], K);
    roll(v, p.cci[2], p.cco[2], V);
  }
}

// The GLA instances hold 138 VGPRs (3 waves per SIMD; a 4-wave bound spills); the delta rule
// fits 128 without spills, so its wrapper asks for 4 waves per SIMD.
template <typename TIn, int KP, bool DELTA, bool NORM = false>
__global__ __launch_bounds__(256) void fr_decode_kernel(FrParams p) {
  fr_decode_body<TIn, KP, DELTA, NORM>(p);
}
template <typename TIn, int KP>
__global__ __launch_bounds__(256, 4) void fr_decode_delta_kernel(FrParams p) {
  fr_decode_body<TIn, KP, true, false>(p);
}
template <typename TIn, int KP>
__global__ __launch_bounds__(256) void fr_decode_conv_kernel(FrParams p) {
  fr_decode_body<TIn, KP, false, true, true>(p);
}

template <typename TIn>
static hipError_t launch_fr_decode_conv(const FrParams& p, hipStream_t s) {
  const int kp = p.K <= 32 ? 32 : (p.K <= 64 ? 64 : 128);
  dim3 grid(p.H * p.N);
  if (kp == 32) hipLaunchKernelGGL((fr_decode_conv_kernel<TIn, 32>), grid, dim3(256), 0, s, p);
  else if (kp == 64) hipLaunchKernelGGL((fr_decode_conv_kernel<TIn, 64>), grid, dim3(256), 0, s, p);
  else hipLaunchKernelGGL((fr_decode_conv_kernel<TIn, 128>), grid, dim3(256), 0, s, p);
  return hipGetLastError();
}

template <typename TIn, bool DELTA = false, bool NORM = false>
static hipError_t launch_fr_decode(const FrParams& p, hipStream_t s) {
  const int kp = p.K <= 32 ? 32 : (p.K <= 64 ? 64 : 128);
  dim3 grid((((p.V + 31) / 32 + 3) / 4) * p.H * p.N);
  if constexpr (DELTA) {
    if (kp == 32) hipLaunchKernelGGL((fr_decode_delta_kernel<TIn, 32>), grid, dim3(256), 0, s, p);
    else if (kp == 64) hipLaunchKernelGGL((fr_decode_delta_kernel<TIn, 64>), grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL((fr_decode_delta_kernel<TIn, 128>), grid, dim3(256), 0, s, p);
  } else {
    if (kp == 32) hipLaunchKernelGGL((fr_decode_kernel<TIn, 32, false, NORM>), grid, dim3(256), 0, s, p);
    else if (kp == 64) hipLaunchKernelGGL((fr_decode_kernel<TIn, 64, false, NORM>), grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL((fr_decode_kernel<TIn, 128, false, NORM>), grid, dim3(256), 0, s, p);
  }
  return hipGetLastError();
}

template <typename TIn, bool BWD>
static hipError_t launch_fr(const FrParams& p, hipStream_t s) {
  const int kp = p.K <= 32 ? 32 : (p.K <= 64 ? 64 : 128);
  dim3 grid(p.NV * p.H * p.N);
  if (kp == 32) hipLaunchKernelGGL((fr_kernel<TIn, 32, BWD>), grid, dim3(256), 0, s, p);
  else if (kp == 64) hipLaunchKernelGGL((fr_kernel<TIn, 64, BWD>), grid, dim3(256), 0, s, p);
  else hipLaunchKernelGGL((fr_kernel<TIn, 128, BWD>), grid, dim3(256), 0, s, p);
  return hipGetLastError();
}

static int fr_check(const char* who, int B, int T, int H, int K, int V, int N,
                    const int32_t* cu_seqlens, int dtype) {
  char msg[160];
  if (B <= 0 || T <= 0 || H <= 0 || K <= 0 || V <= 0 || N <= 0) {
    snprintf(msg, sizeof(msg), "%s: non-positive dimension", who);
    return tops_set_error(TOPS_ERR_SHAPE, msg);
  }
  if (K > 128 || (K % 4)) {
    snprintf(msg, sizeof(msg), "%s: need K <= 128 and K %% 4 == 0", who);
    return tops_set_error(TOPS_ERR_SHAPE, msg);
  }
  if (cu_seqlens && B != 1) {
    snprintf(msg, sizeof(msg), "%s: varlen needs B == 1", who);
    return tops_set_error(TOPS_ERR_SHAPE, msg);
  }
  if (!cu_seqlens && N != B) {
    snprintf(msg, sizeof(msg), "%s: N must equal B", who);
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

extern "C" int64_t tops_gla_fused_recurrent_bwd_workspace(int B, int T, int H, int K, int V, int N,
                                                         int with_gv) {
  const int64_t NV = (V + kFrBV - 1) / kFrBV;
  return (2 * NV * (int64_t)B * T * H * K + (int64_t)N * H * K * V +
          (with_gv ? (int64_t)B * T * H * V : 0)) * 4;
}

extern "C" int tops_gla_fused_recurrent_fwd(const void* q, const void* k, const void* v,
                                            const float* gk, const float* gv, const float* h0,
                                            void* o, float* o32, float* ht,
                                            const int32_t* cu_seqlens, int B, int T, int H, int K,
                                            int V, int N, int dtype, float scale, int reverse,
                                            void* stream) {
  if (!q || !k || !v || !o) return tops_set_error(TOPS_ERR_NULL, "gla_fused_recurrent_fwd: null tensor");
  int rc = fr_check("gla_fused_recurrent_fwd", B, T, H, K, V, N, cu_seqlens, dtype);
  if (rc != TOPS_OK) return rc;
  FrParams p{q, k, v, gk, gv, h0, nullptr, nullptr, o, o32, ht, nullptr, nullptr, nullptr, nullptr,
             nullptr, cu_seqlens, B, T, H, K, V, N, (V + kFrBV - 1) / kFrBV, scale, reverse ? 1 : 0};
  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  if (!cu_seqlens && T <= kFrDecodeT)
    e = dtype == TOPS_BF16 ? launch_fr_decode<uint16_t>(p, s) : launch_fr_decode<float>(p, s);
  else
    e = dtype == TOPS_BF16 ? launch_fr<uint16_t, false>(p, s) : launch_fr<float, false>(p, s);
  if (e != hipSuccess) return tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
  return TOPS_OK;
}

extern "C" int tops_gla_fused_recurrent_fwd_decode(const void* q, const void* k, const void* v,
                                                   const float* gk, const float* gv, const float* h0,
                                                   void* o, float* o32, float* ht,
                                                   const int32_t* cu_seqlens, int B, int T, int H,
                                                   int K, int V, int N, int dtype, float scale,
                                                   int reverse, void* stream) {
  if (!q || !k || !v || !o) return tops_set_error(TOPS_ERR_NULL, "gla_fused_recurrent_fwd_decode: null tensor");
  int rc = fr_check("gla_fused_recurrent_fwd_decode", B, T, H, K, V, N, cu_seqlens, dtype);
  if (rc != TOPS_OK) return rc;
  FrParams p{q, k, v, gk, gv, h0, nullptr, nullptr, o, o32, ht, nullptr, nullptr, nullptr, nullptr,
             nullptr, cu_seqlens, B, T, H, K, V, N, (V + kFrBV - 1) / kFrBV, scale, reverse ? 1 : 0};
  hipStream_t s = (hipStream_t)stream;
  hipError_t e = dtype == TOPS_BF16 ? launch_fr_decode<uint16_t>(p, s) : launch_fr_decode<float>(p, s);
  if (e != hipSuccess) return tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
  return TOPS_OK;
}

extern "C" int tops_gla_fused_recurrent_fwd_decode_norm_gate(
    const void* q, const void* k, const void* v, const float* gk, const float* gv, const float* h0,
    const void* g, const float* weight, float eps, void* y, float* ht, const int32_t* cu_seqlens,
    int B, int T, int H, int K, int V, int N, int dtype, float scale, int reverse, void* stream) {
  if (!q || !k || !v || !y)
    return tops_set_error(TOPS_ERR_NULL, "gla_fused_recurrent_fwd_decode_norm_gate: null tensor");
  int rc = fr_check("gla_fused_recurrent_fwd_decode_norm_gate", B, T, H, K, V, N, cu_seqlens, dtype);
  if (rc != TOPS_OK) return rc;
  if (V > 128)
    return tops_set_error(TOPS_ERR_SHAPE,
                          "gla_fused_recurrent_fwd_decode_norm_gate: the fused norm needs V <= 128");
  if (!(eps >= 0.f))
    return tops_set_error(TOPS_ERR_SHAPE, "gla_fused_recurrent_fwd_decode_norm_gate: eps must be >= 0");
  FrParams p{q, k, v, gk, gv, h0, nullptr, nullptr, y, nullptr, ht, nullptr, nullptr, nullptr, nullptr,
             nullptr, cu_seqlens, B, T, H, K, V, N, (V + kFrBV - 1) / kFrBV, scale, reverse ? 1 : 0};
  p.ng = g;
  p.nw = weight;
  p.neps = eps;
  p.ninv = 1.f / (float)V;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e = dtype == TOPS_BF16 ? launch_fr_decode<uint16_t, false, true>(p, s)
                                    : launch_fr_decode<float, false, true>(p, s);
  if (e != hipSuccess) return tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
  return TOPS_OK;
}

extern "C" int tops_gla_decode_conv_norm_gate(
    const void* xq, const void* xk, const void* xv, const float* conv_w_q, const float* conv_w_k,
    const float* conv_w_v, const float* conv_b_q, const float* conv_b_k, const float* conv_b_v,
    const float* cache_q, const float* cache_k, const float* cache_v, float* cache_q_out,
    float* cache_k_out, float* cache_v_out, int W, int activation, const float* gk,
    const float* h0, const void* g, const float* weight, float eps, void* y, int y_fp32,
    float* ht, const int32_t* cu_seqlens, int B, int T, int H, int K, int V, int N, int dtype,
    float scale, void* stream) {
  if (!xq || !xk || !xv || !conv_w_q || !conv_w_k || !conv_w_v || !y)
    return tops_set_error(TOPS_ERR_NULL, "gla_decode_conv_norm_gate: null tensor");
  int rc = fr_check("gla_decode_conv_norm_gate", B, T, H, K, V, N, cu_seqlens, dtype);
  if (rc != TOPS_OK) return rc;
  if (V > 128)
    return tops_set_error(TOPS_ERR_SHAPE, "gla_decode_conv_norm_gate: the fused norm needs V <= 128");
  if (W < 1 || W > 8)
    return tops_set_error(TOPS_ERR_SHAPE, "gla_decode_conv_norm_gate: need 1 <= W <= 8");
  if (!(eps >= 0.f))
    return tops_set_error(TOPS_ERR_SHAPE, "gla_decode_conv_norm_gate: eps must be >= 0");
  FrParams p{xq, xk, xv, gk, nullptr, h0, nullptr, nullptr, y, nullptr, ht, nullptr, nullptr,
             nullptr, nullptr, nullptr, cu_seqlens, B, T, H, K, V, N, (V + kFrBV - 1) / kFrBV,
             scale, 0};
  p.ng = g;
  p.nw = weight;
  p.neps = eps;
  p.ninv = 1.f / (float)V;
  const float* cw[3] = {conv_w_q, conv_w_k, conv_w_v};
  const float* cb[3] = {conv_b_q, conv_b_k, conv_b_v};
  const float* ci[3] = {cache_q, cache_k, cache_v};
  float* co[3] = {cache_q_out, cache_k_out, cache_v_out};
  for (int i = 0; i < 3; ++i) {
    p.cw[i] = cw[i];
    p.cb[i] = cb[i];
    p.cci[i] = ci[i];
    p.cco[i] = co[i];
  }
  p.cW = W;
  p.cact = activation ? 1 : 0;
  p.y32 = y_fp32 ? 1 : 0;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e = dtype == TOPS_BF16 ? launch_fr_decode_conv<uint16_t>(p, s)
                                    : launch_fr_decode_conv<float>(p, s);
  if (e != hipSuccess) return tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
  return TOPS_OK;
}

extern "C" int tops_kda_fused_recurrent_fwd_decode(const void* q, const void* k, const void* v,
                                                   const float* g, const float* beta,
                                                   const float* h0, void* o, float* ht,
                                                   const int32_t* cu_seqlens, int B, int T, int H,
                                                   int K, int V, int N, int dtype, float scale,
                                                   void* stream) {
  if (!q || !k || !v || !g || !beta || !o)
    return tops_set_error(TOPS_ERR_NULL, "kda_fused_recurrent_fwd_decode: null tensor");
  int rc = fr_check("kda_fused_recurrent_fwd_decode", B, T, H, K, V, N, cu_seqlens, dtype);
  if (rc != TOPS_OK) return rc;
  FrParams p{q, k, v, g, nullptr, h0, nullptr, nullptr, o, nullptr, ht, nullptr, nullptr, nullptr,
             nullptr, nullptr, cu_seqlens, B, T, H, K, V, N, (V + kFrBV - 1) / kFrBV, scale, 0, beta};
  hipStream_t s = (hipStream_t)stream;
  hipError_t e = dtype == TOPS_BF16 ? launch_fr_decode<uint16_t, true>(p, s)
                                    : launch_fr_decode<float, true>(p, s);
  if (e != hipSuccess) return tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
  return TOPS_OK;
}

extern "C" int tops_gla_fused_recurrent_bwd(const void* q, const void* k, const void* v,
                                            const float* gk, const float* gv, const float* o32,
                                            const void* do_, const float* dht, const float* h0,
                                            void* dq, void* dk, void* dv, float* dgk, float* dgv,
                                            float* dh0, float* workspace,
                                            const int32_t* cu_seqlens, int B, int T, int H, int K,
                                            int V, int N, int dtype, float scale, int reverse,
                                            void* stream) {
  if (!q || !k || !v || !do_ || !dq || !dk || !dv || !workspace)
    return tops_set_error(TOPS_ERR_NULL, "gla_fused_recurrent_bwd: null tensor");
  if ((gk && !dgk) || (gv && (!dgv || !o32)))
    return tops_set_error(TOPS_ERR_NULL, "gla_fused_recurrent_bwd: gate gradients need dgk / dgv (and o)");
  int rc = fr_check("gla_fused_recurrent_bwd", B, T, H, K, V, N, cu_seqlens, dtype);
  if (rc != TOPS_OK) return rc;
  const int NV = (V + kFrBV - 1) / kFrBV;
  float* dq_part = workspace;
  float* dk_part = dq_part + (size_t)NV * B * T * H * K;
  float* h_fin = dk_part + (size_t)NV * B * T * H * K;
  float* dv32 = gv ? h_fin + (size_t)N * H * K * V : nullptr;
  FrParams p{q, k, v, gk, gv, h0, dht, do_, nullptr, nullptr, dh0, h_fin, dq_part, dk_part, dv, dv32,
             cu_seqlens, B, T, H, K, V, N, NV, scale, reverse ? 1 : 0};
  hipStream_t s = (hipStream_t)stream;
  hipError_t e = dtype == TOPS_BF16 ? launch_fr<uint16_t, true>(p, s) : launch_fr<float, true>(p, s);
  if (e != hipSuccess) return tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
  FrFinishParams f{q, k, v, o32, do_, dv32, dht, h_fin, dq_part, dk_part, dq, dk, gk ? dgk : nullptr,
                   gv ? dgv : nullptr, cu_seqlens, B, T, H, K, V, N, NV, reverse ? 1 : 0};
  if (dtype == TOPS_BF16)
    hipLaunchKernelGGL((fr_finish_kernel<uint16_t>), dim3(H * N), dim3(256), 0, s, f);
  else
    hipLaunchKernelGGL((fr_finish_kernel<float>), dim3(H * N), dim3(256), 0, s, f);
  e = hipGetLastError();
  if (e != hipSuccess) return tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
  return TOPS_OK;
}
