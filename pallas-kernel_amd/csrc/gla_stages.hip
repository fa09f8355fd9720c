// The separately callable stages of chunked GLA, for gfx950: the chunk-local gate cumsum, the
// inter-chunk state recurrence (forward states and reverse state gradients), the intra-chunk
// attention matrix, the output, and the four backward pieces (dA, dv, intra dq/dk, inter
// dq/dk + dg).  The fused sweeps (gla_sweep.hip, gla_dqkg.hip) compute the same quantities
// without writing the intermediates; these kernels exist so that callers of the reference's
// stage functions (tops/ops/gla/chunk.py:20-760, tops/ops/common/chunk_h.py,
// tops/ops/common/cumsum.py) get them on the GPU with the same shapes and meaning.
//
// Arithmetic is fp32 throughout: products go through v_mfma_f32_16x16x4_f32 (exact fp32
// multiplies, fp32 accumulation -- the reference's Precision.HIGHEST), operands staged in LDS
// as fp32 tiles of at most 64 contraction columns.  One workgroup (4 waves) per (chunk, head)
// or (chunk, head, 64-column tile); the recurrence runs one workgroup per (sequence, head,
// 64-column V tile) walking the chunks in order, as the reference's refs do.
//
// 16x16x4 fp32 MFMA lane layout (lane l, r = l % 16, q = l / 16):
//   A operand A[r][q], B operand B[q][r], result D[4q + i][r] in element i.
#include <math.h>
#include <stdio.h>

#include "tops_common.h"
#include "tops_hip.h"

namespace tops {
namespace {

constexpr int NTH = 256;   // 4 waves
constexpr int SL = 64;     // contraction / column slice
constexpr int LD = SL + 4; // padded row of a 64-wide LDS tile

__device__ __forceinline__ f32x4 mf4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

template <typename T> __device__ __forceinline__ float ldx(const T* p, long long i) {
  return In<T>::ld(p + i);
}

// ------------------------------------------------------------------ chunk-local cumsum
// tops/ops/gla/chunk.py:55-107 (K1) and :110-198: inclusive prefix sum (suffix sum when
// reverse) of each chunk, then * scale.  One thread per (chunk, head, column).
template <typename TIn, typename TOut>
__global__ void __launch_bounds__(NTH) local_cumsum_kernel(
    const TIn* __restrict__ g, TOut* __restrict__ out, const int32_t* __restrict__ cu,
    const int32_t* __restrict__ offs, const int32_t* __restrict__ cmap, int T, int H, int S,
    int C, int head_first, int reverse, float scale, int tiles) {
  const int HS = H * S;
  const int c = blockIdx.x / tiles;
  const int col = (blockIdx.x - c * tiles) * NTH + threadIdx.x;
  if (col >= HS) return;
  int b, t0, len;
  if (cu) {
    const int n = cmap[c];
    b = 0;
    t0 = cu[n] + (c - offs[n]) * C;
    len = min(C, cu[n + 1] - t0);
  } else {
    const int nt = (T + C - 1) / C;
    b = c / nt;
    t0 = (c - b * nt) * C;
    len = min(C, T - t0);
  }
  long long base, step;
  if (head_first) {
    const int h = col / S;
    base = (((long long)b * H + h) * T + t0) * S + (col - h * S);
    step = S;
  } else {
    base = ((long long)b * T + t0) * HS + col;
    step = HS;
  }
  float acc = 0.f;
  if (!reverse) {
    for (int t = 0; t < len; ++t) {
      acc += ldx(g, base + t * step);
      In<TOut>::st(out + base + t * step, acc * scale);
    }
  } else {
    for (int t = len - 1; t >= 0; --t) {
      acc += ldx(g, base + t * step);
      In<TOut>::st(out + base + t * step, acc * scale);
    }
  }
}

// ------------------------------------------------------------------ state recurrence
// Forward (tops/ops/common/chunk_h.py:363-489, tops/ops/gla/chunk.py:206-292): emit the
// state before each chunk, then S <- S * exp(G_last) + (x * exp(G_last - G))^T y with
// x = k, y = v.  Reverse (chunk_h.py:575-682): emit dS (gradient w.r.t. the state after
// the chunk), then dS <- dS * exp(G_last) + (x * scale * exp(G))^T y with x = q, y = do.
// G[t][c] = gk[t][c] + g[t] + gamma * (t_in_chunk + 1), each term optional.
struct RecArgs {
  const float* gk;     // [tokens, H, K] chunk-local cumsum or null
  const float* g;      // [tokens, H] chunk-local cumsum or null
  const float* gamma;  // [H] or null
  const float* s0;     // [N, H, K, V] or null
  float* sfin;         // [N, H, K, V] or null
  const int32_t* cu;   // [N + 1] (multiples of C) or null
  int T, H, K, V, C, NT, every;  // every: states are written every `every` chunks
  float scale;
  int reverse;
};

constexpr int RB = 32;     // token rows staged per step
constexpr int KMAX = 256;

template <typename TIn, typename TSt>
__global__ void __launch_bounds__(NTH) state_rec_kernel(const TIn* __restrict__ x,
                                                        const TIn* __restrict__ y,
                                                        TSt* __restrict__ states, RecArgs a) {
  __shared__ float xs[RB * (KMAX + 4)];
  __shared__ float ys[RB * LD];
  __shared__ float gl_s[KMAX];
  const int n = blockIdx.x / a.H, h = blockIdx.x - n * a.H;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r = lane & 15, q = lane >> 4;
  const int K = a.K, V = a.V, C = a.C, H = a.H;
  const int ldx_ = K + 4;
  const int v0 = blockIdx.y * SL, vw = min(SL, V - v0);
  const bool active = 16 * w < vw;
  const int vcol = v0 + 16 * w + r;
  const int MT = K / 16;
  long long bos, chunk0;
  int nch;
  if (a.cu) {
    bos = a.cu[n];
    nch = (a.cu[n + 1] - a.cu[n]) / C;
    chunk0 = bos / C;
  } else {
    bos = (long long)n * a.T;
    nch = a.NT;
    chunk0 = (long long)n * a.NT;
  }
  const long long sbase = ((long long)n * H + h) * K;
  f32x4 acc[16];
#pragma unroll
  for (int m = 0; m < 16; ++m) {
    acc[m] = zero4();
    if (m < MT && active && a.s0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[m][i] = a.s0[(sbase + 16 * m + 4 * q + i) * V + vcol];
    }
  }
  auto gate = [&](long long tok, int tc, int c) -> float {
    float G = 0.f;
    if (a.gk) G += a.gk[(tok * H + h) * K + c];
    if (a.g) G += a.g[tok * H + h];
    if (a.gamma) G += a.gamma[h] * (float)(tc + 1);
    return G;
  };
  for (int it = 0; it < nch; ++it) {
    const int ci = a.reverse ? nch - 1 - it : it;
    const long long tok0 = bos + (long long)ci * C;
    if (active && ci % a.every == 0) {
      const long long sidx = (chunk0 + ci) / a.every;
      TSt* dst = states + ((sidx * H + h) * K) * V + vcol;
#pragma unroll
      for (int m = 0; m < 16; ++m)
        if (m < MT) {
#pragma unroll
          for (int i = 0; i < 4; ++i) In<TSt>::st(dst + (long long)(16 * m + 4 * q + i) * V, acc[m][i]);
        }
    }
    for (int c = tid; c < K; c += NTH) gl_s[c] = gate(tok0 + C - 1, C - 1, c);
    __syncthreads();
#pragma unroll
    for (int m = 0; m < 16; ++m)
      if (m < MT) {
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[m][i] *= expf(gl_s[16 * m + 4 * q + i]);
      }
    const int rows = min(RB, C);
    for (int rb = 0; rb < C; rb += rows) {
      for (int idx = tid; idx < rows * K; idx += NTH) {
        const int rr = idx / K, c = idx - rr * K;
        const long long tok = tok0 + rb + rr;
        const float G = gate(tok, rb + rr, c);
        const float f = a.reverse ? a.scale * expf(G) : expf(gl_s[c] - G);
        xs[rr * ldx_ + c] = ldx(x, (tok * H + h) * K + c) * f;
      }
      for (int idx = tid; idx < rows * SL; idx += NTH) {
        const int rr = idx >> 6, c = idx & 63;
        const long long tok = tok0 + rb + rr;
        ys[rr * LD + c] = c < vw ? ldx(y, (tok * H + h) * V + v0 + c) : 0.f;
      }
      __syncthreads();
      if (active) {
        for (int s = 0; s < rows / 4; ++s) {
          const float bv = ys[(4 * s + q) * LD + 16 * w + r];
          const float* xr = xs + (4 * s + q) * ldx_ + r;
#pragma unroll
          for (int m = 0; m < 16; ++m)
            if (m < MT) acc[m] = mf4(xr[16 * m], bv, acc[m]);
        }
      }
      __syncthreads();
    }
  }
  if (a.sfin && active) {
#pragma unroll
    for (int m = 0; m < 16; ++m)
      if (m < MT) {
#pragma unroll
        for (int i = 0; i < 4; ++i) a.sfin[(sbase + 16 * m + 4 * q + i) * V + vcol] = acc[m][i];
      }
  }
}

// ------------------------------------------------------------------ chunk geometry
// Chunk-parallel stages: T % C == 0, chunks of the flattened [B*T] token axis in order
// (a varlen batch with chunk-aligned boundaries is the same layout).
struct Geo {
  int H, K, V, C;
  long long tok0;  // first token of this workgroup's chunk
  long long chunk; // global chunk index
  int h;
  __device__ Geo(int H_, int K_, int V_, int C_) : H(H_), K(K_), V(V_), C(C_) {
    chunk = blockIdx.x / H_;
    h = blockIdx.x - (int)chunk * H_;
    tok0 = chunk * C_;
  }
  __device__ long long kof(int row, int c) const { return ((tok0 + row) * H + h) * K + c; }
  __device__ long long vof(int row, int c) const { return ((tok0 + row) * H + h) * V + c; }
  __device__ long long aof(int row, int j) const { return ((tok0 + row) * H + h) * C + j; }
  __device__ long long sof(int kk, int c) const { return ((chunk * H + h) * K + kk) * V + c; }
};

// A[i][j] = scale * sum_c q[i][c] e^{G[i][c] - Gm[c]} k[j][c] e^{Gm[c] - G[j][c]}, full square,
// Gm = (G[0] + G[C-1]) / 2 (tops/ops/gla/chunk.py:300-438).  Tiles (mi, mj) over the waves.
template <typename TIn>
__global__ void __launch_bounds__(NTH) intra_A_kernel(const TIn* __restrict__ q,
                                                      const TIn* __restrict__ k,
                                                      const float* __restrict__ g,
                                                      float* __restrict__ A, int H, int K, int C,
                                                      float scale) {
  __shared__ float qs[128 * LD], ks[128 * LD], gm_s[SL];
  const Geo e(H, K, 0, C);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r = lane & 15, qq = lane >> 4;
  const int nt = C / 16, tiles = nt * nt;
  f32x4 acc[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) acc[j] = zero4();
  for (int k0 = 0; k0 < K; k0 += SL) {
    const int kw = min(SL, K - k0);
    if (tid < kw) gm_s[tid] = 0.5f * (g[e.kof(0, k0 + tid)] + g[e.kof(C - 1, k0 + tid)]);
    __syncthreads();
    for (int idx = tid; idx < C * SL; idx += NTH) {
      const int rr = idx >> 6, c = idx & 63;
      float qv = 0.f, kv = 0.f;
      if (c < kw) {
        const long long o = e.kof(rr, k0 + c);
        const float gg = g[o];
        qv = ldx(q, o) * expf(gg - gm_s[c]);
        kv = ldx(k, o) * expf(gm_s[c] - gg);
      }
      qs[rr * LD + c] = qv;
      ks[rr * LD + c] = kv;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int t = w + 4 * j;
      if (t < tiles) {
        const int mi = t / nt, mj = t - mi * nt;
        const float* ap = qs + (16 * mi + r) * LD + qq;
        const float* bp = ks + (16 * mj + r) * LD + qq;
        for (int s = 0; s < kw / 4; ++s) acc[j] = mf4(ap[4 * s], bp[4 * s], acc[j]);
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int t = w + 4 * j;
    if (t < tiles) {
      const int mi = t / nt, mj = t - mi * nt;
#pragma unroll
      for (int i = 0; i < 4; ++i) A[e.aof(16 * mi + 4 * qq + i, 16 * mj + r)] = acc[j][i] * scale;
    }
  }
}

// o = scale * (q e^{G - Gm}) (h e^{Gm}) + tril(A) v  (tops/ops/gla/chunk.py:1279-1440);
// exp2 instead of exp when use_exp2.  Grid (chunks * H, V tiles); wave w owns 16 columns.
template <typename TIn, typename TOut>
__global__ void __launch_bounds__(NTH) o_gk_kernel(const TIn* __restrict__ q,
                                                   const TIn* __restrict__ v,
                                                   const float* __restrict__ g,
                                                   const float* __restrict__ A,
                                                   const float* __restrict__ hs,
                                                   TOut* __restrict__ o, int H, int K, int V,
                                                   int C, float scale, int use_exp2) {
  __shared__ float as[128 * LD], bs[SL * LD], gm_s[SL];
  const Geo e(H, K, V, C);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r = lane & 15, qq = lane >> 4;
  const int v0 = blockIdx.y * SL, vw = min(SL, V - v0);
  const bool active = 16 * w < vw;
  const int MR = C / 16;
  auto E = [&](float t) { return use_exp2 ? exp2f(t) : expf(t); };
  f32x4 acc[8];
#pragma unroll
  for (int m = 0; m < 8; ++m) acc[m] = zero4();
  for (int k0 = 0; k0 < K; k0 += SL) {
    const int kw = min(SL, K - k0);
    if (tid < kw) gm_s[tid] = 0.5f * (g[e.kof(0, k0 + tid)] + g[e.kof(C - 1, k0 + tid)]);
    __syncthreads();
    for (int idx = tid; idx < C * SL; idx += NTH) {
      const int rr = idx >> 6, c = idx & 63;
      float qv = 0.f;
      if (c < kw) {
        const long long of = e.kof(rr, k0 + c);
        qv = ldx(q, of) * E(g[of] - gm_s[c]);
      }
      as[rr * LD + c] = qv;
    }
    for (int idx = tid; idx < SL * SL; idx += NTH) {
      const int kk = idx >> 6, c = idx & 63;
      bs[kk * LD + c] = (kk < kw && c < vw) ? hs[e.sof(k0 + kk, v0 + c)] * E(gm_s[kk]) : 0.f;
    }
    __syncthreads();
    if (active) {
      for (int s = 0; s < kw / 4; ++s) {
        const float b = bs[(4 * s + qq) * LD + 16 * w + r];
#pragma unroll
        for (int m = 0; m < 8; ++m)
          if (m < MR) acc[m] = mf4(as[(16 * m + r) * LD + 4 * s + qq], b, acc[m]);
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int m = 0; m < 8; ++m) acc[m] *= scale;
  for (int j0 = 0; j0 < C; j0 += SL) {
    const int jw = min(SL, C - j0);
    for (int idx = tid; idx < C * SL; idx += NTH) {
      const int rr = idx >> 6, c = idx & 63;
      as[rr * LD + c] = (c < jw && j0 + c <= rr) ? A[e.aof(rr, j0 + c)] : 0.f;
    }
    for (int idx = tid; idx < SL * SL; idx += NTH) {
      const int jj = idx >> 6, c = idx & 63;
      bs[jj * LD + c] = (jj < jw && c < vw) ? ldx(v, e.vof(j0 + jj, v0 + c)) : 0.f;
    }
    __syncthreads();
    if (active) {
      for (int s = 0; s < jw / 4; ++s) {
        const float b = bs[(4 * s + qq) * LD + 16 * w + r];
#pragma unroll
        for (int m = 0; m < 8; ++m)
          if (m < MR) acc[m] = mf4(as[(16 * m + r) * LD + 4 * s + qq], b, acc[m]);
      }
    }
    __syncthreads();
  }
  if (active) {
#pragma unroll
    for (int m = 0; m < 8; ++m)
      if (m < MR) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          In<TOut>::st(o + e.vof(16 * m + 4 * qq + i, v0 + 16 * w + r), acc[m][i]);
      }
  }
}

// dA[i][j] = scale * do[i] . v[j] for j <= i, else 0 (tops/ops/gla/chunk.py:509-549).
template <typename TIn, typename TOut>
__global__ void __launch_bounds__(NTH) dA_kernel(const TIn* __restrict__ v,
                                                 const TIn* __restrict__ dov,
                                                 TOut* __restrict__ dA, int H, int V, int C,
                                                 float scale) {
  __shared__ float ds[128 * LD], vs[128 * LD];
  const Geo e(H, 0, V, C);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r = lane & 15, qq = lane >> 4;
  const int nt = C / 16, tiles = nt * nt;
  f32x4 acc[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) acc[j] = zero4();
  for (int v0 = 0; v0 < V; v0 += SL) {
    const int vw = min(SL, V - v0);
    for (int idx = tid; idx < C * SL; idx += NTH) {
      const int rr = idx >> 6, c = idx & 63;
      const bool ok = c < vw;
      ds[rr * LD + c] = ok ? ldx(dov, e.vof(rr, v0 + c)) : 0.f;
      vs[rr * LD + c] = ok ? ldx(v, e.vof(rr, v0 + c)) : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int t = w + 4 * j;
      if (t < tiles) {
        const int mi = t / nt, mj = t - mi * nt;
        if (mj <= mi) {
          const float* ap = ds + (16 * mi + r) * LD + qq;
          const float* bp = vs + (16 * mj + r) * LD + qq;
          for (int s = 0; s < vw / 4; ++s) acc[j] = mf4(ap[4 * s], bp[4 * s], acc[j]);
        }
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int t = w + 4 * j;
    if (t < tiles) {
      const int mi = t / nt, mj = t - mi * nt;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 16 * mi + 4 * qq + i, col = 16 * mj + r;
        In<TOut>::st(dA + e.aof(row, col), col <= row ? acc[j][i] * scale : 0.f);
      }
    }
  }
}

// dv[j] = sum_{i >= j} A[i][j] do[i] + (k[j] e^{G_last - G[j]}) dh  (chunk.py:552-605).
template <typename TIn>
__global__ void __launch_bounds__(NTH) dv_kernel(const TIn* __restrict__ k,
                                                 const TIn* __restrict__ dov,
                                                 const float* __restrict__ g,
                                                 const float* __restrict__ A,
                                                 const float* __restrict__ dh,
                                                 float* __restrict__ dv, int H, int K, int V,
                                                 int C) {
  __shared__ float as[128 * LD], bs[SL * LD], gn_s[SL];
  const Geo e(H, K, V, C);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r = lane & 15, qq = lane >> 4;
  const int v0 = blockIdx.y * SL, vw = min(SL, V - v0);
  const bool active = 16 * w < vw;
  const int MR = C / 16, lda = C + 4;
  f32x4 acc[8];
#pragma unroll
  for (int m = 0; m < 8; ++m) acc[m] = zero4();
  // intra: contraction over i in slices of 64 rows; as[ii][j] = A[i0 + ii][j] (i >= j)
  for (int i0 = 0; i0 < C; i0 += SL) {
    const int iw = min(SL, C - i0);
    for (int idx = tid; idx < SL * C; idx += NTH) {
      const int ii = idx / C, j = idx - ii * C;
      as[ii * lda + j] = (ii < iw && i0 + ii >= j) ? A[e.aof(i0 + ii, j)] : 0.f;
    }
    for (int idx = tid; idx < SL * SL; idx += NTH) {
      const int ii = idx >> 6, c = idx & 63;
      bs[ii * LD + c] = (ii < iw && c < vw) ? ldx(dov, e.vof(i0 + ii, v0 + c)) : 0.f;
    }
    __syncthreads();
    if (active) {
      for (int s = 0; s < iw / 4; ++s) {
        const float b = bs[(4 * s + qq) * LD + 16 * w + r];
#pragma unroll
        for (int m = 0; m < 8; ++m)
          if (m < MR) acc[m] = mf4(as[(4 * s + qq) * lda + 16 * m + r], b, acc[m]);
      }
    }
    __syncthreads();
  }
  // inter: contraction over the K channels in slices of 64
  for (int k0 = 0; k0 < K; k0 += SL) {
    const int kw = min(SL, K - k0);
    if (tid < kw) gn_s[tid] = g[e.kof(C - 1, k0 + tid)];
    __syncthreads();
    for (int idx = tid; idx < C * SL; idx += NTH) {
      const int j = idx >> 6, c = idx & 63;
      float kv = 0.f;
      if (c < kw) {
        const long long of = e.kof(j, k0 + c);
        kv = ldx(k, of) * expf(gn_s[c] - g[of]);
      }
      as[j * LD + c] = kv;
    }
    for (int idx = tid; idx < SL * SL; idx += NTH) {
      const int kk = idx >> 6, c = idx & 63;
      bs[kk * LD + c] = (kk < kw && c < vw) ? dh[e.sof(k0 + kk, v0 + c)] : 0.f;
    }
    __syncthreads();
    if (active) {
      for (int s = 0; s < kw / 4; ++s) {
        const float b = bs[(4 * s + qq) * LD + 16 * w + r];
#pragma unroll
        for (int m = 0; m < 8; ++m)
          if (m < MR) acc[m] = mf4(as[(16 * m + r) * LD + 4 * s + qq], b, acc[m]);
      }
    }
    __syncthreads();
  }
  if (active) {
#pragma unroll
    for (int m = 0; m < 8; ++m)
      if (m < MR) {
#pragma unroll
        for (int i = 0; i < 4; ++i) dv[e.vof(16 * m + 4 * qq + i, v0 + 16 * w + r)] = acc[m][i];
      }
  }
}

// dq[i] = e^{G[i] - Gm} sum_j dA[i][j] k[j] e^{Gm - G[j]},
// dk[j] = e^{Gm - G[j]} sum_i dA[i][j] q[i] e^{G[i] - Gm}  (chunk.py:608-662; dA used as
// given, no mask).  Grid (chunks * H, 64-channel tiles of K).
template <typename TIn>
__global__ void __launch_bounds__(NTH) dqk_intra_kernel(const TIn* __restrict__ q,
                                                        const TIn* __restrict__ k,
                                                        const float* __restrict__ g,
                                                        const float* __restrict__ dA,
                                                        float* __restrict__ dq,
                                                        float* __restrict__ dk, int H, int K,
                                                        int C) {
  __shared__ float as[128 * LD], bs[SL * LD], gm_s[SL];
  const Geo e(H, K, 0, C);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r = lane & 15, qq = lane >> 4;
  const int k0 = blockIdx.y * SL, kw = min(SL, K - k0);
  const bool active = 16 * w < kw;
  const int MR = C / 16, lda = C + 4;
  const int ch = k0 + 16 * w + r;
  if (tid < kw) gm_s[tid] = 0.5f * (g[e.kof(0, k0 + tid)] + g[e.kof(C - 1, k0 + tid)]);
  __syncthreads();
  f32x4 acc[8];
#pragma unroll
  for (int m = 0; m < 8; ++m) acc[m] = zero4();
  for (int j0 = 0; j0 < C; j0 += SL) {
    const int jw = min(SL, C - j0);
    for (int idx = tid; idx < C * SL; idx += NTH) {
      const int i = idx >> 6, c = idx & 63;
      as[i * LD + c] = c < jw ? dA[e.aof(i, j0 + c)] : 0.f;
    }
    for (int idx = tid; idx < SL * SL; idx += NTH) {
      const int jj = idx >> 6, c = idx & 63;
      float kv = 0.f;
      if (jj < jw && c < kw) {
        const long long of = e.kof(j0 + jj, k0 + c);
        kv = ldx(k, of) * expf(gm_s[c] - g[of]);
      }
      bs[jj * LD + c] = kv;
    }
    __syncthreads();
    if (active) {
      for (int s = 0; s < jw / 4; ++s) {
        const float b = bs[(4 * s + qq) * LD + 16 * w + r];
#pragma unroll
        for (int m = 0; m < 8; ++m)
          if (m < MR) acc[m] = mf4(as[(16 * m + r) * LD + 4 * s + qq], b, acc[m]);
      }
    }
    __syncthreads();
  }
  if (active) {
    const float gm = gm_s[16 * w + r];
#pragma unroll
    for (int m = 0; m < 8; ++m)
      if (m < MR) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const long long of = e.kof(16 * m + 4 * qq + i, ch);
          dq[of] = expf(g[of] - gm) * acc[m][i];
        }
      }
  }
#pragma unroll
  for (int m = 0; m < 8; ++m) acc[m] = zero4();
  for (int i0 = 0; i0 < C; i0 += SL) {
    const int iw = min(SL, C - i0);
    for (int idx = tid; idx < SL * C; idx += NTH) {
      const int ii = idx / C, j = idx - ii * C;
      as[ii * lda + j] = ii < iw ? dA[e.aof(i0 + ii, j)] : 0.f;
    }
    for (int idx = tid; idx < SL * SL; idx += NTH) {
      const int ii = idx >> 6, c = idx & 63;
      float qv = 0.f;
      if (ii < iw && c < kw) {
        const long long of = e.kof(i0 + ii, k0 + c);
        qv = ldx(q, of) * expf(g[of] - gm_s[c]);
      }
      bs[ii * LD + c] = qv;
    }
    __syncthreads();
    if (active) {
      for (int s = 0; s < iw / 4; ++s) {
        const float b = bs[(4 * s + qq) * LD + 16 * w + r];
#pragma unroll
        for (int m = 0; m < 8; ++m)
          if (m < MR) acc[m] = mf4(as[(4 * s + qq) * lda + 16 * m + r], b, acc[m]);
      }
    }
    __syncthreads();
  }
  if (active) {
    const float gm = gm_s[16 * w + r];
#pragma unroll
    for (int m = 0; m < 8; ++m)
      if (m < MR) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const long long of = e.kof(16 * m + 4 * qq + i, ch);
          dk[of] = expf(gm - g[of]) * acc[m][i];
        }
      }
  }
}

// Inter-chunk dq / dk and the gate gradient (chunk.py:665-760):
//   dq' = dq + scale e^{G - Gm} (do (h e^{Gm})^T),  dk' = dk + e^{G_last - G} (v dh^T)
//   dg  = revcumsum_rows(q dq' - k dk') + e^{G_last} sum_v(h dh) + sum_rows(dk_inter k)
// Grid (chunks * H, 64-channel tiles of K); V contracted in slices of 64.
template <typename TIn>
__global__ void __launch_bounds__(NTH) dqkg_kernel(
    const TIn* __restrict__ q, const TIn* __restrict__ k, const TIn* __restrict__ v,
    const TIn* __restrict__ dov, const float* __restrict__ g, const float* __restrict__ hs,
    const float* __restrict__ dh, const float* __restrict__ dq_in,
    const float* __restrict__ dk_in, float* __restrict__ dq_out, float* __restrict__ dk_out,
    float* __restrict__ dg, int H, int K, int V, int C, float scale) {
  __shared__ float ds[128 * LD], vs[128 * LD], hh[SL * LD], dd[SL * LD], hd_s[SL];
  const Geo e(H, K, V, C);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r = lane & 15, qq = lane >> 4;
  const int k0 = blockIdx.y * SL, kw = min(SL, K - k0);
  const bool active = 16 * w < kw;
  const int MR = C / 16;
  f32x4 aq[8], ak[8];
#pragma unroll
  for (int m = 0; m < 8; ++m) aq[m] = ak[m] = zero4();
  float hd = 0.f;
  for (int v0 = 0; v0 < V; v0 += SL) {
    const int vw = min(SL, V - v0);
    for (int idx = tid; idx < C * SL; idx += NTH) {
      const int rr = idx >> 6, c = idx & 63;
      const bool ok = c < vw;
      ds[rr * LD + c] = ok ? ldx(dov, e.vof(rr, v0 + c)) : 0.f;
      vs[rr * LD + c] = ok ? ldx(v, e.vof(rr, v0 + c)) : 0.f;
    }
    for (int idx = tid; idx < SL * SL; idx += NTH) {
      const int kk = idx >> 6, c = idx & 63;
      const bool ok = kk < kw && c < vw;
      hh[kk * LD + c] = ok ? hs[e.sof(k0 + kk, v0 + c)] : 0.f;
      dd[kk * LD + c] = ok ? dh[e.sof(k0 + kk, v0 + c)] : 0.f;
    }
    __syncthreads();
    if (tid < kw)
      for (int c = 0; c < vw; ++c) hd += hh[tid * LD + c] * dd[tid * LD + c];
    if (active) {
      for (int s = 0; s < vw / 4; ++s) {
        const float bh = hh[(16 * w + r) * LD + 4 * s + qq];
        const float bd = dd[(16 * w + r) * LD + 4 * s + qq];
#pragma unroll
        for (int m = 0; m < 8; ++m)
          if (m < MR) {
            aq[m] = mf4(ds[(16 * m + r) * LD + 4 * s + qq], bh, aq[m]);
            ak[m] = mf4(vs[(16 * m + r) * LD + 4 * s + qq], bd, ak[m]);
          }
      }
    }
    __syncthreads();
  }
  // epilogue: ds <- q dq' - k dk', vs <- dk_inter k (rows x this tile's channels)
  if (tid < kw) hd_s[tid] = hd;
  if (active) {
    const int cl = 16 * w + r, ch = k0 + cl;
    const float g0 = g[e.kof(0, ch)], gl = g[e.kof(C - 1, ch)];
    const float gm = 0.5f * (g0 + gl), egm = expf(gm);
#pragma unroll
    for (int m = 0; m < 8; ++m)
      if (m < MR) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = 16 * m + 4 * qq + i;
          const long long of = e.kof(row, ch);
          const float gg = g[of];
          const float dqi = scale * expf(gg - gm) * (aq[m][i] * egm);
          const float dki = expf(gl - gg) * ak[m][i];
          const float dqt = dq_in[of] + dqi, dkt = dk_in[of] + dki;
          dq_out[of] = dqt;
          dk_out[of] = dkt;
          const float kv = ldx(k, of);
          ds[row * LD + cl] = ldx(q, of) * dqt - kv * dkt;
          vs[row * LD + cl] = dki * kv;
        }
      }
  }
  __syncthreads();
  if (tid < kw) {
    const int ch = k0 + tid;
    float cs = 0.f;
    for (int row = 0; row < C; ++row) cs += vs[row * LD + tid];
    const float dgk = expf(g[e.kof(C - 1, ch)]) * hd_s[tid] + cs;
    float run = 0.f;
    for (int row = C - 1; row >= 0; --row) {
      run += ds[row * LD + tid];
      dg[e.kof(row, ch)] = run + dgk;
    }
  }
}

// KDA intra-chunk backward (tops/ops/kda/chunk_intra.py:283-386 kernel, :477-574 wrapper):
// with E_ij = 2^{g_i - g_j} per channel (g: chunk-local cumsum in log2 units),
//   dq_i  = sum_{j<=i} dAqk_ij k_j E_ij,            dk_j += sum_{i>=j} dAqk_ij q_i E_ij
//   row_i = sum_{j<=i} dAkk_ij k_j E_ij,  db_i = row_i . k_i,  dk_i += beta_i row_i
//   dk_j += sum_{i>=j} beta_i dAkk_ij k_i E_ij
//   dg_i  = q_i dq_i + k_i beta_i row_i - k_i (dk_i from the two column sums)
// (the reference's gradients w.r.t. g carry no ln 2 factor).  One workgroup per (chunk, head)
// walks K in slices of 64; E is split as 2^{g_i - gm} 2^{gm - g_j} with gm the mean of the
// chunk's first and last gate rows.  Writes the intra parts only, fp32; C <= 64.
template <typename TIn>
__global__ void __launch_bounds__(NTH) kda_intra_bwd_kernel(
    const TIn* __restrict__ q, const TIn* __restrict__ k, const float* __restrict__ g,
    const float* __restrict__ beta, const float* __restrict__ dAqk,
    const float* __restrict__ dAkk, float* __restrict__ dq, float* __restrict__ dk,
    float* __restrict__ db, float* __restrict__ dg, int H, int K, int C) {
  __shared__ float aq[64 * LD], ak[64 * LD], qp[64 * LD], kp[64 * LD], kn[64 * LD];
  __shared__ float gm_s[SL], be_s[64], dbw[4][64];
  const Geo e(H, K, 0, C);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r = lane & 15, qq = lane >> 4;
  const int MR = C / 16, lda = C + 4;
  for (int idx = tid; idx < C * C; idx += NTH) {
    const int i = idx / C, j = idx - i * C;
    const bool ok = j <= i;
    aq[i * lda + j] = ok ? dAqk[e.aof(i, j)] : 0.f;
    ak[i * lda + j] = ok ? dAkk[e.aof(i, j)] : 0.f;
  }
  if (tid < C) be_s[tid] = beta[(e.tok0 + tid) * H + e.h];
  float dbl[4][4];
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int i = 0; i < 4; ++i) dbl[m][i] = 0.f;
  for (int k0 = 0; k0 < K; k0 += SL) {
    const int kw = min(SL, K - k0);
    const bool active = 16 * w < kw;
    if (tid < kw) gm_s[tid] = 0.5f * (g[e.kof(0, k0 + tid)] + g[e.kof(C - 1, k0 + tid)]);
    __syncthreads();
    for (int idx = tid; idx < C * SL; idx += NTH) {
      const int i = idx >> 6, c = idx & 63;
      float a = 0.f, b = 0.f, d = 0.f;
      if (c < kw) {
        const long long of = e.kof(i, k0 + c);
        const float t = g[of] - gm_s[c];
        const float ep = exp2f(t), en = exp2f(-t);
        const float kv = ldx(k, of);
        a = ldx(q, of) * ep;
        b = kv * ep;
        d = kv * en;
      }
      qp[i * LD + c] = a;
      kp[i * LD + c] = b;
      kn[i * LD + c] = d;
    }
    __syncthreads();
    if (active) {
      f32x4 p1[4], p2[4], p3[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) p1[m] = p2[m] = p3[m] = zero4();
      for (int s = 0; s < C / 4; ++s) {
        const int jr = 4 * s + qq;
        const float bn = kn[jr * LD + 16 * w + r];
        const float bq = qp[jr * LD + 16 * w + r];
        const float bk = kp[jr * LD + 16 * w + r];
        const float bej = be_s[jr];
#pragma unroll
        for (int m = 0; m < 4; ++m)
          if (m < MR) {
            p1[m] = mf4(aq[(16 * m + r) * lda + jr], bn, p1[m]);
            p2[m] = mf4(ak[(16 * m + r) * lda + jr], bn, p2[m]);
            p3[m] = mf4(aq[jr * lda + 16 * m + r], bq, p3[m]);
            p3[m] = mf4(ak[jr * lda + 16 * m + r] * bej, bk, p3[m]);
          }
      }
      const int ch = k0 + 16 * w + r;
      const float gm = gm_s[16 * w + r];
#pragma unroll
      for (int m = 0; m < 4; ++m)
        if (m < MR) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int row = 16 * m + 4 * qq + i;
            const long long of = e.kof(row, ch);
            const float t = g[of] - gm;
            const float ep = exp2f(t), en = exp2f(-t);
            const float qv = ldx(q, of), kv = ldx(k, of);
            const float dqv = p1[m][i] * ep, rowv = p2[m][i] * ep;
            const float dkrow = be_s[row] * rowv, dkcol = p3[m][i] * en;
            dq[of] = dqv;
            dk[of] = dkrow + dkcol;
            dg[of] = qv * dqv + kv * dkrow - kv * dkcol;
            dbl[m][i] += rowv * kv;
          }
        }
    }
    __syncthreads();
  }
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = dbl[m][i];
      v += __shfl_xor(v, 1, 64);
      v += __shfl_xor(v, 2, 64);
      v += __shfl_xor(v, 4, 64);
      v += __shfl_xor(v, 8, 64);
      if (r == 0 && m < MR) dbw[w][16 * m + 4 * qq + i] = v;
    }
  __syncthreads();
  if (tid < C) db[(e.tok0 + tid) * H + e.h] = dbw[0][tid] + dbw[1][tid] + dbw[2][tid] + dbw[3][tid];
}

bool chunk_ok(int C) { return C == 16 || C == 32 || C == 64 || C == 128; }

int launch_status() {
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? TOPS_OK : tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(err));
}

int stage_check(const char* fn, int B, int T, int H, int C, int dtype) {
  char buf[160];
  if (B <= 0 || T < 0 || H <= 0) {
    snprintf(buf, sizeof buf, "%s: need B > 0, T >= 0, H > 0", fn);
    return tops_set_error(TOPS_ERR_SHAPE, buf);
  }
  if (!chunk_ok(C)) {
    snprintf(buf, sizeof buf, "%s: chunk_size must be 16, 32, 64 or 128 (got %d)", fn, C);
    return tops_set_error(TOPS_ERR_UNSUPPORTED, buf);
  }
  if (T % C) {
    snprintf(buf, sizeof buf, "%s: T (%d) must be a multiple of chunk_size (%d)", fn, T, C);
    return tops_set_error(TOPS_ERR_SHAPE, buf);
  }
  if (dtype != TOPS_F32 && dtype != TOPS_BF16) {
    snprintf(buf, sizeof buf, "%s: dtype must be TOPS_F32 or TOPS_BF16", fn);
    return tops_set_error(TOPS_ERR_DTYPE, buf);
  }
  if ((long long)B * (T / C) * H >= (1LL << 31)) {
    snprintf(buf, sizeof buf, "%s: too many (chunk, head) pairs", fn);
    return tops_set_error(TOPS_ERR_SHAPE, buf);
  }
  return TOPS_OK;
}

int dim16(const char* fn, const char* name, int D) {
  if (D <= 0 || D % 16) {
    char buf[128];
    snprintf(buf, sizeof buf, "%s: %s must be a positive multiple of 16 (got %d)", fn, name, D);
    return tops_set_error(TOPS_ERR_UNSUPPORTED, buf);
  }
  return TOPS_OK;
}

}  // namespace
}  // namespace tops

using namespace tops;

#define STAGE_TRY(x)                 \
  do {                               \
    const int rc_ = (x);             \
    if (rc_ != TOPS_OK) return rc_;  \
  } while (0)

extern "C" int tops_chunk_local_cumsum(const void* g, int g_dtype, void* out, int out_dtype,
                                       const int32_t* cu_seqlens, const int32_t* chunk_offsets,
                                       const int32_t* chunk_map, int total_chunks, int B, int T,
                                       int H, int S, int chunk_size, int head_first, int reverse,
                                       float scale, void* stream) {
  if (!g || !out) return tops_set_error(TOPS_ERR_NULL, "chunk_local_cumsum: null tensor");
  if ((g_dtype != TOPS_F32 && g_dtype != TOPS_BF16) ||
      (out_dtype != TOPS_F32 && out_dtype != TOPS_BF16))
    return tops_set_error(TOPS_ERR_DTYPE, "chunk_local_cumsum: dtypes must be TOPS_F32 or TOPS_BF16");
  if (B <= 0 || T < 0 || H <= 0 || S <= 0 || chunk_size <= 0 ||
      (chunk_size & (chunk_size - 1)))
    return tops_set_error(TOPS_ERR_SHAPE,
                          "chunk_local_cumsum: need B, H, S > 0 and chunk_size a power of 2");
  if (cu_seqlens) {
    if (B != 1 || !chunk_offsets || !chunk_map)
      return tops_set_error(TOPS_ERR_SHAPE,
                            "chunk_local_cumsum: varlen needs B == 1, chunk_offsets and chunk_map");
  } else if (total_chunks != B * ((T + chunk_size - 1) / chunk_size)) {
    return tops_set_error(TOPS_ERR_SHAPE,
                          "chunk_local_cumsum: total_chunks must be B*ceil(T/chunk_size)");
  }
  if (total_chunks <= 0 || T == 0) return TOPS_OK;
  const int tiles = (H * S + NTH - 1) / NTH;
  if ((long long)total_chunks * tiles >= (1LL << 31))
    return tops_set_error(TOPS_ERR_SHAPE, "chunk_local_cumsum: too many chunks");
  hipStream_t s = (hipStream_t)stream;
  const int grid = total_chunks * tiles;
#define CS_LAUNCH(TI, TO)                                                                      \
  local_cumsum_kernel<TI, TO><<<grid, NTH, 0, s>>>((const TI*)g, (TO*)out, cu_seqlens,         \
                                                   chunk_offsets, chunk_map, T, H, S,          \
                                                   chunk_size, head_first, reverse, scale, tiles)
  if (g_dtype == TOPS_F32 && out_dtype == TOPS_F32) CS_LAUNCH(float, float);
  else if (g_dtype == TOPS_F32) CS_LAUNCH(float, uint16_t);
  else if (out_dtype == TOPS_F32) CS_LAUNCH(uint16_t, float);
  else CS_LAUNCH(uint16_t, uint16_t);
#undef CS_LAUNCH
  return launch_status();
}

extern "C" int tops_chunk_state_recurrence(const void* x, const void* y, int dtype,
                                           const float* gk, const float* g, const float* g_gamma,
                                           const float* s0, void* states, int states_dtype,
                                           float* s_final, const int32_t* cu_seqlens, int B,
                                           int T, int H, int K, int V, int N, int chunk_size,
                                           int every, int reverse, float scale, void* stream) {
  const char* fn = "chunk_state_recurrence";
  if (!x || !y || !states) return tops_set_error(TOPS_ERR_NULL, "chunk_state_recurrence: null tensor");
  STAGE_TRY(stage_check(fn, B, T, H, chunk_size, dtype));
  STAGE_TRY(dim16(fn, "K", K));
  STAGE_TRY(dim16(fn, "V", V));
  if (K > KMAX) return tops_set_error(TOPS_ERR_UNSUPPORTED, "chunk_state_recurrence: K must be <= 256");
  if (states_dtype != TOPS_F32 && states_dtype != TOPS_BF16)
    return tops_set_error(TOPS_ERR_DTYPE, "chunk_state_recurrence: states dtype must be TOPS_F32 or TOPS_BF16");
  if (every <= 0 || (T / chunk_size) % every || (cu_seqlens && every != 1))
    return tops_set_error(TOPS_ERR_SHAPE,
                          "chunk_state_recurrence: every must divide T / chunk_size (1 with cu_seqlens)");
  if (cu_seqlens ? (B != 1 || N <= 0) : N != B)
    return tops_set_error(TOPS_ERR_SHAPE, "chunk_state_recurrence: N must be B (or B == 1 with cu_seqlens)");
  if (T == 0) return TOPS_OK;
  RecArgs a{gk, g, g_gamma, s0, s_final, cu_seqlens, T, H, K, V, chunk_size, T / chunk_size,
            every, scale, reverse};
  const dim3 grid(N * H, (V + SL - 1) / SL);
  hipStream_t s = (hipStream_t)stream;
#define SR_LAUNCH(TI, TS) \
  state_rec_kernel<TI, TS><<<grid, NTH, 0, s>>>((const TI*)x, (const TI*)y, (TS*)states, a)
  if (dtype == TOPS_F32 && states_dtype == TOPS_F32) SR_LAUNCH(float, float);
  else if (dtype == TOPS_F32) SR_LAUNCH(float, uint16_t);
  else if (states_dtype == TOPS_F32) SR_LAUNCH(uint16_t, float);
  else SR_LAUNCH(uint16_t, uint16_t);
#undef SR_LAUNCH
  return launch_status();
}

extern "C" int tops_gla_stage_attn(const void* q, const void* k, int dtype, const float* g,
                                      float* A, int B, int T, int H, int K, int chunk_size,
                                      float scale, void* stream) {
  const char* fn = "gla_stage_attn";
  if (!q || !k || !g || !A) return tops_set_error(TOPS_ERR_NULL, "gla_stage_attn: null tensor");
  STAGE_TRY(stage_check(fn, B, T, H, chunk_size, dtype));
  STAGE_TRY(dim16(fn, "K", K));
  if (T == 0) return TOPS_OK;
  const int grid = B * (T / chunk_size) * H;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == TOPS_F32)
    intra_A_kernel<float><<<grid, NTH, 0, s>>>((const float*)q, (const float*)k, g, A, H, K,
                                               chunk_size, scale);
  else
    intra_A_kernel<uint16_t><<<grid, NTH, 0, s>>>((const uint16_t*)q, (const uint16_t*)k, g, A,
                                                  H, K, chunk_size, scale);
  return launch_status();
}

extern "C" int tops_gla_stage_o(const void* q, const void* v, int dtype, const float* g,
                                const float* A, const float* h, void* o, int B, int T, int H,
                                int K, int V, int chunk_size, float scale, int use_exp2,
                                void* stream) {
  const char* fn = "gla_stage_o";
  if (!q || !v || !g || !A || !h || !o) return tops_set_error(TOPS_ERR_NULL, "gla_stage_o: null tensor");
  STAGE_TRY(stage_check(fn, B, T, H, chunk_size, dtype));
  STAGE_TRY(dim16(fn, "K", K));
  STAGE_TRY(dim16(fn, "V", V));
  if (T == 0) return TOPS_OK;
  const dim3 grid(B * (T / chunk_size) * H, (V + SL - 1) / SL);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == TOPS_F32)
    o_gk_kernel<float, float><<<grid, NTH, 0, s>>>((const float*)q, (const float*)v, g, A, h,
                                                   (float*)o, H, K, V, chunk_size, scale,
                                                   use_exp2);
  else
    o_gk_kernel<uint16_t, uint16_t><<<grid, NTH, 0, s>>>((const uint16_t*)q, (const uint16_t*)v,
                                                         g, A, h, (uint16_t*)o, H, K, V,
                                                         chunk_size, scale, use_exp2);
  return launch_status();
}

extern "C" int tops_gla_stage_dattn(const void* v, const void* do_, int dtype, void* dA,
                                 int dA_dtype, int B, int T, int H, int V, int chunk_size,
                                 float scale, void* stream) {
  const char* fn = "gla_stage_dattn";
  if (!v || !do_ || !dA) return tops_set_error(TOPS_ERR_NULL, "gla_stage_dattn: null tensor");
  STAGE_TRY(stage_check(fn, B, T, H, chunk_size, dtype));
  STAGE_TRY(dim16(fn, "V", V));
  if (dA_dtype != TOPS_F32 && dA_dtype != TOPS_BF16)
    return tops_set_error(TOPS_ERR_DTYPE, "gla_stage_dattn: dA dtype must be TOPS_F32 or TOPS_BF16");
  if (T == 0) return TOPS_OK;
  const int grid = B * (T / chunk_size) * H;
  hipStream_t s = (hipStream_t)stream;
#define DA_LAUNCH(TI, TO)                                                                     \
  dA_kernel<TI, TO><<<grid, NTH, 0, s>>>((const TI*)v, (const TI*)do_, (TO*)dA, H, V,         \
                                         chunk_size, scale)
  if (dtype == TOPS_F32 && dA_dtype == TOPS_F32) DA_LAUNCH(float, float);
  else if (dtype == TOPS_F32) DA_LAUNCH(float, uint16_t);
  else if (dA_dtype == TOPS_F32) DA_LAUNCH(uint16_t, float);
  else DA_LAUNCH(uint16_t, uint16_t);
#undef DA_LAUNCH
  return launch_status();
}

extern "C" int tops_gla_stage_dv(const void* k, const void* do_, int dtype, const float* g,
                                 const float* A, const float* dh, float* dv, int B, int T, int H,
                                 int K, int V, int chunk_size, void* stream) {
  const char* fn = "gla_stage_dv";
  if (!k || !do_ || !g || !A || !dh || !dv) return tops_set_error(TOPS_ERR_NULL, "gla_stage_dv: null tensor");
  STAGE_TRY(stage_check(fn, B, T, H, chunk_size, dtype));
  STAGE_TRY(dim16(fn, "K", K));
  STAGE_TRY(dim16(fn, "V", V));
  if (T == 0) return TOPS_OK;
  const dim3 grid(B * (T / chunk_size) * H, (V + SL - 1) / SL);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == TOPS_F32)
    dv_kernel<float><<<grid, NTH, 0, s>>>((const float*)k, (const float*)do_, g, A, dh, dv, H, K,
                                          V, chunk_size);
  else
    dv_kernel<uint16_t><<<grid, NTH, 0, s>>>((const uint16_t*)k, (const uint16_t*)do_, g, A, dh,
                                             dv, H, K, V, chunk_size);
  return launch_status();
}

extern "C" int tops_gla_stage_dqk_intra(const void* q, const void* k, int dtype, const float* g,
                                        const float* dA, float* dq, float* dk, int B, int T,
                                        int H, int K, int chunk_size, void* stream) {
  const char* fn = "gla_stage_dqk_intra";
  if (!q || !k || !g || !dA || !dq || !dk)
    return tops_set_error(TOPS_ERR_NULL, "gla_stage_dqk_intra: null tensor");
  STAGE_TRY(stage_check(fn, B, T, H, chunk_size, dtype));
  STAGE_TRY(dim16(fn, "K", K));
  if (T == 0) return TOPS_OK;
  const dim3 grid(B * (T / chunk_size) * H, (K + SL - 1) / SL);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == TOPS_F32)
    dqk_intra_kernel<float><<<grid, NTH, 0, s>>>((const float*)q, (const float*)k, g, dA, dq, dk,
                                                 H, K, chunk_size);
  else
    dqk_intra_kernel<uint16_t><<<grid, NTH, 0, s>>>((const uint16_t*)q, (const uint16_t*)k, g,
                                                    dA, dq, dk, H, K, chunk_size);
  return launch_status();
}

extern "C" int tops_gla_stage_dqkg(const void* q, const void* k, const void* v, const void* do_,
                                   int dtype, const float* g, const float* h, const float* dh,
                                   const float* dq, const float* dk, float* dq_out,
                                   float* dk_out, float* dg, int B, int T, int H, int K, int V,
                                   int chunk_size, float scale, void* stream) {
  const char* fn = "gla_stage_dqkg";
  if (!q || !k || !v || !do_ || !g || !h || !dh || !dq || !dk || !dq_out || !dk_out || !dg)
    return tops_set_error(TOPS_ERR_NULL, "gla_stage_dqkg: null tensor");
  STAGE_TRY(stage_check(fn, B, T, H, chunk_size, dtype));
  STAGE_TRY(dim16(fn, "K", K));
  STAGE_TRY(dim16(fn, "V", V));
  if (T == 0) return TOPS_OK;
  const dim3 grid(B * (T / chunk_size) * H, (K + SL - 1) / SL);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == TOPS_F32)
    dqkg_kernel<float><<<grid, NTH, 0, s>>>((const float*)q, (const float*)k, (const float*)v,
                                            (const float*)do_, g, h, dh, dq, dk, dq_out, dk_out,
                                            dg, H, K, V, chunk_size, scale);
  else
    dqkg_kernel<uint16_t><<<grid, NTH, 0, s>>>((const uint16_t*)q, (const uint16_t*)k,
                                               (const uint16_t*)v, (const uint16_t*)do_, g, h,
                                               dh, dq, dk, dq_out, dk_out, dg, H, K, V,
                                               chunk_size, scale);
  return launch_status();
}

extern "C" int tops_kda_stage_intra_bwd(const void* q, const void* k, int dtype, const float* g,
                                        const float* beta, const float* dAqk, const float* dAkk,
                                        float* dq, float* dk, float* db, float* dg, int B, int T,
                                        int H, int K, int chunk_size, void* stream) {
  const char* fn = "kda_stage_intra_bwd";
  if (!q || !k || !g || !beta || !dAqk || !dAkk || !dq || !dk || !db || !dg)
    return tops_set_error(TOPS_ERR_NULL, "kda_stage_intra_bwd: null tensor");
  STAGE_TRY(stage_check(fn, B, T, H, chunk_size, dtype));
  STAGE_TRY(dim16(fn, "K", K));
  if (chunk_size > 64)
    return tops_set_error(TOPS_ERR_UNSUPPORTED, "kda_stage_intra_bwd: chunk_size must be 16, 32 or 64");
  if (T == 0) return TOPS_OK;
  const int grid = B * (T / chunk_size) * H;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == TOPS_F32)
    kda_intra_bwd_kernel<float><<<grid, NTH, 0, s>>>((const float*)q, (const float*)k, g, beta,
                                                     dAqk, dAkk, dq, dk, db, dg, H, K,
                                                     chunk_size);
  else
    kda_intra_bwd_kernel<uint16_t><<<grid, NTH, 0, s>>>((const uint16_t*)q, (const uint16_t*)k, g,
                                                        beta, dAqk, dAkk, dq, dk, db, dg, H, K,
                                                        chunk_size);
  return launch_status();
}
