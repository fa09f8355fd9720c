// The GLA layer's neighbours of the op, for gfx950: RMSNorm / FusedRMSNormGated on the
// output side and the causal depthwise ShortConvolution on the input side
// (tops/modules/layernorm.py, fused_norm_gate.py, convolution.py; used by
// tops/layers/gla.py:236-343).
//
// RMSNorm(-gated):  y = x * rsqrt(mean(x^2) + eps) * w * silu(g), computed in fp32 and
// stored in x's dtype.  Rows of D % 8 == 0, 64 <= D <= 2048 take the vector path: a row is
// spread over LPR lanes that each own runs of 8 consecutive elements (one 16-byte bf16
// access), a wave covers 64 / LPR rows and handles two such row groups per iteration so
// that several accesses per lane are in flight.  Other D use one wave per row with scalar
// accesses.  The backward keeps each workgroup's weight-gradient partial in registers and
// writes one partial row per workgroup; launch_colsum adds them in a fixed order.
//
// ShortConvolution:  y[t, d] = act(sum_j x[t - W + 1 + j, d] * w[d, j] + b[d]) within each
// sequence (zero left padding).  One thread per (VC adjacent columns, run of tokens):
// consecutive threads read consecutive columns of a token row (coalesced), the thread
// slides a W-tap window along its run (every x element is read once per run) and loads the
// next four tokens ahead of use.  The backward walks its run from the end, recomputing the
// pre-activation, keeping the last W-1 pre-activation gradients in registers, and
// accumulates the weight / bias gradient partials (reduced like the norm's).
// All of these are HBM-bound streams.
#include <math.h>
#include <stdio.h>

#include "stream_ops.h"
#include "tops_common.h"
#include "tops_hip.h"

namespace tops {

template <typename T> __device__ __forceinline__ float ldf(const T* p, long long i) {
  return In<T>::ld(p + i);
}
template <typename T> __device__ __forceinline__ void stf(T* p, long long i, float v) {
  In<T>::st(p + i, v);
}

// ---------------------------------------------------------------- column sums
// grid (column tiles of 16, row blocks of 64): block (cx, ry) sums rows [64 ry, 64 ry + 64)
// of its 16 columns into dst[ry][c] (or the outputs when there is one row block).
__global__ void __launch_bounds__(256) colsum_kernel(const float* __restrict__ part, int np,
                                                     int ncols, int n0, float* __restrict__ out0,
                                                     float* __restrict__ out1,
                                                     float* __restrict__ dst) {
  __shared__ float red[16][17];
  const int cl = threadIdx.x & 15, rg = threadIdx.x >> 4;
  const int c = blockIdx.x * 16 + cl;
  const int rbeg = blockIdx.y * 64, rend = min(rbeg + 64, np);
  float s = 0.f;
  if (c < ncols)
    for (int r = rbeg + rg; r < rend; r += 16) s += part[(long long)r * ncols + c];
  red[rg][cl] = s;
  __syncthreads();
  if (rg == 0 && c < ncols) {
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) t += red[i][cl];
    if (dst) dst[(long long)blockIdx.y * ncols + c] = t;
    else if (c < n0) out0[c] = t;
    else if (out1) out1[c - n0] = t;
  }
}

static int colsum_blocks(int np) { return np <= 64 ? 1 : (np + 63) / 64; }
static int64_t colsum_scratch(int np, int ncols) { return colsum_scratch_floats(np, ncols); }

// Two levels when np > 64: row blocks of 64 into a scratch of ceil(np / 64) rows that
// follows the partials (part[np * ncols] then the scratch), then one more pass.  The
// callers keep np <= 4096, so the second pass sums at most 64 rows.
hipError_t launch_colsum(float* part, int np, int ncols, int n0, float* out0, float* out1,
                         hipStream_t s) {
  const int gx = (ncols + 15) / 16;
  const int ny = colsum_blocks(np);
  if (ny > 64) return hipErrorInvalidValue;
  const float* src = part;
  int n = np;
  if (ny > 1) {
    float* scratch = part + (int64_t)np * ncols;
    colsum_kernel<<<dim3(gx, ny), 256, 0, s>>>(part, np, ncols, n0, out0, out1, scratch);
    src = scratch;
    n = ny;
  }
  colsum_kernel<<<dim3(gx, 1), 256, 0, s>>>(src, n, ncols, n0, out0, out1, nullptr);
  return hipGetLastError();
}

// ---------------------------------------------------------------- RMSNorm (gated), scalar path
__device__ __forceinline__ float wave_sum64(float x) { return group_sum<64>(x); }

template <typename TX, typename TG, int NV>
__global__ void __launch_bounds__(256) rmsnorm_fwd_kernel(const TX* __restrict__ x,
                                                          const TG* __restrict__ g,
                                                          const float* __restrict__ w,
                                                          TX* __restrict__ y, int rows, int D,
                                                          float eps) {
  const int lane = threadIdx.x & 63;
  const int nw = gridDim.x * 4;
  for (int row = blockIdx.x * 4 + threadIdx.x / 64; row < rows; row += nw) {
    const long long base = (long long)row * D;
    float v[NV];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int d = lane + 64 * i;
      v[i] = d < D ? ldf(x, base + d) : 0.f;
      ss += v[i] * v[i];
    }
    const float r = 1.f / sqrtf(wave_sum64(ss) / (float)D + eps);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int d = lane + 64 * i;
      if (d < D) {
        float o = v[i] * r;
        if (w) o *= w[d];
        if (g) {
          const float gv = ldf(g, base + d);
          o *= gv * sigm(gv);
        }
        stf(y, base + d, o);
      }
    }
  }
}

// dx = r (dxh - xh mean(dxh xh)), dxh = dy w s, s = silu(g) (1 without a gate);
// dg = dy xh w silu'(g); dw partial += dy xh s.
template <typename TX, typename TG, int NV>
__global__ void __launch_bounds__(256) rmsnorm_bwd_kernel(
    const TX* __restrict__ x, const TG* __restrict__ g, const float* __restrict__ w,
    const TX* __restrict__ dy, TX* __restrict__ dx, TG* __restrict__ dg,
    float* __restrict__ part, int rows, int D, float eps) {
  __shared__ float red[4][64 * NV];
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x / 64;
  const int nw = gridDim.x * 4;
  float pw[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) pw[i] = 0.f;
  for (int row = blockIdx.x * 4 + wv; row < rows; row += nw) {
    const long long base = (long long)row * D;
    float v[NV], dv[NV], s[NV], sp[NV];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int d = lane + 64 * i;
      const bool in = d < D;
      v[i] = in ? ldf(x, base + d) : 0.f;
      dv[i] = in ? ldf(dy, base + d) : 0.f;
      s[i] = 1.f;
      sp[i] = 0.f;
      if (g && in) {
        const float gv = ldf(g, base + d);
        const float sg = sigm(gv);
        s[i] = gv * sg;                          // silu(g)
        sp[i] = sg * (1.f + gv * (1.f - sg));    // silu'(g)
      }
      ss += v[i] * v[i];
    }
    const float r = 1.f / sqrtf(wave_sum64(ss) / (float)D + eps);
    float dot = 0.f;
    float dxh[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int d = lane + 64 * i;
      const float wd = (w && d < D) ? w[d] : 1.f;
      const float xh = v[i] * r;
      dxh[i] = dv[i] * wd * s[i];
      dot += dxh[i] * xh;
      pw[i] += dv[i] * xh * s[i];
      if (g && d < D) stf(dg, base + d, dv[i] * xh * wd * sp[i]);
    }
    dot = wave_sum64(dot) / (float)D;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int d = lane + 64 * i;
      if (d < D) stf(dx, base + d, r * (dxh[i] - v[i] * r * dot));
    }
  }
  if (!part) return;
#pragma unroll
  for (int i = 0; i < NV; ++i) red[wv][lane + 64 * i] = pw[i];
  __syncthreads();
  for (int d = threadIdx.x; d < D; d += 256)
    part[(long long)blockIdx.x * D + d] = red[0][d] + red[1][d] + red[2][d] + red[3][d];
}

// ---------------------------------------------------------------- RMSNorm, vector path
// Lane (slot, sub) of a wave: row slot = lane / LPR of the current row group, runs
// sub + LPR * j (j < NC) of 8 elements.  Two row groups per iteration (rg and rg + nw).
template <typename TX, typename TG, int LPR, int NC>
__global__ void __launch_bounds__(256) rmsnorm_fwd_v8(const TX* __restrict__ x,
                                                      const TG* __restrict__ g,
                                                      const float* __restrict__ w,
                                                      TX* __restrict__ y, int rows, int D,
                                                      float eps) {
  constexpr int RPW = 64 / LPR;
  const int lane = threadIdx.x & 63, sub = lane % LPR, slot = lane / LPR;
  const int nw = gridDim.x * 4;
  const int nch = D >> 3;
  const float inv_d = 1.f / (float)D;
  for (int rg = blockIdx.x * 4 + (threadIdx.x >> 6); rg * RPW < rows; rg += 2 * nw) {
    float v[2][NC][8], gv[2][NC][8];
    bool ok[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int row = (rg + u * nw) * RPW + slot;
      ok[u] = row < rows;
#pragma unroll
      for (int j = 0; j < NC; ++j) {
        const int c = sub + LPR * j;
        if (ok[u] && c < nch) {
          V8<TX>::ld(x + (long long)row * D + c * 8, v[u][j]);
          if (g) V8<TG>::ld(g + (long long)row * D + c * 8, gv[u][j]);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) v[u][j][e] = gv[u][j][e] = 0.f;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < NC; ++j)
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += v[u][j][e] * v[u][j][e];
      const float r = 1.f / sqrtf(group_sum<LPR>(ss) * inv_d + eps);
      const int row = (rg + u * nw) * RPW + slot;
#pragma unroll
      for (int j = 0; j < NC; ++j) {
        const int c = sub + LPR * j;
        if (!ok[u] || c >= nch) continue;
        float wv[8];
        if (w) V8<float>::ld(w + c * 8, wv);
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          o[e] = v[u][j][e] * r;
          if (w) o[e] *= wv[e];
          if (g) o[e] *= gv[u][j][e] * sigm(gv[u][j][e]);
        }
        V8<TX>::st(y + (long long)row * D + c * 8, o);
      }
    }
  }
}

template <typename TX, typename TG, int LPR, int NC>
__global__ void __launch_bounds__(256) rmsnorm_bwd_v8(
    const TX* __restrict__ x, const TG* __restrict__ g, const float* __restrict__ w,
    const TX* __restrict__ dy, TX* __restrict__ dx, TG* __restrict__ dg,
    float* __restrict__ part, int rows, int D, float eps) {
  constexpr int RPW = 64 / LPR;
  __shared__ float red[4][2048];
  const int lane = threadIdx.x & 63, sub = lane % LPR, slot = lane / LPR;
  const int wv_ = threadIdx.x >> 6;
  const int nw = gridDim.x * 4;
  const int nch = D >> 3;
  const float inv_d = 1.f / (float)D;
  float pw[NC][8];
#pragma unroll
  for (int j = 0; j < NC; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) pw[j][e] = 0.f;
  for (int rg = blockIdx.x * 4 + wv_; rg * RPW < rows; rg += nw) {
    const int row = rg * RPW + slot;
    const bool ok = row < rows;
    const long long base = (long long)row * D;
    float v[NC][8], dv[NC][8], gv[NC][8];
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      const int c = sub + LPR * j;
      if (ok && c < nch) {
        V8<TX>::ld(x + base + c * 8, v[j]);
        V8<TX>::ld(dy + base + c * 8, dv[j]);
        if (g) V8<TG>::ld(g + base + c * 8, gv[j]);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[j][e] = dv[j][e] = gv[j][e] = 0.f;
      }
    }
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NC; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += v[j][e] * v[j][e];
    const float r = 1.f / sqrtf(group_sum<LPR>(ss) * inv_d + eps);
    float dot = 0.f;
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      const int c = sub + LPR * j;
      const bool in = ok && c < nch;
      float wv[8];
      if (w && in) V8<float>::ld(w + c * 8, wv);
      float dgo[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float wd = (w && in) ? wv[e] : 1.f;
        float s = 1.f, sp = 0.f;
        if (g) {
          const float sg = sigm(gv[j][e]);
          s = gv[j][e] * sg;
          sp = sg * (1.f + gv[j][e] * (1.f - sg));
        }
        const float xh = v[j][e] * r;
        const float dxh = dv[j][e] * wd * s;
        dot += dxh * xh;
        pw[j][e] += dv[j][e] * xh * s;
        dgo[e] = dv[j][e] * xh * wd * sp;
        dv[j][e] = dxh;  // reuse: dxh for the dx pass
      }
      if (g && in) V8<TG>::st(dg + base + c * 8, dgo);
    }
    dot = group_sum<LPR>(dot) * inv_d;
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      const int c = sub + LPR * j;
      if (!ok || c >= nch) continue;
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = r * (dv[j][e] - v[j][e] * r * dot);
      V8<TX>::st(dx + base + c * 8, o);
    }
  }
  if (!part) return;
  // add the row slots of the wave, then the 4 waves, in a fixed order
#pragma unroll
  for (int j = 0; j < NC; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
      for (int o = LPR; o < 64; o <<= 1) pw[j][e] += __shfl_xor(pw[j][e], o, 64);
  if (slot == 0) {
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      const int c = sub + LPR * j;
      if (c < nch)
#pragma unroll
        for (int e = 0; e < 8; ++e) red[wv_][c * 8 + e] = pw[j][e];
    }
  }
  __syncthreads();
  for (int d = threadIdx.x; d < D; d += 256)
    part[(long long)blockIdx.x * D + d] = (red[0][d] + red[1][d]) + (red[2][d] + red[3][d]);
}

// ---------------------------------------------------------------- ShortConvolution
struct SeqCursor {
  const int32_t* cu;  // [N+1] or null (fixed length T)
  int N, T;
  int n, bos, eos;
  __device__ void find(int t) {
    if (cu) {
      int lo = 0, hi = N;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (cu[mid] <= t) lo = mid; else hi = mid - 1;
      }
      n = lo;
      bos = cu[n];
      eos = cu[n + 1];
    } else {
      n = t / T;
      bos = n * T;
      eos = bos + T;
    }
  }
};

template <typename T, int VC> struct VecC;
template <typename T> struct VecC<T, 1> {
  __device__ __forceinline__ static void ld(const T* p, float* v) { v[0] = In<T>::ld(p); }
  __device__ __forceinline__ static void st(T* p, const float* v) { In<T>::st(p, v[0]); }
};
template <> struct VecC<uint16_t, 2> {
  __device__ __forceinline__ static void ld(const uint16_t* p, float* v) { In<uint16_t>::ld2(p, v[0], v[1]); }
  __device__ __forceinline__ static void st(uint16_t* p, const float* v) {
    *(uint32_t*)p = pack_bf16x2(v[0], v[1]);
  }
};
template <> struct VecC<float, 2> {
  __device__ __forceinline__ static void ld(const float* p, float* v) { In<float>::ld2(p, v[0], v[1]); }
  __device__ __forceinline__ static void st(float* p, const float* v) { *(float2*)p = make_float2(v[0], v[1]); }
};
template <typename T> struct VecC<T, 4> {
  __device__ __forceinline__ static void ld(const T* p, float* v) { V4<T>::ld(p, v); }
  __device__ __forceinline__ static void st(T* p, const float* v) { V4<T>::st(p, v); }
};

// taps right-aligned in MAXW registers: wt[c][MAXW - W + j] = w[d + c, j]; wt[c][MAXW-1]
// multiplies x[t]
template <int MAXW, int VC>
__device__ __forceinline__ void load_taps(const float* w, int d0, int W, float (&wt)[VC][MAXW]) {
#pragma unroll
  for (int c = 0; c < VC; ++c)
#pragma unroll
    for (int j = 0; j < MAXW; ++j)
      wt[c][j] = j >= MAXW - W ? w[(long long)(d0 + c) * W + j - (MAXW - W)] : 0.f;
}

// y = act(conv(x) + b)
template <typename TX, typename TY, int MAXW, int VC>
__global__ void __launch_bounds__(256) short_conv_fwd_kernel(
    const TX* __restrict__ x, const float* __restrict__ w, const float* __restrict__ b,
    TY* __restrict__ y, const int32_t* __restrict__ cu, int N, int T, int total, int D, int W,
    int per, int act) {
  const int d0 = (blockIdx.x * 256 + threadIdx.x) * VC;
  if (d0 >= D) return;
  const int r0 = blockIdx.y * per;
  const int r1 = min(r0 + per, total);
  if (r0 >= r1) return;
  float wt[VC][MAXW];
  load_taps<MAXW, VC>(w, d0, W, wt);
  float bias[VC];
#pragma unroll
  for (int c = 0; c < VC; ++c) bias[c] = b ? b[d0 + c] : 0.f;
  SeqCursor sc{cu, N, T, 0, 0, 0};
  sc.find(r0);
  float win[VC][MAXW];  // win[c][j] = x[t - MAXW + 1 + j, d0 + c]
#pragma unroll
  for (int j = 0; j < MAXW - 1; ++j) {
    const int p = r0 - MAXW + 1 + j;
    float v[VC];
    if (p >= sc.bos) VecC<TX, VC>::ld(x + (long long)p * D + d0, v);
    else
#pragma unroll
      for (int c = 0; c < VC; ++c) v[c] = 0.f;
#pragma unroll
    for (int c = 0; c < VC; ++c) win[c][j + 1] = v[c];
  }
#pragma unroll
  for (int c = 0; c < VC; ++c) win[c][0] = 0.f;
  // the next four tokens are loaded while the current four are processed
  float xin[4][VC];
#pragma unroll
  for (int u = 0; u < 4; ++u)
    if (r0 + u < r1) VecC<TX, VC>::ld(x + (long long)(r0 + u) * D + d0, xin[u]);
  for (int t = r0; t < r1; t += 4) {
    float xnx[4][VC];
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (t + 4 + u < r1) VecC<TX, VC>::ld(x + (long long)(t + 4 + u) * D + d0, xnx[u]);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int p = t + u;
      if (p >= r1) break;
      if (p >= sc.eos) {
        sc.find(p);
#pragma unroll
        for (int c = 0; c < VC; ++c)
#pragma unroll
          for (int j = 1; j < MAXW; ++j) win[c][j] = 0.f;
      }
      float o[VC];
#pragma unroll
      for (int c = 0; c < VC; ++c) {
#pragma unroll
        for (int j = 0; j < MAXW - 1; ++j) win[c][j] = win[c][j + 1];
        win[c][MAXW - 1] = xin[u][c];
        float pre = bias[c];
#pragma unroll
        for (int j = 0; j < MAXW; ++j) pre += win[c][j] * wt[c][j];
        o[c] = act ? pre * sigm(pre) : pre;
      }
      VecC<TY, VC>::st(y + (long long)p * D + d0, o);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int c = 0; c < VC; ++c) xin[u][c] = xnx[u][c];
  }
}

// final state [N, D, W] (x's dtype): the last W inputs of each sequence, zero left-padded
template <typename TX>
__global__ void __launch_bounds__(256) short_conv_state_kernel(const TX* __restrict__ x,
                                                               TX* __restrict__ st,
                                                               const int32_t* __restrict__ cu,
                                                               int N, int T, int D, int W) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long long)N * D * W) return;
  const int j = (int)(i % W);
  const int d = (int)((i / W) % D);
  const int n = (int)(i / ((long long)W * D));
  const int bos = cu ? cu[n] : n * T;
  const int eos = cu ? cu[n + 1] : bos + T;
  const int p = eos - W + j;
  st[i] = p >= bos ? x[(long long)p * D + d] : (TX)0;
}

// backward, walking the run from its end.  xw[c][j] = x[t - MAXW + 1 + j] (zero before bos),
// dp[c][i] = dpre[t + 1 + i] (zero at or after eos), i < MAXW - 1.  Partials: [nrb][W*D + D]
// with the weight gradient at d * W + j and the bias gradient at W * D + d.
template <typename TX, typename TY, int MAXW, int VC, bool ACT>
__global__ void __launch_bounds__(256) short_conv_bwd_kernel(
    const TX* __restrict__ x, const float* __restrict__ w, const float* __restrict__ b,
    const TY* __restrict__ dy, TX* __restrict__ dx, float* __restrict__ part,
    const int32_t* __restrict__ cu, int N, int T, int total, int D, int W, int per) {
  // the 4 waves of a workgroup share 64 * VC columns and take 4 consecutive runs; their
  // weight / bias partials are added in LDS, one partial row per workgroup
  __shared__ float red[4][(MAXW + 1) * 64 * VC];
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int d0 = (blockIdx.x * 64 + lane) * VC;
  const bool col_ok = d0 < D;
  const int da = col_ok ? d0 : 0;
  const int rb = blockIdx.y * 4 + wv;
  const int r0 = rb * per;
  const int r1 = min(r0 + per, total);
  float wt[VC][MAXW];
  load_taps<MAXW, VC>(w, col_ok ? d0 : 0, W, wt);
  float bias[VC];
#pragma unroll
  for (int c = 0; c < VC; ++c) bias[c] = (b && col_ok) ? b[d0 + c] : 0.f;
  float pw[VC][MAXW], pb[VC];
#pragma unroll
  for (int c = 0; c < VC; ++c) {
    pb[c] = 0.f;
#pragma unroll
    for (int j = 0; j < MAXW; ++j) pw[c][j] = 0.f;
  }
  auto dpre_of = [&](float pre, float g) -> float {
    // a compile-time switch: a run-time flag here splits every token of the walk into
    // separate blocks
    if constexpr (!ACT) return g;
    const float s = sigm(pre);
    return g * (s * (1.f + pre * (1.f - s)));
  };
  auto ldx = [&](int p, float* v) {
    VecC<TX, VC>::ld(x + (long long)p * D + da, v);
  };

  if (r0 < r1) {
    SeqCursor sc{cu, N, T, 0, 0, 0};
    int t = r1 - 1;
    sc.find(t);
    float xw[VC][MAXW], dp[VC][MAXW];
    {
      // warm-up: x[t - MAXW + 1 .. t + MAXW - 1] and dpre[t + 1 .. t + MAXW - 1]
      float xa[2 * MAXW - 1][VC];
#pragma unroll
      for (int j = 0; j < 2 * MAXW - 1; ++j) {
        const int p = t - MAXW + 1 + j;
        if (p >= sc.bos && p < sc.eos) ldx(p, xa[j]);
        else
#pragma unroll
          for (int c = 0; c < VC; ++c) xa[j][c] = 0.f;
      }
#pragma unroll
      for (int c = 0; c < VC; ++c) {
#pragma unroll
        for (int j = 0; j < MAXW; ++j) xw[c][j] = xa[j][c];
        dp[c][MAXW - 1] = 0.f;
      }
#pragma unroll
      for (int i = 0; i < MAXW - 1; ++i) {
        const int p = t + 1 + i;
        float gy[VC];
        const bool in = p < sc.eos;
        if (in) VecC<TY, VC>::ld(dy + (long long)p * D + da, gy);
#pragma unroll
        for (int c = 0; c < VC; ++c) {
          float v = 0.f;
          if (in) {
            float pre = bias[c];
#pragma unroll
            for (int j = 0; j < MAXW; ++j) pre += xa[i + 1 + j][c] * wt[c][j];
            v = dpre_of(pre, gy[c]);
          }
          dp[c][i] = v;
        }
      }
    }
    // dy for steps t0 .. t0-3 and the x entering the window after each
    auto load_group = [&](int t0, float (&gyv)[4][VC], float (&xn)[4][VC]) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int cur = t0 - s;
        if (cur >= r0) {
          VecC<TY, VC>::ld(dy + (long long)cur * D + da, gyv[s]);
          const int p = cur - MAXW;
          if (p >= 0) ldx(p, xn[s]);
          else
#pragma unroll
            for (int c = 0; c < VC; ++c) xn[s][c] = 0.f;
        }
      }
    };
    float gyv[4][VC], xn[4][VC];
    load_group(t, gyv, xn);
    bool done = false;
    while (!done) {
      // the next group's loads are issued before this group is processed
      float gy2[4][VC], xn2[4][VC];
      load_group(t - 4, gy2, xn2);
      // one token of the walk: dx at cur from the pre-activation gradients in the window,
      // the weight / bias partials, then both windows shift one token toward the past
      auto step = [&](const float (&gy)[VC], float (&g)[VC]) {
#pragma unroll
        for (int c = 0; c < VC; ++c) {
          float pre = bias[c];
#pragma unroll
          for (int j = 0; j < MAXW; ++j) pre += xw[c][j] * wt[c][j];
          const float dpt = dpre_of(pre, gy[c]);
          // dx[cur] = sum_i dpre[cur + i] w[W - 1 - i]
          float a = dpt * wt[c][MAXW - 1];
#pragma unroll
          for (int i = 0; i < MAXW - 1; ++i) a += dp[c][i] * wt[c][MAXW - 2 - i];
          g[c] = a;
#pragma unroll
          for (int j = 0; j < MAXW; ++j) pw[c][j] += xw[c][j] * dpt;
          pb[c] += dpt;
#pragma unroll
          for (int i = MAXW - 2; i > 0; --i) dp[c][i] = dp[c][i - 1];
          dp[c][0] = dpt;
#pragma unroll
          for (int j = MAXW - 1; j > 0; --j) xw[c][j] = xw[c][j - 1];
        }
      };
      if (t - 4 >= r0 && t - 3 - MAXW >= sc.bos) {
        // the whole group and the next token lie inside the run and inside one sequence with
        // full windows: no branch, so the window shifts compile to register renaming
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          float g[VC];
          step(gyv[s], g);
          if (col_ok) VecC<TX, VC>::st(dx + (long long)(t - s) * D + da, g);
#pragma unroll
          for (int c = 0; c < VC; ++c) xw[c][0] = xn[s][c];
        }
      } else {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int cur = t - s;
        float g[VC];
        step(gyv[s], g);
        if (col_ok) VecC<TX, VC>::st(dx + (long long)cur * D + da, g);
        const int nxt = cur - 1;
        if (nxt < r0) {
          done = true;
          break;
        }
        if (nxt < sc.bos) {
          // entering the previous sequence: no later gradient, reload the window
          sc.find(nxt);
#pragma unroll
          for (int j = 0; j < MAXW; ++j) {
            const int p = nxt - MAXW + 1 + j;
            float v[VC];
            if (p >= sc.bos) ldx(p, v);
            else
#pragma unroll
              for (int c = 0; c < VC; ++c) v[c] = 0.f;
#pragma unroll
            for (int c = 0; c < VC; ++c) xw[c][j] = v[c];
          }
#pragma unroll
          for (int c = 0; c < VC; ++c)
#pragma unroll
            for (int i = 0; i < MAXW; ++i) dp[c][i] = 0.f;
        } else {
          const bool in = nxt - MAXW + 1 >= sc.bos;
#pragma unroll
          for (int c = 0; c < VC; ++c) xw[c][0] = in ? xn[s][c] : 0.f;
        }
      }
      }
      t -= 4;
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int c = 0; c < VC; ++c) {
          gyv[s][c] = gy2[s][c];
          xn[s][c] = xn2[s][c];
        }
    }
  }
  // LDS slot of (local column lc, tap j): j * 64 * VC + lc; the bias after the MAXW taps
#pragma unroll
  for (int c = 0; c < VC; ++c) {
#pragma unroll
    for (int j = 0; j < MAXW; ++j) red[wv][j * 64 * VC + lane * VC + c] = pw[c][j];
    red[wv][MAXW * 64 * VC + lane * VC + c] = pb[c];
  }
  __syncthreads();
  float* pp = part + (long long)blockIdx.y * (W + 1) * D;
  const int dbase = blockIdx.x * 64 * VC;
  for (int i = threadIdx.x; i < (W + 1) * 64 * VC; i += 256) {
    const int j = i / (64 * VC), lc = i - j * 64 * VC;   // j == W: the bias
    const int d = dbase + lc;
    if (d >= D) continue;
    const int slot = (j < W ? j + MAXW - W : MAXW) * 64 * VC + lc;
    const float v = (red[0][slot] + red[1][slot]) + (red[2][slot] + red[3][slot]);
    if (j < W) pp[(long long)d * W + j] = v;
    else pp[(long long)W * D + d] = v;
  }
}

// decode step: cache [N, D, W] rolled by one with x appended, y = act(sum cache * w + b)
template <typename TX, typename TY>
__global__ void __launch_bounds__(256) short_conv_step_kernel(
    const TX* __restrict__ x, const float* __restrict__ cin, float* __restrict__ cout,
    const float* __restrict__ w, const float* __restrict__ b, TY* __restrict__ y, int N, int D,
    int W, int act) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;  // over N * D
  if (i >= (long long)N * D) return;
  const int d = (int)(i % D);
  const float xv = ldf(x, i);
  float pre = b ? b[d] : 0.f;
  if (cin) {
    // ascending j reads c[j + 1] before c[j + 1] is overwritten, so cout may alias cin
    const float* c = cin + i * W;
    float* co = cout + i * W;
    for (int j = 0; j < W - 1; ++j) {
      const float cj = c[j + 1];
      co[j] = cj;
      pre += cj * w[(long long)d * W + j];
    }
    co[W - 1] = xv;
    pre += xv * w[(long long)d * W + W - 1];
  } else {
    pre += xv * w[(long long)d * W + W - 1];
  }
  stf(y, i, act ? pre * sigm(pre) : pre);
}

}  // namespace tops

using namespace tops;

static int dt_ok(int dt) { return dt == TOPS_F32 || dt == TOPS_BF16; }

// ---------------------------------------------------------------- RMSNorm entry points
// vector path layout for D: lanes per row and runs per lane; false when D does not fit
static bool rms_v8_shape(int D, int& lpr, int& nc) {
  if (D % 8 || D < 64 || D > 2048) return false;
  const int nch = D / 8;
  lpr = 8;
  while (lpr < 64 && lpr < nch) lpr <<= 1;
  nc = (nch + lpr - 1) / lpr;
  return nc == 1 || nc == 2 || nc == 4;
}

template <typename TX, typename TG>
static hipError_t rms_fwd_t(const void* x, const void* g, const float* w, void* y, int rows,
                            int D, float eps, hipStream_t s) {
  int lpr, nc;
  if (rms_v8_shape(D, lpr, nc)) {
    const int rpw = 64 / lpr;
    long long groups = ((long long)rows + rpw - 1) / rpw;
    int grid = (int)((groups + 7) / 8);  // 4 waves x 2 row groups per block
    if (grid > 16384) grid = 16384;
    if (grid < 1) grid = 1;
#define TOPS_RMS_V(L, C)                                                              \
  rmsnorm_fwd_v8<TX, TG, L, C><<<grid, 256, 0, s>>>((const TX*)x, (const TG*)g, w,  \
                                                    (TX*)y, rows, D, eps)
    if (lpr == 8) TOPS_RMS_V(8, 1);
    else if (lpr == 16) TOPS_RMS_V(16, 1);
    else if (lpr == 32) TOPS_RMS_V(32, 1);
    else if (nc == 1) TOPS_RMS_V(64, 1);
    else if (nc == 2) TOPS_RMS_V(64, 2);
    else TOPS_RMS_V(64, 4);
#undef TOPS_RMS_V
    return hipGetLastError();
  }
  int grid = (rows + 3) / 4;
  if (grid > 4096) grid = 4096;
  if (grid < 1) grid = 1;
#define TOPS_RMS_F(NV)                                                                     \
  rmsnorm_fwd_kernel<TX, TG, NV><<<grid, 256, 0, s>>>((const TX*)x, (const TG*)g, w, (TX*)y, \
                                                      rows, D, eps)
  if (D <= 64) TOPS_RMS_F(1);
  else if (D <= 128) TOPS_RMS_F(2);
  else if (D <= 256) TOPS_RMS_F(4);
  else if (D <= 512) TOPS_RMS_F(8);
  else if (D <= 1024) TOPS_RMS_F(16);
  else TOPS_RMS_F(32);
#undef TOPS_RMS_F
  return hipGetLastError();
}

// workgroups of the backward (each writes one weight-gradient partial row)
static int rms_blocks(int rows, int D) {
  int lpr, nc;
  long long waves_needed;
  if (rms_v8_shape(D, lpr, nc)) waves_needed = ((long long)rows + 64 / lpr - 1) / (64 / lpr);
  else waves_needed = rows;
  long long grid = (waves_needed + 3) / 4;
  if (grid > 1024) grid = 1024;
  return grid < 1 ? 1 : (int)grid;
}

template <typename TX, typename TG>
static hipError_t rms_bwd_t(const void* x, const void* g, const float* w, const void* dy,
                            void* dx, void* dg, float* part, int rows, int D, float eps,
                            hipStream_t s) {
  const int grid = rms_blocks(rows, D);
  int lpr, nc;
  if (rms_v8_shape(D, lpr, nc)) {
#define TOPS_RMS_BV(L, C)                                                                   \
  rmsnorm_bwd_v8<TX, TG, L, C><<<grid, 256, 0, s>>>((const TX*)x, (const TG*)g, w,         \
                                                    (const TX*)dy, (TX*)dx, (TG*)dg, part, \
                                                    rows, D, eps)
    if (lpr == 8) TOPS_RMS_BV(8, 1);
    else if (lpr == 16) TOPS_RMS_BV(16, 1);
    else if (lpr == 32) TOPS_RMS_BV(32, 1);
    else if (nc == 1) TOPS_RMS_BV(64, 1);
    else if (nc == 2) TOPS_RMS_BV(64, 2);
    else TOPS_RMS_BV(64, 4);
#undef TOPS_RMS_BV
    return hipGetLastError();
  }
#define TOPS_RMS_B(NV)                                                                         \
  rmsnorm_bwd_kernel<TX, TG, NV><<<grid, 256, 0, s>>>((const TX*)x, (const TG*)g, w,           \
                                                      (const TX*)dy, (TX*)dx, (TG*)dg, part, \
                                                      rows, D, eps)
  if (D <= 64) TOPS_RMS_B(1);
  else if (D <= 128) TOPS_RMS_B(2);
  else if (D <= 256) TOPS_RMS_B(4);
  else if (D <= 512) TOPS_RMS_B(8);
  else if (D <= 1024) TOPS_RMS_B(16);
  else TOPS_RMS_B(32);
#undef TOPS_RMS_B
  return hipGetLastError();
}

static int rms_check(const char* who, int x_dtype, const void* g, int g_dtype, int rows, int D) {
  char msg[160];
  if (!dt_ok(x_dtype) || (g && !dt_ok(g_dtype))) {
    snprintf(msg, sizeof(msg), "%s: dtypes must be TOPS_F32 or TOPS_BF16", who);
    return tops_set_error(TOPS_ERR_DTYPE, msg);
  }
  if (rows < 0 || D <= 0 || D > 2048) {
    snprintf(msg, sizeof(msg), "%s: need rows >= 0 and 0 < D <= 2048", who);
    return tops_set_error(TOPS_ERR_SHAPE, msg);
  }
  return TOPS_OK;
}

extern "C" int tops_rmsnorm_gated_fwd(const void* x, int x_dtype, const void* g, int g_dtype,
                                      const float* weight, void* y, int rows, int D, float eps,
                                      void* stream) {
  if (!x || !y) return tops_set_error(TOPS_ERR_NULL, "rmsnorm_gated_fwd: null tensor");
  int rc = rms_check("rmsnorm_gated_fwd", x_dtype, g, g_dtype, rows, D);
  if (rc != TOPS_OK) return rc;
  if (rows == 0) return TOPS_OK;
  hipStream_t s = (hipStream_t)stream;
  const bool xb = x_dtype == TOPS_BF16, gb = g && g_dtype == TOPS_BF16;
  hipError_t e = xb ? (gb ? rms_fwd_t<uint16_t, uint16_t>(x, g, weight, y, rows, D, eps, s)
                          : rms_fwd_t<uint16_t, float>(x, g, weight, y, rows, D, eps, s))
                    : (gb ? rms_fwd_t<float, uint16_t>(x, g, weight, y, rows, D, eps, s)
                          : rms_fwd_t<float, float>(x, g, weight, y, rows, D, eps, s));
  return e == hipSuccess ? TOPS_OK : tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
}

extern "C" int64_t tops_rmsnorm_gated_bwd_workspace(int rows, int D) {
  if (rows < 0 || D <= 0) return TOPS_ERR_SHAPE;
  const int nb = rms_blocks(rows, D);
  return (int64_t)nb * D + colsum_scratch(nb, D);
}

extern "C" int tops_rmsnorm_gated_bwd(const void* x, int x_dtype, const void* g, int g_dtype,
                                      const float* weight, const void* dy, void* dx, void* dg,
                                      float* dweight, float* workspace, int64_t workspace_floats,
                                      int rows, int D, float eps, void* stream) {
  if (!x || !dy || !dx || (g && !dg) || (weight && (!dweight || !workspace)))
    return tops_set_error(TOPS_ERR_NULL, "rmsnorm_gated_bwd: null tensor");
  int rc = rms_check("rmsnorm_gated_bwd", x_dtype, g, g_dtype, rows, D);
  if (rc != TOPS_OK) return rc;
  const int nb = rms_blocks(rows, D);
  if (weight && workspace_floats < (int64_t)nb * D + colsum_scratch(nb, D))
    return tops_set_error(TOPS_ERR_SHAPE, "rmsnorm_gated_bwd: workspace smaller than tops_rmsnorm_gated_bwd_workspace()");
  hipStream_t s = (hipStream_t)stream;
  float* part = weight ? workspace : nullptr;
  hipError_t e = hipSuccess;
  if (rows > 0) {
    const bool xb = x_dtype == TOPS_BF16, gb = g && g_dtype == TOPS_BF16;
    e = xb ? (gb ? rms_bwd_t<uint16_t, uint16_t>(x, g, weight, dy, dx, dg, part, rows, D, eps, s)
                 : rms_bwd_t<uint16_t, float>(x, g, weight, dy, dx, dg, part, rows, D, eps, s))
           : (gb ? rms_bwd_t<float, uint16_t>(x, g, weight, dy, dx, dg, part, rows, D, eps, s)
                 : rms_bwd_t<float, float>(x, g, weight, dy, dx, dg, part, rows, D, eps, s));
    if (e != hipSuccess) return tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
  }
  if (weight) e = launch_colsum(part, rows > 0 ? nb : 0, D, D, dweight, nullptr, s);
  return e == hipSuccess ? TOPS_OK : tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
}

// ---------------------------------------------------------------- ShortConvolution entry points
static int conv_check(const char* who, int x_dtype, int y_dtype, const int32_t* cu, int B, int T,
                      int D, int W, int N) {
  char msg[160];
  if (!dt_ok(x_dtype) || !dt_ok(y_dtype)) {
    snprintf(msg, sizeof(msg), "%s: dtypes must be TOPS_F32 or TOPS_BF16", who);
    return tops_set_error(TOPS_ERR_DTYPE, msg);
  }
  if (B <= 0 || T < 0 || D <= 0 || W < 1 || W > 8 || N <= 0) {
    snprintf(msg, sizeof(msg), "%s: need B, D, N > 0, T >= 0 and 1 <= W <= 8", who);
    return tops_set_error(TOPS_ERR_SHAPE, msg);
  }
  if (cu && B != 1) {
    snprintf(msg, sizeof(msg), "%s: cu_seqlens requires B == 1", who);
    return tops_set_error(TOPS_ERR_SHAPE, msg);
  }
  if (!cu && N != B) {
    snprintf(msg, sizeof(msg), "%s: N must equal B", who);
    return tops_set_error(TOPS_ERR_SHAPE, msg);
  }
  if ((long long)B * T >= (1LL << 31) || (long long)(W + 1) * D >= (1LL << 31)) {
    snprintf(msg, sizeof(msg), "%s: too large", who);
    return tops_set_error(TOPS_ERR_SHAPE, msg);
  }
  return TOPS_OK;
}

static int conv_vc(int D) { return D % 4 == 0 ? 4 : 1; }

// Workgroups of a kernel instance that are resident on the whole device at once (CUs x
// workgroups per CU at the instance's register and LDS use).  The walks below are all of one
// length, so a grid of exactly one such round finishes together; a round and a fraction
// leaves most of the device idle during the fraction (short_conv_bwd at [8, 4096, 2048]:
// 0.19 ms with one round of 128-token runs, 0.24 ms with one and a half rounds, 0.21 ms with
// two rounds of 64-token runs).
template <typename Kern>
static int resident_wgs(Kern kernel) {
  int dev = 0, cus = 0, per_cu = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, 256, 0) != hipSuccess) {
    (void)hipGetLastError();
    return 2048;
  }
  return cus * per_cu > 0 ? cus * per_cu : 2048;
}

// row blocks: `target` workgroups over (column tiles x row blocks), runs of >= 16 tokens,
// at most 4096 blocks
static void conv_split(int total, int D, int target, int& nrb, int& per) {
  const int tiles = (D / conv_vc(D) + 255) / 256;
  nrb = (target + tiles - 1) / tiles;
  int maxb = (total + 15) / 16;
  if (nrb > maxb) nrb = maxb;
  if (nrb > 4096) nrb = 4096;
  if (nrb < 1) nrb = 1;
  per = (total + nrb - 1) / nrb;
  if (per < 1) per = 1;
  nrb = (total + per - 1) / per;
  if (nrb < 1) nrb = 1;
}

// backward: runs of tokens per column group (one wave each, `waves` of them, at most 8192),
// 4 runs per workgroup, one weight-gradient partial row per workgroup.  The workspace is
// sized for 8192 waves, which bounds the partial rows of every smaller target.
static int conv_bwd_vc(int D) { return D % 2 == 0 ? 2 : 1; }
static void conv_bwd_split(int total, int D, int waves, int& nrb4, int& per) {
  const int tiles = (D / conv_bwd_vc(D) + 63) / 64;
  if (waves > 8192 || waves < 1) waves = 8192;
  int runs = (waves + tiles - 1) / tiles;
  const int maxr = (total + 15) / 16;
  if (runs > maxr) runs = maxr;
  if (runs > 4 * 4096) runs = 4 * 4096;
  if (runs < 1) runs = 1;
  per = (total + runs - 1) / runs;
  if (per < 1) per = 1;
  runs = (total + per - 1) / per;
  if (runs < 1) runs = 1;
  nrb4 = (runs + 3) / 4;
}

template <typename TX, typename TY>
static hipError_t conv_fwd_t(const void* x, const float* w, const float* b, void* y,
                             const int32_t* cu, int N, int T, int total, int D, int W, int act,
                             hipStream_t s) {
  const int vc = conv_vc(D);
#define TOPS_CONV_F(MW, VC)                                                                   \
  do {                                                                                        \
    static const int target = resident_wgs(short_conv_fwd_kernel<TX, TY, MW, VC>);           \
    int nrb, per;                                                                             \
    conv_split(total, D, target, nrb, per);                                                   \
    dim3 grid((D / vc + 255) / 256, nrb);                                                     \
    short_conv_fwd_kernel<TX, TY, MW, VC><<<grid, 256, 0, s>>>((const TX*)x, w, b, (TY*)y,   \
                                                               cu, N, T, total, D, W, per, act); \
  } while (0)
  if (vc == 4) {
    if (W <= 4) TOPS_CONV_F(4, 4); else TOPS_CONV_F(8, 4);
  } else {
    if (W <= 4) TOPS_CONV_F(4, 1); else TOPS_CONV_F(8, 1);
  }
#undef TOPS_CONV_F
  return hipGetLastError();
}

extern "C" int tops_short_conv_fwd(const void* x, int x_dtype, const float* weight,
                                   const float* bias, void* y, int y_dtype, void* final_state,
                                   const int32_t* cu_seqlens, int B, int T, int D, int W, int N,
                                   int activation, void* stream) {
  if (!x || !weight || !y) return tops_set_error(TOPS_ERR_NULL, "short_conv_fwd: null tensor");
  int rc = conv_check("short_conv_fwd", x_dtype, y_dtype, cu_seqlens, B, T, D, W, N);
  if (rc != TOPS_OK) return rc;
  hipStream_t s = (hipStream_t)stream;
  const int total = B * T;
  const int act = activation ? 1 : 0;
  hipError_t e = hipSuccess;
  if (total > 0) {
    const bool xb = x_dtype == TOPS_BF16, yb = y_dtype == TOPS_BF16;
    e = xb ? (yb ? conv_fwd_t<uint16_t, uint16_t>(x, weight, bias, y, cu_seqlens, N, T, total, D, W, act, s)
                 : conv_fwd_t<uint16_t, float>(x, weight, bias, y, cu_seqlens, N, T, total, D, W, act, s))
           : (yb ? conv_fwd_t<float, uint16_t>(x, weight, bias, y, cu_seqlens, N, T, total, D, W, act, s)
                 : conv_fwd_t<float, float>(x, weight, bias, y, cu_seqlens, N, T, total, D, W, act, s));
    if (e != hipSuccess) return tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
  }
  if (final_state) {
    const long long n = (long long)N * D * W;
    const int grid = (int)((n + 255) / 256);
    if (x_dtype == TOPS_BF16)
      short_conv_state_kernel<uint16_t><<<grid, 256, 0, s>>>((const uint16_t*)x,
                                                             (uint16_t*)final_state, cu_seqlens,
                                                             N, T, D, W);
    else
      short_conv_state_kernel<float><<<grid, 256, 0, s>>>((const float*)x, (float*)final_state,
                                                          cu_seqlens, N, T, D, W);
    e = hipGetLastError();
  }
  return e == hipSuccess ? TOPS_OK : tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
}

extern "C" int64_t tops_short_conv_bwd_workspace(int B, int T, int D, int W) {
  if (B <= 0 || T < 0 || D <= 0 || W < 1) return TOPS_ERR_SHAPE;
  int nrb, per;
  conv_bwd_split(B * T, D, 8192, nrb, per);
  const int ncols = (W + 1) * D;
  return (int64_t)nrb * ncols + colsum_scratch(nrb, ncols);
}

template <typename TX, typename TY>
static hipError_t conv_bwd_t(const void* x, const float* w, const float* b, const void* dy,
                             void* dx, float* part, const int32_t* cu, int N, int T, int total,
                             int D, int W, int act, hipStream_t s, int& nrb) {
  const int vc = conv_bwd_vc(D);
#define TOPS_CONV_B(MW, VC)                                                                  \
  do {                                                                                       \
    static const int waves = 4 * resident_wgs(short_conv_bwd_kernel<TX, TY, MW, VC, true>);  \
    int per;                                                                                 \
    conv_bwd_split(total, D, waves, nrb, per);                                               \
    dim3 grid((D / vc + 63) / 64, nrb);                                                      \
    if (act)                                                                                 \
      short_conv_bwd_kernel<TX, TY, MW, VC, true><<<grid, 256, 0, s>>>(                      \
          (const TX*)x, w, b, (const TY*)dy, (TX*)dx, part, cu, N, T, total, D, W, per);     \
    else                                                                                     \
      short_conv_bwd_kernel<TX, TY, MW, VC, false><<<grid, 256, 0, s>>>(                     \
          (const TX*)x, w, b, (const TY*)dy, (TX*)dx, part, cu, N, T, total, D, W, per);     \
  } while (0)
  if (vc == 2) {
    if (W <= 4) TOPS_CONV_B(4, 2); else TOPS_CONV_B(8, 2);
  } else {
    if (W <= 4) TOPS_CONV_B(4, 1); else TOPS_CONV_B(8, 1);
  }
#undef TOPS_CONV_B
  return hipGetLastError();
}

extern "C" int tops_short_conv_bwd(const void* x, int x_dtype, const float* weight,
                                   const float* bias, const void* dy, int dy_dtype, void* dx,
                                   float* dweight, float* dbias, float* workspace,
                                   int64_t workspace_floats, const int32_t* cu_seqlens, int B,
                                   int T, int D, int W, int N, int activation, void* stream) {
  if (!x || !weight || !dy || !dx || !dweight || !workspace)
    return tops_set_error(TOPS_ERR_NULL, "short_conv_bwd: null tensor");
  int rc = conv_check("short_conv_bwd", x_dtype, dy_dtype, cu_seqlens, B, T, D, W, N);
  if (rc != TOPS_OK) return rc;
  const int total = B * T;
  int nrb, per;
  conv_bwd_split(total, D, 8192, nrb, per);   // the bound the workspace is sized for
  const int ncols = (W + 1) * D;
  if (workspace_floats < (int64_t)nrb * ncols + colsum_scratch(nrb, ncols))
    return tops_set_error(TOPS_ERR_SHAPE, "short_conv_bwd: workspace smaller than tops_short_conv_bwd_workspace()");
  hipStream_t s = (hipStream_t)stream;
  const int act = activation ? 1 : 0;
  hipError_t e = hipSuccess;
  if (total > 0) {
    const bool xb = x_dtype == TOPS_BF16, yb = dy_dtype == TOPS_BF16;
    e = xb ? (yb ? conv_bwd_t<uint16_t, uint16_t>(x, weight, bias, dy, dx, workspace, cu_seqlens, N, T, total, D, W, act, s, nrb)
                 : conv_bwd_t<uint16_t, float>(x, weight, bias, dy, dx, workspace, cu_seqlens, N, T, total, D, W, act, s, nrb))
           : (yb ? conv_bwd_t<float, uint16_t>(x, weight, bias, dy, dx, workspace, cu_seqlens, N, T, total, D, W, act, s, nrb)
                 : conv_bwd_t<float, float>(x, weight, bias, dy, dx, workspace, cu_seqlens, N, T, total, D, W, act, s, nrb));
    if (e != hipSuccess) return tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
  }
  e = launch_colsum(workspace, total > 0 ? nrb : 0, ncols, W * D, dweight, dbias, s);
  return e == hipSuccess ? TOPS_OK : tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
}

extern "C" int tops_short_conv_step(const void* x, int x_dtype, const float* cache_in,
                                    float* cache_out, const float* weight, const float* bias,
                                    void* y, int y_dtype, int N, int D, int W, int activation,
                                    void* stream) {
  if (!x || !weight || !y || (cache_in && !cache_out))
    return tops_set_error(TOPS_ERR_NULL, "short_conv_step: null tensor");
  if (!dt_ok(x_dtype) || !dt_ok(y_dtype))
    return tops_set_error(TOPS_ERR_DTYPE, "short_conv_step: dtypes must be TOPS_F32 or TOPS_BF16");
  if (N < 0 || D <= 0 || W < 1 || W > 8)
    return tops_set_error(TOPS_ERR_SHAPE, "short_conv_step: need N >= 0, D > 0 and 1 <= W <= 8");
  if (N == 0) return TOPS_OK;
  hipStream_t s = (hipStream_t)stream;
  const long long n = (long long)N * D;
  const int grid = (int)((n + 255) / 256);
  const int act = activation ? 1 : 0;
  const bool xb = x_dtype == TOPS_BF16, yb = y_dtype == TOPS_BF16;
  if (xb && yb)
    short_conv_step_kernel<uint16_t, uint16_t><<<grid, 256, 0, s>>>((const uint16_t*)x, cache_in, cache_out, weight, bias, (uint16_t*)y, N, D, W, act);
  else if (xb)
    short_conv_step_kernel<uint16_t, float><<<grid, 256, 0, s>>>((const uint16_t*)x, cache_in, cache_out, weight, bias, (float*)y, N, D, W, act);
  else if (yb)
    short_conv_step_kernel<float, uint16_t><<<grid, 256, 0, s>>>((const float*)x, cache_in, cache_out, weight, bias, (uint16_t*)y, N, D, W, act);
  else
    short_conv_step_kernel<float, float><<<grid, 256, 0, s>>>((const float*)x, cache_in, cache_out, weight, bias, (float*)y, N, D, W, act);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? TOPS_OK : tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
}
