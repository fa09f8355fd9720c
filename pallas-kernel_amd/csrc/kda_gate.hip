// KDA gate activation (forward, chunk-local cumsum, backward) and the row L2 normalisation of
// q / k used by fused_recurrent_kda(use_qk_l2norm_in_kernel=True), for gfx950.
//
// Gate (tops/cpu/ops/kda/gate.py:60-115, tops/ops/kda/gate.py:54-119):
//     standard      y = -exp(A[h]) * softplus(g + b[h, k])
//     lower bound   y = lb * sigmoid(exp(A[h]) * (g + b[h, k]))
// A_log may hold fewer heads than g (head h reads A_log[h / (H / A_heads)]), and dt_bias
// either H or A_heads rows of K (tops/cpu/ops/kda/gate.py:21-57).  The backward sums
// dA and dbias over tokens and over the heads that share a parameter row: every
// workgroup of the elementwise pass writes one partial per (head, column) and a second
// small kernel adds the partials in a fixed order, so the result does not depend on
// scheduling (no atomics).
//
// The cumsum (tops/ops/kda/gate.py:19-51 and tops/cpu/ops/kda/gate.py:179-204) runs one
// thread per (chunk, head, column): consecutive threads read consecutive columns of a
// token row, so each row load of a wave is one contiguous 256-byte (fp32) segment; the
// thread walks its chunk's tokens carrying the running sum in a register.
//
// All of these are HBM-bound streams (a few flops per 4-8 bytes).
#include <math.h>
#include <stdio.h>

#include "stream_ops.h"
#include "tops_common.h"
#include "tops_hip.h"

namespace tops {

struct GateArgs {
  const float* A_log;  // [A_heads]
  const float* bias;   // [bias_heads * K] or null
  int H, K;
  int rep_a, rep_b;    // head h reads A_log[h / rep_a], bias row h / rep_b
  int mode;            // TOPS_KDA_GATE_*
  float lb;
};

// softplus and sigmoid from one e = exp(-|x|) (no overflow for any x):
//   softplus(x) = max(x, 0) + log1p(e),  sigmoid(x) = (x >= 0 ? 1 : e) / (1 + e).
// log1p(e), 0 <= e <= 1, by Kahan's correction log(u) * e / (u - 1) with u = fl(1 + e): exact
// to a few ulp given an accurate log2 (the hardware log2 / reciprocal here, 1 ulp each).
__device__ __forceinline__ float rcp_f(float x) { return __builtin_amdgcn_rcpf(x); }
__device__ __forceinline__ float log1p_unit(float e) {
  const float u = 1.f + e;
  const float d = u - 1.f;
  return d == 0.f ? e : log2f(u) * kLn2 * (e * rcp_f(d));
}
__device__ __forceinline__ float softplus_f(float x) {
  return fmaxf(x, 0.f) + log1p_unit(expf(-fabsf(x)));
}
__device__ __forceinline__ float sigmoid_f(float x) {
  const float e = expf(-fabsf(x));
  const float r = rcp_f(1.f + e);
  return x >= 0.f ? r : e * r;
}
__device__ __forceinline__ void softplus_sigmoid(float x, float& sp, float& sg) {
  const float e = expf(-fabsf(x));
  const float r = rcp_f(1.f + e);
  sp = fmaxf(x, 0.f) + log1p_unit(e);
  sg = x >= 0.f ? r : e * r;
}

// activated gate of one element; eA = exp(A_log[h]), x = g + bias
__device__ __forceinline__ float gate_act(float x, float eA, int mode, float lb) {
  return mode == TOPS_KDA_GATE_LOWER_BOUND ? lb * sigmoid_f(eA * x) : -eA * softplus_f(x);
}

// ---------------------------------------------------------------- forward
// grid (tiles of 1024 columns, row blocks): 4 consecutive columns per thread (K % 4 == 0, so
// the 4 share a head), rows of the block four at a time with the loads issued first
template <typename TIn>
__global__ void __launch_bounds__(256) kda_gate_fwd_kernel(const TIn* __restrict__ g,
                                                           float* __restrict__ y, GateArgs a,
                                                           int rows, int per) {
  const int HK = a.H * a.K;
  const int col = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (col >= HK) return;
  const int h = col / a.K;
  const float eA = expf(a.A_log[h / a.rep_a]);
  float b[4] = {0.f, 0.f, 0.f, 0.f};
  if (a.bias) V4<float>::ld(a.bias + (h / a.rep_b) * a.K + (col - h * a.K), b);
  const int r0 = blockIdx.y * per, r1 = min(r0 + per, rows);
  for (int r = r0; r < r1; r += 4) {
    float v[4][4];
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (r + u < r1) V4<TIn>::ld(g + (long long)(r + u) * HK + col, v[u]);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (r + u >= r1) break;
#pragma unroll
      for (int j = 0; j < 4; ++j) v[u][j] = gate_act(v[u][j] + b[j], eA, a.mode, a.lb);
      V4<float>::st(y + (long long)(r + u) * HK + col, v[u]);
    }
  }
}

// ---------------------------------------------------------------- chunk-local cumsum
// out[t] = scale * sum_{s = chunk start .. t} act(g[s]) per (head, column); act is the
// identity for TOPS_KDA_GATE_NONE.  Chunk c covers tokens [bos, eos) of the flattened
// [B*T] (or packed varlen) token axis.
template <typename TIn>
__global__ void __launch_bounds__(256) kda_gate_cumsum_kernel(
    const TIn* __restrict__ g, float* __restrict__ out, GateArgs a, float scale,
    const int32_t* __restrict__ cu, const int32_t* __restrict__ offs,
    const int32_t* __restrict__ cmap, int T, int C, int tiles) {
  const int HK = a.H * a.K;
  const int c = blockIdx.x / tiles;
  const int col = (blockIdx.x - c * tiles) * 256 + threadIdx.x;
  if (col >= HK) return;
  int bos, eos;
  if (cu) {
    const int n = cmap[c];
    bos = cu[n] + (c - offs[n]) * C;
    eos = min(bos + C, cu[n + 1]);
  } else {
    const int nt = (T + C - 1) / C;
    const int b = c / nt;
    bos = b * T + (c - b * nt) * C;
    eos = min(bos + C, b * T + T);
  }
  const int h = col / a.K;
  float eA = 0.f, bias = 0.f;
  if (a.mode != TOPS_KDA_GATE_NONE) {
    eA = expf(a.A_log[h / a.rep_a]);
    if (a.bias) bias = a.bias[(h / a.rep_b) * a.K + (col - h * a.K)];
  }
  const TIn* gp = g + (long long)bos * HK + col;
  float* op = out + (long long)bos * HK + col;
  float acc = 0.f;
#pragma unroll 8
  for (int t = 0; t < eos - bos; ++t) {
    float x = In<TIn>::ld(gp + (long long)t * HK);
    if (a.mode != TOPS_KDA_GATE_NONE) x = gate_act(x + bias, eA, a.mode, a.lb);
    acc += x * scale;
    op[(long long)t * HK] = acc;
  }
}

// ---------------------------------------------------------------- backward
// grid (tiles of 1024 columns, row blocks).  Each thread owns 4 columns of one head over
// the block's rows: writes dg and one partial per column of dA (per element: dyg * y, or
// dg * x for the lower bound) and of dbias (dg), laid out [row block][2 * H * K].
template <typename TIn>
__global__ void __launch_bounds__(256) kda_gate_bwd_kernel(
    const TIn* __restrict__ g, const float* __restrict__ dyg, TIn* __restrict__ dg,
    float* __restrict__ part, GateArgs a, int rows, int per) {
  const int HK = a.H * a.K;
  const int col = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (col >= HK) return;
  const int rb = blockIdx.y;
  const int r0 = rb * per, r1 = min(r0 + per, rows);
  const int h = col / a.K;
  const float eA = expf(a.A_log[h / a.rep_a]);
  float b[4] = {0.f, 0.f, 0.f, 0.f};
  if (a.bias) V4<float>::ld(a.bias + (h / a.rep_b) * a.K + (col - h * a.K), b);
  float sa[4] = {0.f, 0.f, 0.f, 0.f}, sb[4] = {0.f, 0.f, 0.f, 0.f};
  for (int r = r0; r < r1; r += 4) {
    float x[4][4], dy[4][4];
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (r + u < r1) {
        V4<TIn>::ld(g + (long long)(r + u) * HK + col, x[u]);
        V4<float>::ld(dyg + (long long)(r + u) * HK + col, dy[u]);
      }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (r + u >= r1) break;
      float d[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float xv = x[u][j] + b[j];
        if (a.mode == TOPS_KDA_GATE_LOWER_BOUND) {
          const float s = sigmoid_f(eA * xv);
          d[j] = dy[u][j] * (a.lb * s * (1.f - s)) * eA;
          sa[j] += d[j] * xv;
        } else {
          float sp, sg;
          softplus_sigmoid(xv, sp, sg);
          d[j] = -eA * (dy[u][j] * sg);
          sa[j] += dy[u][j] * (-eA * sp);
        }
        sb[j] += d[j];
      }
      V4<TIn>::st(dg + (long long)(r + u) * HK + col, d);
    }
  }
  float* pp = part + (long long)rb * 2 * HK;
  V4<float>::st(pp + col, sa);
  V4<float>::st(pp + HK + col, sb);
}

// tot_a / tot_b [H * K]: the partials summed over row blocks.  Blocks [0, A_heads):
// dA[ha] = sum over its heads' columns (fixed-order tree); blocks after: dbias[hb * K + k],
// one thread each, summing the heads that share the row.
__global__ void __launch_bounds__(256) kda_gate_fold_kernel(
    const float* __restrict__ tot_a, const float* __restrict__ tot_b, GateArgs a, int A_heads,
    int bias_heads, float* __restrict__ dA, float* __restrict__ dbias) {
  const int tid = threadIdx.x;
  if ((int)blockIdx.x < A_heads) {
    __shared__ float red[256];
    const int ha = blockIdx.x;
    float s = 0.f;
    for (int j = tid; j < a.rep_a * a.K; j += 256) s += tot_a[ha * a.rep_a * a.K + j];
    red[tid] = s;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
      if (tid < w) red[tid] += red[tid + w];
      __syncthreads();
    }
    if (tid == 0) dA[ha] = red[0];
    return;
  }
  const int idx = ((int)blockIdx.x - A_heads) * 256 + tid;
  if (!dbias || idx >= bias_heads * a.K) return;
  const int hb = idx / a.K, k = idx - hb * a.K;
  float s = 0.f;
  for (int i = 0; i < a.rep_b; ++i) s += tot_b[(hb * a.rep_b + i) * a.K + k];
  dbias[idx] = s;
}

// ---------------------------------------------------------------- L2 normalisation
// one wave64 per row of D <= 64 * NV elements: y = x / sqrt(sum x^2 + 1e-6)
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
  return x;
}

template <typename TIn, int NV>
__global__ void __launch_bounds__(256) l2norm_fwd_kernel(const TIn* __restrict__ x,
                                                         float* __restrict__ y, int rows, int D) {
  const int row = blockIdx.x * 4 + threadIdx.x / 64;
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;  // whole wave leaves together
  const TIn* xr = x + (long long)row * D;
  float v[NV];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int d = lane + 64 * i;
    v[i] = d < D ? In<TIn>::ld(xr + d) : 0.f;
    ss += v[i] * v[i];
  }
  const float den = sqrtf(wave_sum(ss) + 1e-6f);
  float* yr = y + (long long)row * D;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int d = lane + 64 * i;
    if (d < D) yr[d] = v[i] / den;
  }
}

// dx = r (dy - y (y . dy)), r = 1 / sqrt(sum x^2 + 1e-6), y = x r
template <typename TIn, int NV>
__global__ void __launch_bounds__(256) l2norm_bwd_kernel(const TIn* __restrict__ x,
                                                         const float* __restrict__ dy,
                                                         TIn* __restrict__ dx, int rows, int D) {
  const int row = blockIdx.x * 4 + threadIdx.x / 64;
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const long long base = (long long)row * D;
  float v[NV], w[NV];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int d = lane + 64 * i;
    v[i] = d < D ? In<TIn>::ld(x + base + d) : 0.f;
    w[i] = d < D ? dy[base + d] : 0.f;
    ss += v[i] * v[i];
  }
  const float r = 1.f / sqrtf(wave_sum(ss) + 1e-6f);
  float sd = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) sd += (v[i] * r) * w[i];
  sd = wave_sum(sd);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int d = lane + 64 * i;
    if (d < D) In<TIn>::st(dx + base + d, r * (w[i] - (v[i] * r) * sd));
  }
}

// vector path (D % 8 == 0, 64 <= D <= 512): LPR lanes per row, 8 consecutive elements per
// lane, 64 / LPR rows per wave, two row groups per iteration in the forward
template <typename TIn, int LPR>
__global__ void __launch_bounds__(256) l2norm_fwd_v8(const TIn* __restrict__ x,
                                                     float* __restrict__ y, int rows, int D) {
  constexpr int RPW = 64 / LPR;
  const int lane = threadIdx.x & 63, sub = lane % LPR, slot = lane / LPR;
  const int nw = gridDim.x * 4;
  const bool col_ok = sub < (D >> 3);
  for (int rg = blockIdx.x * 4 + (threadIdx.x >> 6); rg * RPW < rows; rg += 2 * nw) {
    float v[2][8];
    bool ok[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int row = (rg + u * nw) * RPW + slot;
      ok[u] = row < rows && col_ok;
      if (ok[u]) V8<TIn>::ld(x + (long long)row * D + sub * 8, v[u]);
      else
#pragma unroll
        for (int e = 0; e < 8; ++e) v[u][e] = 0.f;
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += v[u][e] * v[u][e];
      const float den = sqrtf(group_sum<LPR>(ss) + 1e-6f);
      if (!ok[u]) continue;
      const int row = (rg + u * nw) * RPW + slot;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[u][e] = v[u][e] / den;
      V8<float>::st(y + (long long)row * D + sub * 8, v[u]);
    }
  }
}

template <typename TIn, int LPR>
__global__ void __launch_bounds__(256) l2norm_bwd_v8(const TIn* __restrict__ x,
                                                     const float* __restrict__ dy,
                                                     TIn* __restrict__ dx, int rows, int D) {
  constexpr int RPW = 64 / LPR;
  const int lane = threadIdx.x & 63, sub = lane % LPR, slot = lane / LPR;
  const int nw = gridDim.x * 4;
  const bool col_ok = sub < (D >> 3);
  for (int rg = blockIdx.x * 4 + (threadIdx.x >> 6); rg * RPW < rows; rg += nw) {
    const int row = rg * RPW + slot;
    const bool ok = row < rows && col_ok;
    const long long base = (long long)row * D + sub * 8;
    float v[8], w[8];
    if (ok) {
      V8<TIn>::ld(x + base, v);
      V8<float>::ld(dy + base, w);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = w[e] = 0.f;
    }
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += v[e] * v[e];
    const float r = 1.f / sqrtf(group_sum<LPR>(ss) + 1e-6f);
    float sd = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) sd += (v[e] * r) * w[e];
    sd = group_sum<LPR>(sd);
    if (!ok) continue;
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = r * (w[e] - (v[e] * r) * sd);
    V8<TIn>::st(dx + base, o);
  }
}

}  // namespace tops

using namespace tops;

static int gate_check(const char* who, const void* g, int g_dtype, const float* A_log, int rows,
                      int H, int K, int A_heads, int bias_heads, const float* dt_bias, int mode,
                      bool allow_none, GateArgs& a) {
  char msg[200];
  if (!g) {
    snprintf(msg, sizeof(msg), "%s: null gate tensor", who);
    return tops_set_error(TOPS_ERR_NULL, msg);
  }
  if (g_dtype != TOPS_F32 && g_dtype != TOPS_BF16) {
    snprintf(msg, sizeof(msg), "%s: gate dtype must be TOPS_F32 or TOPS_BF16", who);
    return tops_set_error(TOPS_ERR_DTYPE, msg);
  }
  if (rows < 0 || H <= 0 || K <= 0 || (K % 4)) {
    snprintf(msg, sizeof(msg), "%s: need rows >= 0, H > 0, K > 0 and K %% 4 == 0", who);
    return tops_set_error(TOPS_ERR_SHAPE, msg);
  }
  if ((long long)H * K >= (1LL << 30)) {
    snprintf(msg, sizeof(msg), "%s: H * K too large", who);
    return tops_set_error(TOPS_ERR_SHAPE, msg);
  }
  const bool none = mode == TOPS_KDA_GATE_NONE;
  if (!(mode == TOPS_KDA_GATE_SOFTPLUS || mode == TOPS_KDA_GATE_LOWER_BOUND ||
        (allow_none && none))) {
    snprintf(msg, sizeof(msg), "%s: unknown gate mode %d", who, mode);
    return tops_set_error(TOPS_ERR_SHAPE, msg);
  }
  a = GateArgs{A_log, dt_bias, H, K, 1, 1, mode, 0.f};
  if (none) return TOPS_OK;
  if (!A_log) {
    snprintf(msg, sizeof(msg), "%s: A_log is required for gate mode %d", who, mode);
    return tops_set_error(TOPS_ERR_NULL, msg);
  }
  if (A_heads <= 0 || H % A_heads) {
    snprintf(msg, sizeof(msg), "%s: A_log heads %d must divide H %d", who, A_heads, H);
    return tops_set_error(TOPS_ERR_SHAPE, msg);
  }
  a.rep_a = H / A_heads;
  if (dt_bias) {
    if (bias_heads != A_heads && bias_heads != H) {
      snprintf(msg, sizeof(msg), "%s: dt_bias must hold A_heads*K or H*K values", who);
      return tops_set_error(TOPS_ERR_SHAPE, msg);
    }
    a.rep_b = H / bias_heads;
  }
  return TOPS_OK;
}

// row blocks over (tiles of 1024 columns x row blocks): about `target` workgroups, at most
// 4096 row blocks, runs of whole rows
static void row_split(int rows, int HK, int target, int& nrb, int& per) {
  const int tiles = (HK / 4 + 255) / 256;
  nrb = (target + tiles - 1) / tiles;
  if (nrb > rows) nrb = rows;
  if (nrb > 4096) nrb = 4096;
  if (nrb < 1) nrb = 1;
  per = (rows + nrb - 1) / nrb;
  if (per < 1) per = 1;
  nrb = (rows + per - 1) / per;
  if (nrb < 1) nrb = 1;
}

extern "C" int tops_kda_gate_fwd(const void* g, int g_dtype, const float* A_log,
                                 const float* dt_bias, float* y, int rows, int H, int K,
                                 int A_heads, int bias_heads, int gate_mode, float lower_bound,
                                 void* stream) {
  GateArgs a;
  int rc = gate_check("kda_gate_fwd", g, g_dtype, A_log, rows, H, K, A_heads, bias_heads,
                      dt_bias, gate_mode, false, a);
  if (rc != TOPS_OK) return rc;
  if (!y) return tops_set_error(TOPS_ERR_NULL, "kda_gate_fwd: null output");
  a.lb = lower_bound;
  if (rows == 0) return TOPS_OK;
  hipStream_t s = (hipStream_t)stream;
  const int HK = H * K;
  int nrb, per;
  row_split(rows, HK, 8192, nrb, per);
  dim3 grid((HK / 4 + 255) / 256, nrb);
  if (g_dtype == TOPS_BF16)
    kda_gate_fwd_kernel<uint16_t><<<grid, 256, 0, s>>>((const uint16_t*)g, y, a, rows, per);
  else
    kda_gate_fwd_kernel<float><<<grid, 256, 0, s>>>((const float*)g, y, a, rows, per);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? TOPS_OK : tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
}

extern "C" int tops_kda_gate_chunk_cumsum(const void* g, int g_dtype, const float* A_log,
                                          const float* dt_bias, float* out,
                                          const int32_t* cu_seqlens, const int32_t* chunk_offsets,
                                          const int32_t* chunk_map, int total_chunks, int B,
                                          int T, int H, int K, int A_heads, int bias_heads,
                                          int chunk_size, int gate_mode, float lower_bound,
                                          float scale, void* stream) {
  GateArgs a;
  int rc = gate_check("kda_gate_chunk_cumsum", g, g_dtype, A_log, B * T, H, K, A_heads,
                      bias_heads, dt_bias, gate_mode, true, a);
  if (rc != TOPS_OK) return rc;
  if (!out) return tops_set_error(TOPS_ERR_NULL, "kda_gate_chunk_cumsum: null output");
  a.lb = lower_bound;
  if (B <= 0 || T < 0 || chunk_size <= 0)
    return tops_set_error(TOPS_ERR_SHAPE, "kda_gate_chunk_cumsum: need B > 0, T >= 0, chunk_size > 0");
  if (cu_seqlens) {
    if (B != 1 || !chunk_offsets || !chunk_map)
      return tops_set_error(TOPS_ERR_SHAPE,
                            "kda_gate_chunk_cumsum: varlen needs B == 1, chunk_offsets and chunk_map");
  } else if (total_chunks != B * ((T + chunk_size - 1) / chunk_size)) {
    return tops_set_error(TOPS_ERR_SHAPE,
                          "kda_gate_chunk_cumsum: total_chunks must be B*ceil(T/chunk_size)");
  }
  if (total_chunks <= 0 || T == 0) return TOPS_OK;
  const int tiles = (H * K + 255) / 256;
  if ((long long)total_chunks * tiles >= (1LL << 31))
    return tops_set_error(TOPS_ERR_SHAPE, "kda_gate_chunk_cumsum: too many chunks");
  hipStream_t s = (hipStream_t)stream;
  const int grid = total_chunks * tiles;
  if (g_dtype == TOPS_BF16)
    kda_gate_cumsum_kernel<uint16_t><<<grid, 256, 0, s>>>(
        (const uint16_t*)g, out, a, scale, cu_seqlens, chunk_offsets, chunk_map, T, chunk_size, tiles);
  else
    kda_gate_cumsum_kernel<float><<<grid, 256, 0, s>>>(
        (const float*)g, out, a, scale, cu_seqlens, chunk_offsets, chunk_map, T, chunk_size, tiles);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? TOPS_OK : tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
}

// backward workspace: partials [nrb][2 * H * K], the column sum's scratch, totals [2 * H * K]
static void gate_bwd_layout(int rows, int H, int K, int& nrb, int& per, int64_t& n_part,
                            int64_t& n_total) {
  const int HK = H * K;
  row_split(rows > 0 ? rows : 1, HK, 2048, nrb, per);
  n_part = (int64_t)nrb * 2 * HK;
  n_total = n_part + colsum_scratch_floats(nrb, 2 * HK) + 2LL * HK;
}

extern "C" int64_t tops_kda_gate_bwd_workspace(int rows, int H, int K) {
  if (rows < 0 || H <= 0 || K <= 0 || (long long)H * K >= (1LL << 30)) return TOPS_ERR_SHAPE;
  int nrb, per;
  int64_t n_part, n_total;
  gate_bwd_layout(rows, H, K, nrb, per, n_part, n_total);
  return n_total;
}

extern "C" int tops_kda_gate_bwd(const void* g, int g_dtype, const float* A_log,
                                 const float* dt_bias, const float* dyg, void* dg, float* dA,
                                 float* dbias, float* workspace, int64_t workspace_floats,
                                 int rows, int H, int K, int A_heads, int bias_heads,
                                 int gate_mode, float lower_bound, void* stream) {
  GateArgs a;
  int rc = gate_check("kda_gate_bwd", g, g_dtype, A_log, rows, H, K, A_heads, bias_heads,
                      dt_bias, gate_mode, false, a);
  if (rc != TOPS_OK) return rc;
  if (!dyg || !dg || !dA || !workspace || (dt_bias && !dbias))
    return tops_set_error(TOPS_ERR_NULL, "kda_gate_bwd: null tensor");
  a.lb = lower_bound;
  int nrb, per;
  int64_t n_part, n_total;
  gate_bwd_layout(rows, H, K, nrb, per, n_part, n_total);
  if (workspace_floats < n_total)
    return tops_set_error(TOPS_ERR_SHAPE, "kda_gate_bwd: workspace smaller than tops_kda_gate_bwd_workspace()");
  hipStream_t s = (hipStream_t)stream;
  const int HK = H * K;
  float* part = workspace;
  float* tot = workspace + n_total - 2LL * HK;
  hipError_t e = hipSuccess;
  if (rows > 0) {
    dim3 grid((HK / 4 + 255) / 256, nrb);
    if (g_dtype == TOPS_BF16)
      kda_gate_bwd_kernel<uint16_t><<<grid, 256, 0, s>>>((const uint16_t*)g, dyg, (uint16_t*)dg,
                                                          part, a, rows, per);
    else
      kda_gate_bwd_kernel<float><<<grid, 256, 0, s>>>((const float*)g, dyg, (float*)dg, part, a,
                                                       rows, per);
    e = hipGetLastError();
    if (e != hipSuccess) return tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
  }
  // no tokens: zero partial rows, so dA and dbias come out zero
  e = launch_colsum(part, rows > 0 ? nrb : 0, 2 * HK, HK, tot, tot + HK, s);
  if (e != hipSuccess) return tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
  const int nb = dt_bias ? bias_heads : 0;
  const int grid2 = A_heads + (nb * K + 255) / 256;
  kda_gate_fold_kernel<<<grid2, 256, 0, s>>>(tot, tot + HK, a, A_heads, nb, dA,
                                             dt_bias ? dbias : nullptr);
  e = hipGetLastError();
  return e == hipSuccess ? TOPS_OK : tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
}

// L2 norm: vector path for D % 8 == 0, 64 <= D <= 512 (LPR = D / 8 rounded up to a power of
// two); other D one wave per row
static int l2_lpr(int D) {
  if (D % 8 || D < 64 || D > 512) return 0;
  int l = 8;
  while (l < D / 8) l <<= 1;
  return l;
}

template <int NV>
static hipError_t l2_fwd(const void* x, int dt, float* y, int rows, int D, hipStream_t s) {
  if (const int lpr = l2_lpr(D)) {
    const long long groups = ((long long)rows + 64 / lpr - 1) / (64 / lpr);
    long long gl = (groups + 7) / 8;
    const int grid = (int)(gl > 16384 ? 16384 : (gl < 1 ? 1 : gl));
#define TOPS_L2F(L)                                                                        \
  (dt == TOPS_BF16                                                                         \
       ? (l2norm_fwd_v8<uint16_t, L><<<grid, 256, 0, s>>>((const uint16_t*)x, y, rows, D)) \
       : (l2norm_fwd_v8<float, L><<<grid, 256, 0, s>>>((const float*)x, y, rows, D)))
    if (lpr == 8) TOPS_L2F(8);
    else if (lpr == 16) TOPS_L2F(16);
    else if (lpr == 32) TOPS_L2F(32);
    else TOPS_L2F(64);
#undef TOPS_L2F
    return hipGetLastError();
  }
  const int grid = (rows + 3) / 4;
  if (dt == TOPS_BF16)
    l2norm_fwd_kernel<uint16_t, NV><<<grid, 256, 0, s>>>((const uint16_t*)x, y, rows, D);
  else
    l2norm_fwd_kernel<float, NV><<<grid, 256, 0, s>>>((const float*)x, y, rows, D);
  return hipGetLastError();
}

template <int NV>
static hipError_t l2_bwd(const void* x, int dt, const float* dy, void* dx, int rows, int D,
                         hipStream_t s) {
  if (const int lpr = l2_lpr(D)) {
    const long long groups = ((long long)rows + 64 / lpr - 1) / (64 / lpr);
    long long gl = (groups + 3) / 4;
    const int grid = (int)(gl > 16384 ? 16384 : (gl < 1 ? 1 : gl));
#define TOPS_L2B(L)                                                                          \
  (dt == TOPS_BF16 ? (l2norm_bwd_v8<uint16_t, L><<<grid, 256, 0, s>>>(                       \
                         (const uint16_t*)x, dy, (uint16_t*)dx, rows, D))                    \
                   : (l2norm_bwd_v8<float, L><<<grid, 256, 0, s>>>((const float*)x, dy,      \
                                                                   (float*)dx, rows, D)))
    if (lpr == 8) TOPS_L2B(8);
    else if (lpr == 16) TOPS_L2B(16);
    else if (lpr == 32) TOPS_L2B(32);
    else TOPS_L2B(64);
#undef TOPS_L2B
    return hipGetLastError();
  }
  const int grid = (rows + 3) / 4;
  if (dt == TOPS_BF16)
    l2norm_bwd_kernel<uint16_t, NV><<<grid, 256, 0, s>>>((const uint16_t*)x, dy, (uint16_t*)dx,
                                                         rows, D);
  else
    l2norm_bwd_kernel<float, NV><<<grid, 256, 0, s>>>((const float*)x, dy, (float*)dx, rows, D);
  return hipGetLastError();
}

static int l2_check(const char* who, int dtype, int rows, int D) {
  char msg[160];
  if (dtype != TOPS_F32 && dtype != TOPS_BF16) {
    snprintf(msg, sizeof(msg), "%s: dtype must be TOPS_F32 or TOPS_BF16", who);
    return tops_set_error(TOPS_ERR_DTYPE, msg);
  }
  if (rows < 0 || D <= 0 || D > 256 || rows > (1 << 30)) {
    snprintf(msg, sizeof(msg), "%s: need rows >= 0 and 0 < D <= 256", who);
    return tops_set_error(TOPS_ERR_SHAPE, msg);
  }
  return TOPS_OK;
}

extern "C" int tops_l2norm_fwd(const void* x, int x_dtype, float* y, int rows, int D,
                               void* stream) {
  if (!x || !y) return tops_set_error(TOPS_ERR_NULL, "l2norm_fwd: null tensor");
  int rc = l2_check("l2norm_fwd", x_dtype, rows, D);
  if (rc != TOPS_OK) return rc;
  if (rows == 0) return TOPS_OK;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e = D <= 64 ? l2_fwd<1>(x, x_dtype, y, rows, D, s)
               : D <= 128 ? l2_fwd<2>(x, x_dtype, y, rows, D, s)
                          : l2_fwd<4>(x, x_dtype, y, rows, D, s);
  return e == hipSuccess ? TOPS_OK : tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
}

extern "C" int tops_l2norm_bwd(const void* x, int x_dtype, const float* dy, void* dx, int rows,
                               int D, void* stream) {
  if (!x || !dy || !dx) return tops_set_error(TOPS_ERR_NULL, "l2norm_bwd: null tensor");
  int rc = l2_check("l2norm_bwd", x_dtype, rows, D);
  if (rc != TOPS_OK) return rc;
  if (rows == 0) return TOPS_OK;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e = D <= 64 ? l2_bwd<1>(x, x_dtype, dy, dx, rows, D, s)
               : D <= 128 ? l2_bwd<2>(x, x_dtype, dy, dx, rows, D, s)
                          : l2_bwd<4>(x, x_dtype, dy, dx, rows, D, s);
  return e == hipSuccess ? TOPS_OK : tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
}
