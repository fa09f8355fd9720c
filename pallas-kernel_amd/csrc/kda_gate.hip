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

__device__ __forceinline__ float softplus_f(float x) {
  return fmaxf(x, 0.f) + log1pf(expf(-fabsf(x)));
}
__device__ __forceinline__ float sigmoid_f(float x) { return 1.f / (1.f + expf(-x)); }

// activated gate of one element; eA = exp(A_log[h]), x = g + bias
__device__ __forceinline__ float gate_act(float x, float eA, int mode, float lb) {
  return mode == TOPS_KDA_GATE_LOWER_BOUND ? lb * sigmoid_f(eA * x) : -eA * softplus_f(x);
}

template <typename TIn> struct Vec4;
template <> struct Vec4<float> {
  __device__ __forceinline__ static void ld(const float* p, float* v) {
    float4 u = *(const float4*)p;
    v[0] = u.x; v[1] = u.y; v[2] = u.z; v[3] = u.w;
  }
  __device__ __forceinline__ static void st(float* p, const float* v) {
    *(float4*)p = make_float4(v[0], v[1], v[2], v[3]);
  }
};
template <> struct Vec4<uint16_t> {
  __device__ __forceinline__ static void ld(const uint16_t* p, float* v) {
    uint2 u = *(const uint2*)p;
    v[0] = __uint_as_float(u.x << 16); v[1] = __uint_as_float(u.x & 0xffff0000u);
    v[2] = __uint_as_float(u.y << 16); v[3] = __uint_as_float(u.y & 0xffff0000u);
  }
  __device__ __forceinline__ static void st(uint16_t* p, const float* v) {
    *(uint2*)p = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
  }
};

// ---------------------------------------------------------------- forward
// 4 consecutive columns per thread (K % 4 == 0, so the 4 share a head)
template <typename TIn>
__global__ void __launch_bounds__(256) kda_gate_fwd_kernel(const TIn* __restrict__ g,
                                                           float* __restrict__ y, GateArgs a,
                                                           long long n4) {
  const int HK = a.H * a.K;
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n4;
       i += (long long)gridDim.x * 256) {
    const long long e = i * 4;
    const int col = (int)(e % HK);
    const int h = col / a.K;
    const float eA = expf(a.A_log[h / a.rep_a]);
    float v[4];
    Vec4<TIn>::ld(g + e, v);
    if (a.bias) {
      const float* b = a.bias + (h / a.rep_b) * a.K + (col - h * a.K);
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] += b[j];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = gate_act(v[j], eA, a.mode, a.lb);
    Vec4<float>::st(y + e, v);
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
// grid (column tiles of 256, row blocks).  Each thread owns one (head, column) over the
// block's rows: writes dg and one partial of dA (per element: dyg * y, or dg * x for the
// lower bound) and of dbias (dg).
template <typename TIn>
__global__ void __launch_bounds__(256) kda_gate_bwd_kernel(
    const TIn* __restrict__ g, const float* __restrict__ dyg, TIn* __restrict__ dg,
    float* __restrict__ part_a, float* __restrict__ part_b, GateArgs a, int rows,
    int rows_per_blk) {
  const int HK = a.H * a.K;
  const int col = blockIdx.x * 256 + threadIdx.x;
  if (col >= HK) return;
  const int rb = blockIdx.y;
  const int r0 = rb * rows_per_blk;
  const int r1 = min(r0 + rows_per_blk, rows);
  const int h = col / a.K;
  const float eA = expf(a.A_log[h / a.rep_a]);
  const float bias = a.bias ? a.bias[(h / a.rep_b) * a.K + (col - h * a.K)] : 0.f;
  float sa = 0.f, sb = 0.f;
#pragma unroll 4
  for (int r = r0; r < r1; ++r) {
    const long long off = (long long)r * HK + col;
    const float x = In<TIn>::ld(g + off) + bias;
    const float dy = dyg[off];
    float d;
    if (a.mode == TOPS_KDA_GATE_LOWER_BOUND) {
      const float s = sigmoid_f(eA * x);
      d = dy * (a.lb * s * (1.f - s)) * eA;
      sa += d * x;
    } else {
      d = -eA * (dy * sigmoid_f(x));
      sa += dy * (-eA * softplus_f(x));
    }
    sb += d;
    In<TIn>::st(dg + off, d);
  }
  part_a[(long long)rb * HK + col] = sa;
  part_b[(long long)rb * HK + col] = sb;
}

// blocks [0, A_heads): dA[ha] = sum over its heads, columns and row blocks (fixed-order tree
// over the workgroup); blocks after: dbias[hb * K + k], one thread each.
__global__ void __launch_bounds__(256) kda_gate_bwd_reduce_kernel(
    const float* __restrict__ part_a, const float* __restrict__ part_b, int nrb, GateArgs a,
    int A_heads, int bias_heads, float* __restrict__ dA, float* __restrict__ dbias) {
  const int HK = a.H * a.K;
  const int tid = threadIdx.x;
  if ((int)blockIdx.x < A_heads) {
    __shared__ float red[256];
    const int ha = blockIdx.x;
    float s = 0.f;
    for (int j = tid; j < a.rep_a * a.K; j += 256) {
      const int col = ha * a.rep_a * a.K + j;  // heads ha*rep_a .. are contiguous columns
      for (int r = 0; r < nrb; ++r) s += part_a[(long long)r * HK + col];
    }
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
  for (int i = 0; i < a.rep_b; ++i) {
    const int col = (hb * a.rep_b + i) * a.K + k;
    for (int r = 0; r < nrb; ++r) s += part_b[(long long)r * HK + col];
  }
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

static int grid_of(long long n, int per_block, int cap) {
  long long b = (n + per_block - 1) / per_block;
  return (int)(b < 1 ? 1 : (b > cap ? cap : b));
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
  const long long n4 = (long long)rows * H * K / 4;
  if (n4 == 0) return TOPS_OK;
  hipStream_t s = (hipStream_t)stream;
  const int grid = grid_of(n4, 256, 256 * 32);
  if (g_dtype == TOPS_BF16)
    kda_gate_fwd_kernel<uint16_t><<<grid, 256, 0, s>>>((const uint16_t*)g, y, a, n4);
  else
    kda_gate_fwd_kernel<float><<<grid, 256, 0, s>>>((const float*)g, y, a, n4);
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

// row blocks of the backward: about 2048 workgroups in all
static void gate_bwd_split(int rows, int H, int K, int& nrb, int& per) {
  const int tiles = (H * K + 255) / 256;
  nrb = (2048 + tiles - 1) / tiles;
  if (nrb > rows) nrb = rows;
  if (nrb < 1) nrb = 1;
  per = (rows + nrb - 1) / nrb;
  if (per < 1) per = 1;
  nrb = (rows + per - 1) / per;
  if (nrb < 1) nrb = 1;
}

extern "C" int64_t tops_kda_gate_bwd_workspace(int rows, int H, int K) {
  if (rows < 0 || H <= 0 || K <= 0) return TOPS_ERR_SHAPE;
  int nrb, per;
  gate_bwd_split(rows, H, K, nrb, per);
  return 2LL * nrb * H * K;
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
  gate_bwd_split(rows, H, K, nrb, per);
  const long long HK = (long long)H * K;
  if (workspace_floats < 2LL * nrb * HK)
    return tops_set_error(TOPS_ERR_SHAPE, "kda_gate_bwd: workspace smaller than tops_kda_gate_bwd_workspace()");
  hipStream_t s = (hipStream_t)stream;
  float* part_a = workspace;
  float* part_b = workspace + (long long)nrb * HK;
  const int tiles = (int)((HK + 255) / 256);
  if (rows > 0) {
    dim3 grid(tiles, nrb);
    if (g_dtype == TOPS_BF16)
      kda_gate_bwd_kernel<uint16_t><<<grid, 256, 0, s>>>((const uint16_t*)g, dyg, (uint16_t*)dg,
                                                          part_a, part_b, a, rows, per);
    else
      kda_gate_bwd_kernel<float><<<grid, 256, 0, s>>>((const float*)g, dyg, (float*)dg, part_a,
                                                       part_b, a, rows, per);
  } else {
    nrb = 0;  // no tokens: dA and dbias are zero
  }
  const int nb = dt_bias ? bias_heads : 0;
  const int grid2 = A_heads + (nb * K + 255) / 256;
  kda_gate_bwd_reduce_kernel<<<grid2, 256, 0, s>>>(part_a, part_b, nrb, a, A_heads, nb,
                                                   dA, dt_bias ? dbias : nullptr);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? TOPS_OK : tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
}

template <int NV>
static hipError_t l2_fwd(const void* x, int dt, float* y, int rows, int D, hipStream_t s) {
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
