// Gate gradient of the value-gated recurrence (fused_recurrent_gla with gv, the chunked
// backward of tops/ops/gla/fused_recurrent.py:496-619; oracle
// tops/cpu/ops/gla/fused_recurrent.py:171-358):
//     dgv[t, v] = sum over t' >= t in the same sequence of (o[t', v] dO[t', v] - v[t', v] dv[t', v])
//                 + c[n, v],
// c[n] = sum_k (dht * ht)[n, k, :] the final-state term (or none).  One workgroup per
// (sequence, head, 64-column tile): 16 token parts x 64 columns; each part first sums its own
// tokens, the parts' totals are combined through LDS, and a second walk writes the running
// suffix sums.  HBM-bound: o and dv fp32, dO and v bf16 read twice, dgv written once.
#include "tops_common.h"
#include "tops_hip.h"

namespace tops {

namespace {

constexpr int kCols = 64, kParts = 16;

__global__ __launch_bounds__(kCols * kParts) void gv_gate_grad_kernel(
    const float* o32, const uint16_t* dO, const uint16_t* v, const float* dv32, const float* c,
    float* dgv, const int32_t* cu_seqlens, int T, int H, int V, int NVT) {
  const int col = threadIdx.x % kCols, part = threadIdx.x / kCols;
  const int vt = blockIdx.x % NVT, hh = (blockIdx.x / NVT) % H, n = blockIdx.x / (NVT * H);
  const int vv = vt * kCols + col;
  int t0, L;
  if (cu_seqlens) {
    t0 = cu_seqlens[n];
    L = cu_seqlens[n + 1] - t0;
  } else {
    t0 = n * T;
    L = T;
  }
  // this part's tokens [p0, p1) of the sequence
  const int per = (L + kParts - 1) / kParts;
  const int p0 = min(L, part * per), p1 = min(L, p0 + per);
  const bool ok = vv < V;
  const size_t rs = (size_t)H * V;                       // elements between tokens
  const size_t base = ((size_t)t0 * H + hh) * V + vv;
  auto term = [&](int t) {
    const size_t e = base + (size_t)t * rs;
    return o32[e] * bf16_to_f32(dO[e]) - bf16_to_f32(v[e]) * dv32[e];
  };
  float s = 0.f;
  if (ok) {
#pragma unroll 8
    for (int t = p1 - 1; t >= p0; --t) s += term(t);
  }
  __shared__ float tot[kParts][kCols];
  tot[part][col] = s;
  __syncthreads();
  float run = (ok && c) ? c[((size_t)n * H + hh) * V + vv] : 0.f;
  for (int p = kParts - 1; p > part; --p) run += tot[p][col];
  if (ok) {
#pragma unroll 8
    for (int t = p1 - 1; t >= p0; --t) {
      run += term(t);
      dgv[base + (size_t)t * rs] = run;
    }
  }
}

}  // namespace

}  // namespace tops

extern "C" int tops_gv_gate_grad(const float* o32, const void* dO, const void* v, const float* dv32,
                                 const float* c, float* dgv, const int32_t* cu_seqlens, int B,
                                 int T, int H, int V, int N, int dtype, void* stream) {
  using namespace tops;
  if (!o32 || !dO || !v || !dv32 || !dgv) return tops_set_error(TOPS_ERR_NULL, "gv_gate_grad: null tensor");
  if (dtype != TOPS_BF16) return tops_set_error(TOPS_ERR_DTYPE, "gv_gate_grad: dO and v must be TOPS_BF16");
  if (B <= 0 || T <= 0 || H <= 0 || V <= 0 || N <= 0)
    return tops_set_error(TOPS_ERR_SHAPE, "gv_gate_grad: non-positive dimension");
  if (cu_seqlens && B != 1) return tops_set_error(TOPS_ERR_SHAPE, "gv_gate_grad: varlen needs B == 1");
  if (!cu_seqlens && N != B) return tops_set_error(TOPS_ERR_SHAPE, "gv_gate_grad: N must equal B");
  const int NVT = (V + kCols - 1) / kCols;
  hipLaunchKernelGGL(gv_gate_grad_kernel, dim3(N * H * NVT), dim3(kCols * kParts), 0,
                     (hipStream_t)stream, o32, (const uint16_t*)dO, (const uint16_t*)v, dv32, c,
                     dgv, cu_seqlens, T, H, V, NVT);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
  return TOPS_OK;
}
