// Gate gradient of the value-gated recurrence (fused_recurrent_gla with gv, the chunked
// backward of tops/ops/gla/fused_recurrent.py:496-619; oracle
// tops/cpu/ops/gla/fused_recurrent.py:171-358):
//     dgv[t, v] = sum over t' >= t in the same sequence of (o[t', v] dO[t', v] - v[t', v] dv[t', v])
//                 + c[n, v],
// c[n] = sum_k (dht * ht)[n, k, :] the final-state term (or none).  One workgroup per
// (sequence, head, 64-column tile) walks the sequence from its end in blocks of 16 runs x 8
// tokens: each thread holds one run of one column in registers, forms the run's own suffix
// sums, the 16 run totals are combined through LDS (double-buffered, one barrier per block)
// and the carry from the later blocks is added.  The next block's inputs are fetched before
// the current block is scanned; loads and stores are non-temporal, as nothing is touched
// twice (159 against 179 us at B16 T2048 H8 V128).  Each input is read once and dgv written
// once: HBM-bound at 16 bytes per (token, column) with o and dv fp32 and dO and v bf16, 2
// more when the bf16 copy of dv is written on the way.
#include "tops_common.h"
#include "tops_hip.h"

namespace tops {

namespace {

constexpr int kCols = 64, kRuns = 16, kRun = 8, kBlock = kRuns * kRun;

__global__ __launch_bounds__(kCols * kRuns) void gv_gate_grad_kernel(
    const float* o32, const uint16_t* dO, const uint16_t* v, const float* dv32, const float* c,
    float* dgv, uint16_t* dv_out, const int32_t* cu_seqlens, int T, int H, int V, int NVT) {
  const int col = threadIdx.x % kCols, run = threadIdx.x / kCols;
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
  const bool ok = vv < V;
  const size_t rs = (size_t)H * V;                       // elements between tokens
  const size_t base = ((size_t)t0 * H + hh) * V + vv;
  // block b (counted from the sequence's end) holds tokens [L - (b + 1) kBlock, L - b kBlock);
  // this thread's run of it starts at first(b); tokens before the sequence's start are zeros
  auto first = [&](int b) { return L - (b + 1) * kBlock + run * kRun; };
  float xo[kRun], xd[kRun];
  uint16_t xg[kRun], xv[kRun];
  auto fetch = [&](int b) {
    const int tb = first(b);
#pragma unroll
    for (int j = 0; j < kRun; ++j) {
      const int t = tb + j;
      if (ok && t >= 0) {
        const size_t e = base + (size_t)t * rs;
        xo[j] = __builtin_nontemporal_load(o32 + e);
        xd[j] = __builtin_nontemporal_load(dv32 + e);
        xg[j] = __builtin_nontemporal_load(dO + e);
        xv[j] = __builtin_nontemporal_load(v + e);
      } else {
        xo[j] = xd[j] = 0.f;
        xg[j] = xv[j] = 0;
      }
    }
  };
  __shared__ float tot[2][kRuns][kCols];
  float carry = (ok && c) ? c[((size_t)n * H + hh) * V + vv] : 0.f;
  const int nblk = (L + kBlock - 1) / kBlock;
  fetch(0);
  for (int b = 0; b < nblk; ++b) {
    const int tb = first(b);
    float s[kRun];
#pragma unroll
    for (int j = 0; j < kRun; ++j) s[j] = xo[j] * bf16_to_f32(xg[j]) - bf16_to_f32(xv[j]) * xd[j];
    if (dv_out && ok) {
#pragma unroll
      for (int j = 0; j < kRun; ++j)
        if (tb + j >= 0) __builtin_nontemporal_store(f32_to_bf16(xd[j]), dv_out + base + (size_t)(tb + j) * rs);
    }
    if (b + 1 < nblk) fetch(b + 1);
#pragma unroll
    for (int j = kRun - 2; j >= 0; --j) s[j] += s[j + 1];
    float(*tt)[kCols] = tot[b & 1];
    tt[run][col] = s[0];
    __syncthreads();
    // every thread of the column adds the run totals in the same order, so all of them carry
    // the same value into the next block; off is the carry plus the totals of the later runs
    float acc = carry, off = carry;
#pragma unroll
    for (int r = kRuns - 1; r >= 0; --r) {
      if (r == run) off = acc;
      acc += tt[r][col];
    }
    if (ok) {
#pragma unroll
      for (int j = 0; j < kRun; ++j)
        if (tb + j >= 0) __builtin_nontemporal_store(off + s[j], dgv + base + (size_t)(tb + j) * rs);
    }
    carry = acc;
  }
}

}  // namespace

}  // namespace tops

extern "C" int tops_gv_gate_grad(const float* o32, const void* dO, const void* v, const float* dv32,
                                 const float* c, float* dgv, void* dv_out,
                                 const int32_t* cu_seqlens, int B, int T, int H, int V, int N,
                                 int dtype, void* stream) {
  using namespace tops;
  if (!o32 || !dO || !v || !dv32 || !dgv) return tops_set_error(TOPS_ERR_NULL, "gv_gate_grad: null tensor");
  if (dtype != TOPS_BF16) return tops_set_error(TOPS_ERR_DTYPE, "gv_gate_grad: dO and v must be TOPS_BF16");
  if (B <= 0 || T <= 0 || H <= 0 || V <= 0 || N <= 0)
    return tops_set_error(TOPS_ERR_SHAPE, "gv_gate_grad: non-positive dimension");
  if (cu_seqlens && B != 1) return tops_set_error(TOPS_ERR_SHAPE, "gv_gate_grad: varlen needs B == 1");
  if (!cu_seqlens && N != B) return tops_set_error(TOPS_ERR_SHAPE, "gv_gate_grad: N must equal B");
  const int NVT = (V + kCols - 1) / kCols;
  hipLaunchKernelGGL(gv_gate_grad_kernel, dim3(N * H * NVT), dim3(kCols * kRuns), 0,
                     (hipStream_t)stream, o32, (const uint16_t*)dO, (const uint16_t*)v, dv32, c,
                     dgv, (uint16_t*)dv_out, cu_seqlens, T, H, V, NVT);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
  return TOPS_OK;
}
