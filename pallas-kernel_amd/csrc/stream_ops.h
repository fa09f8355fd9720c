// Helpers of the streaming (HBM-bound) kernels: 8- and 4-element vector loads / stores
// (one 16-byte access for 8 bf16 values), sums over aligned lane groups, and a deterministic
// column-sum launcher for per-workgroup partials.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tops_common.h"

namespace tops {

template <typename T> struct V8;
template <> struct V8<uint16_t> {
  __device__ __forceinline__ static void ld(const uint16_t* p, float* v) {
    const uint4 u = *(const uint4*)p;
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
  __device__ __forceinline__ static void st(uint16_t* p, const float* v) {
    *(uint4*)p = make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]),
                            pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7]));
  }
};
template <> struct V8<float> {
  __device__ __forceinline__ static void ld(const float* p, float* v) {
    const float4 a = *(const float4*)p, b = *(const float4*)(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
  __device__ __forceinline__ static void st(float* p, const float* v) {
    *(float4*)p = make_float4(v[0], v[1], v[2], v[3]);
    *(float4*)(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
  }
};

template <typename T> struct V4;
template <> struct V4<uint16_t> {
  __device__ __forceinline__ static void ld(const uint16_t* p, float* v) {
    const uint2 u = *(const uint2*)p;
    v[0] = __uint_as_float(u.x << 16); v[1] = __uint_as_float(u.x & 0xffff0000u);
    v[2] = __uint_as_float(u.y << 16); v[3] = __uint_as_float(u.y & 0xffff0000u);
  }
  __device__ __forceinline__ static void st(uint16_t* p, const float* v) {
    *(uint2*)p = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
  }
};
template <> struct V4<float> {
  __device__ __forceinline__ static void ld(const float* p, float* v) {
    const float4 a = *(const float4*)p;
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  }
  __device__ __forceinline__ static void st(float* p, const float* v) {
    *(float4*)p = make_float4(v[0], v[1], v[2], v[3]);
  }
};

// sum over each aligned group of L lanes (L a power of two <= 64)
template <int L> __device__ __forceinline__ float group_sum(float x) {
#pragma unroll
  for (int o = L / 2; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
  return x;
}

// out0[c] (c < n0) / out1[c - n0] (c >= n0, out1 may be null) = sum over r < np of
// part[r * ncols + c], added in a fixed order.  np <= 4096; when np > 64 the ceil(np / 64) *
// ncols floats after the partials are used as scratch.  Defined in norm_conv.hip.
hipError_t launch_colsum(float* part, int np, int ncols, int n0, float* out0, float* out1,
                         hipStream_t s);
// floats of scratch launch_colsum needs after np rows of ncols partials
inline int64_t colsum_scratch_floats(int np, int ncols) {
  const int ny = np <= 64 ? 1 : (np + 63) / 64;
  return ny > 1 ? (int64_t)ny * ncols : 0;
}

}  // namespace tops
