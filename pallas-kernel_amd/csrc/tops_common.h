// Shared CDNA4 (gfx950) building blocks for the tops-hip GLA kernels.
//
// Precision scheme: every matrix product runs on v_mfma_f32_16x16x32_bf16 with
// fp32 accumulation.  An operand that is not exactly representable in bf16
// (gated q/k, fp32 states, fp32 inputs) is staged in LDS as a pair of bf16
// planes x = hi + lo (hi = rne(x), lo = rne(x - hi)), which carries ~16
// mantissa bits.  A product then issues hi*hi (+ lo*hi) (+ hi*lo): the lo*lo
// term (~2^-16 relative) is dropped.  Operands that are already bf16 inputs
// (v, do, q, k for bf16 callers) carry no lo plane.
//
// MFMA 16x16x32 bf16 lane layout (verified on gfx950):
//   A (16x32, M x K):  lane l holds A[l%16][8*(l/16) + 0..7]
//   B (32x16, K x N):  lane l holds B[8*(l/16) + 0..7][l%16]
//   D (16x16 fp32)  :  lane l holds D[4*(l/16) + 0..3][l%16]
// The contraction index may be permuted freely as long as A and B agree;
// kernels use this to feed accumulator tiles straight back as operands.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tops {

typedef short bf16x8 __attribute__((__vector_size__(8 * sizeof(short))));
typedef float f32x4 __attribute__((__vector_size__(4 * sizeof(float))));
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;
typedef __attribute__((__vector_size__(2 * sizeof(float)))) float f32x2_t;

constexpr int kChunk = 64;      // tokens per chunk (C)
constexpr int kThreads = 256;   // 4 wave64s per workgroup
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// ---------------------------------------------------------------- scalar helpers
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(((uint32_t)b) << 16);
}
// round-to-nearest-even pack of two floats (v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  f32x2_t x = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(x, bf16x2_t));
}
__device__ __forceinline__ uint16_t f32_to_bf16(float a) {
  return (uint16_t)(pack_bf16x2(a, 0.f) & 0xffffu);
}
// hi/lo split of two floats: returns packed hi pair and packed lo pair
__device__ __forceinline__ void split_bf16x2(float a, float b, uint32_t& hi, uint32_t& lo) {
  hi = pack_bf16x2(a, b);
  float ah = __uint_as_float(hi << 16);
  float bh = __uint_as_float(hi & 0xffff0000u);
  lo = pack_bf16x2(a - ah, b - bh);
}
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Input element loads (bf16 stored as uint16_t, or fp32)
template <typename T> struct In;
template <> struct In<uint16_t> {
  static constexpr bool kExactBf16 = true;
  __device__ __forceinline__ static float ld(const uint16_t* p) { return bf16_to_f32(*p); }
  __device__ __forceinline__ static void ld2(const uint16_t* p, float& a, float& b) {
    uint32_t u = *(const uint32_t*)p;
    a = __uint_as_float(u << 16);
    b = __uint_as_float(u & 0xffff0000u);
  }
  __device__ __forceinline__ static void st(uint16_t* p, float x) { *p = f32_to_bf16(x); }
};
template <> struct In<float> {
  static constexpr bool kExactBf16 = false;
  __device__ __forceinline__ static float ld(const float* p) { return *p; }
  __device__ __forceinline__ static void ld2(const float* p, float& a, float& b) {
    float2 u = *(const float2*)p;
    a = u.x;
    b = u.y;
  }
  __device__ __forceinline__ static void st(float* p, float x) { *p = x; }
};

// ---------------------------------------------------------------- MFMA
__device__ __forceinline__ f32x4 mfma(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
// split product: hi*hi (+ lo_a*hi_b) (+ hi_a*lo_b)
template <bool SA, bool SB>
__device__ __forceinline__ f32x4 mma(f32x4 c, const bf16x8& ah, const bf16x8& al,
                                     const bf16x8& bh, const bf16x8& bl) {
  if constexpr (SA) c = mfma(al, bh, c);
  if constexpr (SB) c = mfma(ah, bl, c);
  return mfma(ah, bh, c);
}

// ---------------------------------------------------------------- LDS planes
// A plane stores a matrix as [outer][contraction] (contraction contiguous),
// bf16 hi plane plus (optionally) a lo plane at a fixed offset.
struct Plane {
  uint16_t* hi;
  uint16_t* lo;
  int ld;  // elements between consecutive outer rows (multiple of 8)
  __device__ __forceinline__ bf16x8 hi8(int r, int c) const {
    return __builtin_bit_cast(bf16x8, *(const uint4*)(hi + r * ld + c));
  }
  __device__ __forceinline__ bf16x8 lo8(int r, int c) const {
    return __builtin_bit_cast(bf16x8, *(const uint4*)(lo + r * ld + c));
  }
  // two runs of 4 contiguous elements: [c0, c0+4) and [c1, c1+4)
  __device__ __forceinline__ bf16x8 hi44(int r, int c0, int c1) const {
    uint2 x = *(const uint2*)(hi + r * ld + c0);
    uint2 y = *(const uint2*)(hi + r * ld + c1);
    uint4 z = {x.x, x.y, y.x, y.y};
    return __builtin_bit_cast(bf16x8, z);
  }
  __device__ __forceinline__ bf16x8 lo44(int r, int c0, int c1) const {
    uint2 x = *(const uint2*)(lo + r * ld + c0);
    uint2 y = *(const uint2*)(lo + r * ld + c1);
    uint4 z = {x.x, x.y, y.x, y.y};
    return __builtin_bit_cast(bf16x8, z);
  }
  // store x at (r, c) as hi (and lo)
  template <bool SPLIT>
  __device__ __forceinline__ void put2(int r, int c, float a, float b) const {
    if constexpr (SPLIT) {
      uint32_t h, l;
      split_bf16x2(a, b, h, l);
      *(uint32_t*)(hi + r * ld + c) = h;
      *(uint32_t*)(lo + r * ld + c) = l;
    } else {
      *(uint32_t*)(hi + r * ld + c) = pack_bf16x2(a, b);
    }
  }
  // store n (even, 4..16) consecutive contraction values for one outer row
  template <bool SPLIT, int NV>
  __device__ __forceinline__ void put_run(int r, int c, const float* x) const {
    uint32_t h[NV / 2], l[NV / 2];
#pragma unroll
    for (int i = 0; i < NV / 2; ++i) {
      if constexpr (SPLIT) split_bf16x2(x[2 * i], x[2 * i + 1], h[i], l[i]);
      else h[i] = pack_bf16x2(x[2 * i], x[2 * i + 1]);
    }
    static_assert(NV % 4 == 0, "runs are written as 8-byte pieces");
#pragma unroll
    for (int i = 0; i < NV / 2; i += 2) {
      *(uint2*)(hi + r * ld + c + 2 * i) = make_uint2(h[i], h[i + 1]);
      if constexpr (SPLIT) *(uint2*)(lo + r * ld + c + 2 * i) = make_uint2(l[i], l[i + 1]);
    }
  }
};

// 4 consecutive fp32 accumulator values (rows 4*(l/16)+0..3 of one column)
// converted to hi/lo bf16 halves of an operand register.
__device__ __forceinline__ void acc_to_bf16x4(const f32x4& a, uint2& hi, uint2& lo) {
  split_bf16x2(a[0], a[1], hi.x, lo.x);
  split_bf16x2(a[2], a[3], hi.y, lo.y);
}
__device__ __forceinline__ bf16x8 cat44(const uint2& x, const uint2& y) {
  uint4 z = {x.x, x.y, y.x, y.y};
  return __builtin_bit_cast(bf16x8, z);
}

__device__ __forceinline__ int cdiv(int a, int b) { return (a + b - 1) / b; }

// Map a linear workgroup id so that `group` consecutive logical ids land on
// the same XCD (dispatch round-robins workgroups over the 8 XCDs): logical
// ids that share data (e.g. the V tiles of one head) then share an L2.
__device__ __forceinline__ int xcd_remap(int wg, int nwg, int group) {
  constexpr int kXcd = 8;
  if (group <= 1 || (nwg % (kXcd * group)) != 0) return wg;
  int xcd = wg % kXcd;
  int slot = wg / kXcd;
  int per_xcd = nwg / kXcd;
  int blk = slot / group, sub = slot % group;
  (void)per_xcd;
  return (blk * kXcd + xcd) * group + sub;
}

}  // namespace tops
