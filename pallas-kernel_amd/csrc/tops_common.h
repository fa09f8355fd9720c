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

// sigmoid from e = exp(-|x|) and the hardware reciprocal (1 ulp); no overflow for any x.
// e is the hardware 2^x of -|x| log2(e): its relative error, about |x| 2^-24 from rounding
// the product, moves the sigmoid by at most ~1e-7 for |x| < 16 (and e itself is below 2^-23
// beyond that), two VALU operations instead of the library expf's range reduction.
__device__ __forceinline__ float sigm(float x) {
  const float e = fast_exp2(-fabsf(x) * kLog2e);
  const float r = __builtin_amdgcn_rcpf(1.f + e);
  return x >= 0.f ? r : e * r;
}

// Cross-lane sums inside one 16-lane DPP row, on the VALU (no LDS round trip).  A lane whose
// DPP source lies outside its row reads 0.
template <int CTRL>
__device__ __forceinline__ float dpp_row(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
// every lane of a row gets the sum over the row's 16 lanes
__device__ __forceinline__ float row16_sum(float x) {
  x += dpp_row<0xB1>(x);   // quad_perm [1,0,3,2]: pairs
  x += dpp_row<0x4E>(x);   // quad_perm [2,3,0,1]: quads
  x += dpp_row<0x141>(x);  // row_half_mirror: lane i <- 7 - i, the other quad of the half
  x += dpp_row<0x140>(x);  // row_mirror: lane i <- 15 - i, the other half of the row
  return x;
}
// lane l of a row gets the sum over lanes l .. 15 of its row (inclusive suffix sum)
__device__ __forceinline__ float row16_suffix_sum(float x) {
  x += dpp_row<0x101>(x);  // row_shl:1, lane l <- l + 1
  x += dpp_row<0x102>(x);
  x += dpp_row<0x104>(x);
  x += dpp_row<0x108>(x);
  return x;
}

// Inclusive scan over the four 8-lane segments of each half-wave: lane l (l & 31 = 8 s + c)
// gets the sum of t over lanes 8 s' + c (s' <= s) of its half-wave.  DPP row_shr:8 adds the
// first segment of a 16-lane row to the second, row_shl:8 spreads the row's total over the
// row, v_permlane16_swap hands the even row's total to the odd row: all on the VALU (a
// cross-lane shuffle goes through the LDS queue).  Call with every lane active.
__device__ __forceinline__ float seg8x4_scan(float t, int lane) {
  const bool hi = (lane & 15) >= 8, odd = lane & 16;
  const float a = t + dpp_row<0x118>(t);                // 0 from lanes 0..7 of a row
  // a sum, not a select: the compiler may turn a select into a branch, and a DPP read in it
  // finds its source lanes switched off
  const float rt = dpp_row<0x108>(a) + (hi ? a : 0.f);  // 0 from lanes 8..15 of a row
  const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(rt), __float_as_uint(rt),
                                                   false, false);
  return a + (odd ? __uint_as_float(sw[0]) : 0.f);
}
// the value of lane l ^ 16 and of lane l ^ 32 (v_permlane16_swap / v_permlane32_swap)
__device__ __forceinline__ float lane_xor16(float x, int lane) {
  const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x),
                                                  false, false);
  return __uint_as_float((lane & 16) ? s[0] : s[1]);
}
__device__ __forceinline__ float lane_xor32(float x, int lane) {
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                  false, false);
  return __uint_as_float((lane & 32) ? s[0] : s[1]);
}

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

// fp16 elements (_Float16): 11 mantissa bits and an exponent range inside bf16's, so a bf16
// hi / lo pair holds every fp16 value exactly and fp16 inputs take the split path of fp32
// ones.  The word types are distinct from the bf16 ones (uint2 / uint32_t) so that the
// unpack overloads pick the fp16 conversion.
struct H4 { uint2 u; };        // 4 consecutive fp16 elements
struct H2 { uint32_t u; };     // 2 consecutive fp16 elements
__device__ __forceinline__ float f16_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(h & 0xffffu));
}
// round-to-nearest-even pack of two floats to fp16 (v_cvt_f16_f32)
__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
  const uint32_t lo = __builtin_bit_cast(uint16_t, (_Float16)a);
  const uint32_t hi = __builtin_bit_cast(uint16_t, (_Float16)b);
  return lo | (hi << 16);
}
template <> struct In<_Float16> {
  static constexpr bool kExactBf16 = false;
  __device__ __forceinline__ static float ld(const _Float16* p) { return (float)*p; }
  __device__ __forceinline__ static void ld2(const _Float16* p, float& a, float& b) {
    const uint32_t u = *(const uint32_t*)p;
    a = f16_to_f32(u);
    b = f16_to_f32(u >> 16);
  }
  __device__ __forceinline__ static void st(_Float16* p, float x) { *p = (_Float16)x; }
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

// ---------------------------------------------------------------- LDS transpose reads
// ds_read_b64_tr_b16 (gfx950), lane layout measured on MI355X: within each group of 16
// lanes, lane i supplies the address of row i/4, columns 4(i%4)..4(i%4)+3 of a 4 x 16 block
// of a row-major 16-bit matrix, and receives column i's four rows.  Two such reads give an
// MFMA 16x16x32 operand whose contraction index runs down the rows of a row-major plane:
// lane l gets P[r0 + 8(l/16) + 0..7][c0 + l%16].
typedef short v4i16 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ bf16x8 tr_read8(const uint16_t* plane, int ld, int r0, int c0, int lane) {
  const int g = lane >> 4, i = lane & 15;
  const uint16_t* p = plane + (r0 + 8 * g + (i >> 2)) * ld + c0 + 4 * (i & 3);
  typedef __attribute__((address_space(3))) v4i16 lds_v4;
  const v4i16 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4*)(p));
  const v4i16 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4*)(p + 4 * ld));
  const uint2 ua = __builtin_bit_cast(uint2, a), ub = __builtin_bit_cast(uint2, b);
  return __builtin_bit_cast(bf16x8, make_uint4(ua.x, ua.y, ub.x, ub.y));
}
// The same for two separate 4-row blocks (rows ra + 4(l/16) + 0..3 and rb + 4(l/16) + 0..3):
// the operand of a contraction permuted as the accumulator tiles of two 16-blocks hold it.
__device__ __forceinline__ bf16x8 tr_read44(const uint16_t* plane, int ld, int ra, int rb, int c0,
                                           int lane) {
  const int g = lane >> 4, i = lane & 15;
  typedef __attribute__((address_space(3))) v4i16 lds_v4;
  const uint16_t* pa = plane + (ra + 4 * g + (i >> 2)) * ld + c0 + 4 * (i & 3);
  const uint16_t* pb = plane + (rb + 4 * g + (i >> 2)) * ld + c0 + 4 * (i & 3);
  const v4i16 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4*)(pa));
  const v4i16 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4*)(pb));
  const uint2 ua = __builtin_bit_cast(uint2, a), ub = __builtin_bit_cast(uint2, b);
  return __builtin_bit_cast(bf16x8, make_uint4(ua.x, ua.y, ub.x, ub.y));
}

// ---------------------------------------------------------------- buffer resources
// Raw (stride 0) buffer descriptors: 32-bit byte offsets from an SGPR base, and the
// hardware range check returns 0 for a load (drops a store) whose offset is at or past
// num_records.  Masked elements use kOOB, which is past any num_records set here
// (num_records is capped at 2^31 - 1).  The software row / column masks are what keep
// every access inside its tensor (the check covers the VGPR offset; the per-row SGPR
// offsets the kernels add are guarded by their row masks); the resources of the chunk
// kernels are built with make_rsrc_rows so that they also end at the tensor's end.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr uint32_t kOOB = 0x80000000u;
constexpr int kRsrcFlags = 0x00020000;  // gfx9 family: raw untyped dword access

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, long long bytes) {
  const int n = bytes <= 0 ? 0 : (bytes > 0x7fffffffLL ? 0x7fffffff : (int)bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, n, kRsrcFlags);
}
// Resource over the tail of a row tensor [nrows, width] of element type T (a [B, T, H, W]
// tensor is nrows = B*T*H rows of W), starting at row e0 (= token_row * H + head): the range
// ends exactly at the end of the tensor, whatever head e0 names, so the hardware check
// drops any access past the last element.
template <typename T>
__device__ __forceinline__ rsrc_t make_rsrc_rows(const T* t, size_t e0, long long nrows, int width) {
  if (t == nullptr) return make_rsrc(nullptr, 0);
  return make_rsrc(t + e0 * (size_t)width, (nrows - (long long)e0) * width * (long long)sizeof(T));
}
// Resource over one chunk of one head of a row tensor [.., H, width]: nval token rows of
// `width` elements, `tstride` elements apart, from row e0 (= token_row * H + head).  The range
// ends at the end of the last valid token's row, so the rows past the chunk's valid tokens (a
// ragged tail, the next sequence) fail the hardware check and need no mask of their own;
// nval <= 0 gives an empty range.
// (32-bit sizes: a chunk spans less than 2^31 bytes, which the entry points check as
// kChunk * H * max(K, V) * 4 < 2^31.)
template <typename T>
__device__ __forceinline__ rsrc_t chunk_rsrc(const T* t, size_t e0, int nval, int tstride,
                                             int width) {
  const int n = (t != nullptr && nval > 0) ? ((nval - 1) * tstride + width) * (int)sizeof(T) : 0;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(t + e0 * (size_t)width), (short)0, n,
                                           kRsrcFlags);
}
__device__ __forceinline__ uint32_t bld32(rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 0);
}
__device__ __forceinline__ uint2 bld64(rsrc_t r, uint32_t voff, uint32_t soff) {
  auto v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)voff, (int)soff, 0);
  return make_uint2(v[0], v[1]);
}
__device__ __forceinline__ uint4 bld128(rsrc_t r, uint32_t voff, uint32_t soff) {
  auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ void bst32(rsrc_t r, uint32_t x, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_buffer_store_b32(x, r, (int)voff, (int)soff, 0);
}
__device__ __forceinline__ void bst64(rsrc_t r, uint2 x, uint32_t voff, uint32_t soff) {
  typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
  u32x2 v = {x.x, x.y};
  __builtin_amdgcn_raw_buffer_store_b64(v, r, (int)voff, (int)soff, 0);
}
__device__ __forceinline__ void bst128(rsrc_t r, uint4 x, uint32_t voff, uint32_t soff) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  u32x4 v = {x.x, x.y, x.z, x.w};
  __builtin_amdgcn_raw_buffer_store_b128(v, r, (int)voff, (int)soff, 0);
}

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

// ---------------------------------------------------------------- shared helpers
// Raw input words -> floats (bf16 bits or fp32)
__device__ __forceinline__ void unpack4(const uint2& u, float* x) {
  x[0] = __uint_as_float(u.x << 16);
  x[1] = __uint_as_float(u.x & 0xffff0000u);
  x[2] = __uint_as_float(u.y << 16);
  x[3] = __uint_as_float(u.y & 0xffff0000u);
}
__device__ __forceinline__ void unpack4(const uint4& u, float* x) {
  x[0] = __uint_as_float(u.x); x[1] = __uint_as_float(u.y);
  x[2] = __uint_as_float(u.z); x[3] = __uint_as_float(u.w);
}
__device__ __forceinline__ void unpack2(const uint32_t& u, float& a, float& b) {
  a = __uint_as_float(u << 16);
  b = __uint_as_float(u & 0xffff0000u);
}
__device__ __forceinline__ void unpack2(const uint2& u, float& a, float& b) {
  a = __uint_as_float(u.x);
  b = __uint_as_float(u.y);
}
__device__ __forceinline__ void unpack4(const H4& w, float* x) {
  x[0] = f16_to_f32(w.u.x); x[1] = f16_to_f32(w.u.x >> 16);
  x[2] = f16_to_f32(w.u.y); x[3] = f16_to_f32(w.u.y >> 16);
}
__device__ __forceinline__ void unpack2(const H2& w, float& a, float& b) {
  a = f16_to_f32(w.u);
  b = f16_to_f32(w.u >> 16);
}
// 8 fp16 elements of a 16-byte piece
__device__ __forceinline__ void unpack8_f16(const uint4& u, float* x) {
  unpack4(H4{make_uint2(u.x, u.y)}, x);
  unpack4(H4{make_uint2(u.z, u.w)}, x + 4);
}
// Word types: 4 and 2 consecutive elements of TIn
template <typename TIn> struct Words;
template <> struct Words<uint16_t> {
  typedef uint2 W4;
  typedef uint32_t W2;
  __device__ __forceinline__ static W4 ld4(rsrc_t r, uint32_t v, uint32_t s) { return bld64(r, v, s); }
  __device__ __forceinline__ static W2 ld2(rsrc_t r, uint32_t v, uint32_t s) { return bld32(r, v, s); }
  __device__ __forceinline__ static void st4(rsrc_t r, const f32x4& x, uint32_t v, uint32_t s) {
    bst64(r, make_uint2(pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3])), v, s);
  }
};
template <> struct Words<_Float16> {
  typedef H4 W4;
  typedef H2 W2;
  __device__ __forceinline__ static W4 ld4(rsrc_t r, uint32_t v, uint32_t s) { return H4{bld64(r, v, s)}; }
  __device__ __forceinline__ static W2 ld2(rsrc_t r, uint32_t v, uint32_t s) { return H2{bld32(r, v, s)}; }
  __device__ __forceinline__ static void st4(rsrc_t r, const f32x4& x, uint32_t v, uint32_t s) {
    bst64(r, make_uint2(pack_f16x2(x[0], x[1]), pack_f16x2(x[2], x[3])), v, s);
  }
};
template <> struct Words<float> {
  typedef uint4 W4;
  typedef uint2 W2;
  __device__ __forceinline__ static W4 ld4(rsrc_t r, uint32_t v, uint32_t s) { return bld128(r, v, s); }
  __device__ __forceinline__ static W2 ld2(rsrc_t r, uint32_t v, uint32_t s) { return bld64(r, v, s); }
  __device__ __forceinline__ static void st4(rsrc_t r, const f32x4& x, uint32_t v, uint32_t s) {
    bst128(r, make_uint4(__float_as_uint(x[0]), __float_as_uint(x[1]), __float_as_uint(x[2]),
                         __float_as_uint(x[3])), v, s);
  }
};

// write n (1, 2, 4 or 8) consecutive contraction values of one plane row, hi (and lo)
template <bool SPLIT, int NE>
__device__ __forceinline__ void put_n(const Plane& P, int r, int c, const float* x) {
  if constexpr (NE == 1) {
    uint32_t h, l;
    if constexpr (SPLIT) split_bf16x2(x[0], 0.f, h, l);
    else h = pack_bf16x2(x[0], 0.f);
    P.hi[r * P.ld + c] = (uint16_t)(h & 0xffffu);
    if constexpr (SPLIT) P.lo[r * P.ld + c] = (uint16_t)(l & 0xffffu);
  } else {
    uint32_t h[NE / 2], l[NE / 2];
#pragma unroll
    for (int i = 0; i < NE / 2; ++i) {
      if constexpr (SPLIT) split_bf16x2(x[2 * i], x[2 * i + 1], h[i], l[i]);
      else h[i] = pack_bf16x2(x[2 * i], x[2 * i + 1]);
    }
    uint16_t* ph = P.hi + r * P.ld + c;
    uint16_t* pl = P.lo + r * P.ld + c;
    if constexpr (NE == 2) {
      *(uint32_t*)ph = h[0];
      if constexpr (SPLIT) *(uint32_t*)pl = l[0];
    } else if constexpr (NE == 4) {
      *(uint2*)ph = make_uint2(h[0], h[1]);
      if constexpr (SPLIT) *(uint2*)pl = make_uint2(l[0], l[1]);
    } else {
      static_assert(NE == 8, "1, 2, 4 or 8 elements");
      *(uint4*)ph = make_uint4(h[0], h[1], h[2], h[3]);
      if constexpr (SPLIT) *(uint4*)pl = make_uint4(l[0], l[1], l[2], l[3]);
    }
  }
}

// Four outputs of one channel slice of a sliced call, summed over the slices in fp32: mode 1
// writes the sum buffer (Ra, byte offset fo), 2 adds into it, 3 writes the final value to the
// output (Ro, offsets oo / so); 4 (an unsliced call that wants both) writes the value to the
// sum buffer and to the output.
template <typename TIn>
__device__ __forceinline__ void acc_slice_t(const rsrc_t& Ro, const rsrc_t& Ra, f32x4 acc,
                                            uint32_t fo, uint32_t oo, uint32_t so, int mode) {
  if (mode == 2 || mode == 3) {
    const uint4 prev = bld128(Ra, fo, 0);
    acc[0] += __uint_as_float(prev.x);
    acc[1] += __uint_as_float(prev.y);
    acc[2] += __uint_as_float(prev.z);
    acc[3] += __uint_as_float(prev.w);
  }
  if (mode == 3 || mode == 4) Words<TIn>::st4(Ro, acc, oo, so);
  if (mode != 3)
    bst128(Ra, make_uint4(__float_as_uint(acc[0]), __float_as_uint(acc[1]), __float_as_uint(acc[2]),
                          __float_as_uint(acc[3])), fo, 0);
}

// ---- fp16 state checkpoints (SweepParams::ckpt16).  A sweep workgroup holds the [K, 64]
// state tile of one (chunk, head, V tile) in MFMA accumulators: wave w's tile i covers rows
// 16 msb + 4 (lane >> 4) + r (r = 0..3) and column 16 nn + (lane & 15), nn = (w NHT + i) % 4.
// The checkpoint stores it as fp16 times 2^(14 - e), e the exponent of the tile's largest
// |S| (so every stored value is below 2^15; fp16's largest normal is 65504), and the factor
// 2^(e - 14) as one fp32.
//
// This wave's largest |S| as fp32 bits (non-negative floats order as their bit patterns):
// DPP maxima inside each 16-lane row, then the four rows' lane 0 by readlane, all on the VALU
// (a cross-lane shuffle would queue behind the sweep's LDS traffic); lane 0 writes smx[wave].
// Call with every lane active.
template <int NHT>
__device__ __forceinline__ void state_absmax(const f32x4 (&S)[NHT], uint32_t* smx, int wave,
                                             int lane) {
  uint32_t m = 0u;
#pragma unroll
  for (int i = 0; i < NHT; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) m = max(m, __float_as_uint(S[i][r]) & 0x7fffffffu);
  m = max(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0xB1, 0xF, 0xF, false));
  m = max(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x4E, 0xF, 0xF, false));
  m = max(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x141, 0xF, 0xF, false));
  m = max(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x140, 0xF, 0xF, false));
  const uint32_t w = max(max((uint32_t)__builtin_amdgcn_readlane((int)m, 0),
                             (uint32_t)__builtin_amdgcn_readlane((int)m, 16)),
                         max((uint32_t)__builtin_amdgcn_readlane((int)m, 32),
                             (uint32_t)__builtin_amdgcn_readlane((int)m, 48)));
  if (lane == 0) smx[wave] = w;
}
// The checkpoint of this wave's fragment (smx of every wave visible), into the [K, V] fp16
// slot `base` (row length V) and its factor into *fac (thread 0 of the workgroup).  Lanes
// 2j, 2j + 1 hold adjacent columns of the same rows: each packs its two rows of a row pair,
// the pair swap their packs (DPP quad_perm [1,0,3,2]) and v_perm picks the even lane's first
// row and the odd lane's second, so every store is one 4-byte run of a row.
template <int NHT, int NW>
__device__ __forceinline__ void store_state16(const f32x4 (&S)[NHT], const uint32_t* smx,
                                              uint16_t* base, float* fac, int K, int V, int vt,
                                              int wave, int msb, int lane, int tid) {
  uint32_t m = smx[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) m = max(m, smx[w]);
  int ex = (int)((m >> 23) & 0xffu) - 127;
  ex = ex < -100 ? -100 : ex;
  const float sinv = __uint_as_float((uint32_t)(141 - ex) << 23);
  if (tid == 0) *fac = __uint_as_float((uint32_t)(113 + ex) << 23);
  const rsrc_t R = make_rsrc(base, (long long)K * V * 2);
  const int l16 = lane & 15, lg = lane >> 4;
  const int odd = l16 & 1;
  const uint32_t sel = odd ? 0x03020706u : 0x05040100u;
  // rows kr + odd and kr + 2 + odd (kr + 3 < K whenever kr < K: K is a multiple of 8); the
  // second row pair is a uniform offset of two rows
  const int kr = 16 * msb + 4 * lg;
#pragma unroll
  for (int i = 0; i < NHT; ++i) {
    const int nn = (wave * NHT + i) % 4;
    const int vv = vt * 64 + 16 * nn + (l16 & ~1);
    const uint32_t vo = (kr < K && vv < V) ? ((uint32_t)(kr + odd) * V + vv) * 2u : kOOB;
#pragma unroll
    for (int rp = 0; rp < 2; ++rp) {
      const uint32_t own = pack_f16x2(S[i][2 * rp] * sinv, S[i][2 * rp + 1] * sinv);
      const uint32_t other = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)own, 0xB1, 0xF, 0xF, false);
      bst32(R, __builtin_amdgcn_perm(other, own, sel), vo, (uint32_t)(rp * 4 * V));
    }
  }
}

// The same checkpoint from transposed fragments (lane (l16, lg) of tile (msb, nn) holding
// S[16 msb + l16][16 nn + 4 lg + r], r = 0..3): each lane's four values are one 8-byte run
// of a row, stored directly.
template <int NHT, int NW>
__device__ __forceinline__ void store_state16_t(const f32x4 (&S)[NHT], const uint32_t* smx,
                                                uint16_t* base, float* fac, int K, int V, int vt,
                                                int wave, int msb, int lane, int tid) {
  uint32_t m = smx[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) m = max(m, smx[w]);
  int ex = (int)((m >> 23) & 0xffu) - 127;
  ex = ex < -100 ? -100 : ex;
  const float sinv = __uint_as_float((uint32_t)(141 - ex) << 23);
  if (tid == 0) *fac = __uint_as_float((uint32_t)(113 + ex) << 23);
  const rsrc_t R = make_rsrc(base, (long long)K * V * 2);
  const int l16 = lane & 15, lg = lane >> 4;
  const int kr = 16 * msb + l16;
#pragma unroll
  for (int i = 0; i < NHT; ++i) {
    const int nn = (wave * NHT + i) % 4;
    const int vv = vt * 64 + 16 * nn + 4 * lg;
    // (V % 8 == 0: vv < V keeps the run inside the row)
    const uint32_t vo = (kr < K && vv < V) ? ((uint32_t)kr * V + vv) * 2u : kOOB;
    bst64(R, make_uint2(pack_f16x2(S[i][0] * sinv, S[i][1] * sinv),
                        pack_f16x2(S[i][2] * sinv, S[i][3] * sinv)), vo, 0);
  }
}

}  // namespace tops
