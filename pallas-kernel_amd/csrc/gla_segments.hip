// Sequence-parallel chunk sweeps: a long sequence is cut at chunk boundaries into segments
// that sweep concurrently.  The recurrence of every K row is linear,
//   S_end = 2^{D} S_begin + S_local,   D = sum of the log2 gates over the segment,
// so (1) a state-only sweep per segment from a zero state gives (D, S_local), (2) a short
// scan over the segments of each sequence gives every segment's incoming state, and (3) the
// full sweep runs over the segments with those states injected.  The reverse sweep is the
// mirror image (segments scanned from the end of the sequence).  The associative form is
// the one the reference's state recurrence implies (tops/ops/common/chunk_h.py:160-238 for
// the forward, :685-878 for the reverse); the reference itself sweeps each sequence serially.
#include <stdio.h>

#include "gla_sweep.h"
#include "tops_common.h"
#include "tops_hip.h"

namespace tops {

// One thread per (sequence, head, K row, 4 V columns): walks the state-pass entries of its
// sequence in sweep order, carrying the state across them, and writes the incoming state of
// every segment.  Sequence n owns the segments [seg_first[n], seg_first[n+1]) of the full list
// and the entries [st_first[n], st_first[n+1]) (stored in sweep order); after entry e the
// running state enters segment st_dst[e] (or no segment: -1, when the entry ends inside one).
__global__ void __launch_bounds__(256)
state_combine_kernel(const float* __restrict__ s_loc, const float* __restrict__ dec,
                     const float* __restrict__ s_in, float* __restrict__ init,
                     const int32_t* __restrict__ seg_first, const int32_t* __restrict__ st_first,
                     const int32_t* __restrict__ st_dst, int Nreal, int H, int K, int V,
                     int reverse) {
  const int V4 = V >> 2;
  const long long gid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long per_seq = (long long)H * K * V4;
  if (gid >= (long long)Nreal * per_seq) return;
  const int n = (int)(gid / per_seq);
  const long long rem = gid - (long long)n * per_seq;   // (h, k, v4)
  const int hk = (int)(rem / V4);                        // h * K + k
  const int v4 = (int)(rem - (long long)hk * V4);
  const size_t hkv = (size_t)hk * V + 4 * v4;            // offset inside one [H,K,V] state
  const size_t st = (size_t)H * K * V;
  float4 S = s_in ? *(const float4*)(s_in + (size_t)n * st + hkv) : make_float4(0.f, 0.f, 0.f, 0.f);
  const int j_first = reverse ? seg_first[n + 1] - 1 : seg_first[n];
  *(float4*)(init + (size_t)j_first * st + hkv) = S;
  for (int e = st_first[n]; e < st_first[n + 1]; ++e) {
    const float a = exp2f(dec[(size_t)e * H * K + hk]);
    const float4 l = *(const float4*)(s_loc + (size_t)e * st + hkv);
    S.x = a * S.x + l.x;
    S.y = a * S.y + l.y;
    S.z = a * S.z + l.z;
    S.w = a * S.w + l.w;
    const int j = st_dst[e];
    if (j >= 0) *(float4*)(init + (size_t)j * st + hkv) = S;
  }
}

}  // namespace tops

using namespace tops;

extern "C" int tops_chunk_state_pass(const void* z, const void* y, const float* g, int gate_mode,
                                     float* s_loc, float* dec, const int32_t* seg_start,
                                     const int32_t* seg_end, int T, int H, int K, int V, int N,
                                     int dtype, float scale, int reverse, void* stream) {
  if (!z || !y || !g || !s_loc || !dec || !seg_start || !seg_end)
    return tops_set_error(TOPS_ERR_NULL, "chunk_state_pass: null tensor");
  if (T <= 0 || H <= 0 || K <= 0 || V <= 0 || N <= 0)
    return tops_set_error(TOPS_ERR_SHAPE, "chunk_state_pass: non-positive dimension");
  if (K > 128 || V > 128 || (K % 8) || (V % 8))
    return tops_set_error(TOPS_ERR_SHAPE, "chunk_state_pass: need K, V <= 128 and multiples of 8");
  if ((long long)kChunk * H * (K > V ? K : V) * 4 >= (1LL << 31))
    return tops_set_error(TOPS_ERR_SHAPE, "chunk_state_pass: H * max(K, V) too large");
  if (gate_mode != kGateK && gate_mode != kGateS && gate_mode != kGateGamma && gate_mode != kGateGammaK)
    return tops_set_error(TOPS_ERR_SHAPE, "chunk_state_pass: unknown gate mode");
  // z fills both the q and the k slot: the state-only sweep multiplies only one of them.
  SweepParams p{z, z, g, y, nullptr, nullptr, s_loc, nullptr, seg_start, nullptr,
                1, T, H, K, V, N, (V + 63) / 64, scale, gate_mode};
  p.dec_fin = dec;
  p.seg_end = seg_end;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  if (dtype == TOPS_BF16)
    e = reverse ? launch_gla_state_pass<uint16_t, true>(p, s) : launch_gla_state_pass<uint16_t, false>(p, s);
  else if (dtype == TOPS_F32)
    e = reverse ? launch_gla_state_pass<float, true>(p, s) : launch_gla_state_pass<float, false>(p, s);
  else if (dtype == TOPS_F16)
    e = reverse ? launch_gla_state_pass<_Float16, true>(p, s) : launch_gla_state_pass<_Float16, false>(p, s);
  else
    return tops_set_error(TOPS_ERR_DTYPE, "chunk_state_pass: dtype must be TOPS_F32, TOPS_BF16 or TOPS_F16");
  if (e != hipSuccess) return tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
  return TOPS_OK;
}

extern "C" int tops_chunk_state_combine(const float* s_loc, const float* dec, const float* s_in,
                                        float* init, const int32_t* seg_first,
                                        const int32_t* st_first, const int32_t* st_dst,
                                        int Nreal, int H, int K, int V, int reverse,
                                        void* stream) {
  if (!init || !seg_first || !st_first || !st_dst)
    return tops_set_error(TOPS_ERR_NULL, "chunk_state_combine: null tensor");
  if (Nreal <= 0 || H <= 0 || K <= 0 || V <= 0 || (V % 4))
    return tops_set_error(TOPS_ERR_SHAPE, "chunk_state_combine: need positive sizes, V % 4 == 0");
  const long long n = (long long)Nreal * H * K * (V / 4);
  const long long blocks = (n + 255) / 256;
  if (blocks > 0x7fffffffLL) return tops_set_error(TOPS_ERR_SHAPE, "chunk_state_combine: too large");
  hipLaunchKernelGGL(state_combine_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     (hipStream_t)stream, s_loc, dec, s_in, init, seg_first, st_first, st_dst,
                     Nreal, H, K, V, reverse);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
  return TOPS_OK;
}
