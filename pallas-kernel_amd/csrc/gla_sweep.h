// Internal interfaces of the GLA chunk kernels (gla_sweep.hip, gla_dqkg.hip).
#pragma once
#include <hip/hip_runtime.h>

namespace tops {

struct SweepParams {
  const void* q;
  const void* k;
  const float* g;
  const void* y;         // v (forward) or dO (reverse)
  const float* s0;       // h0 (forward) or dht (reverse), [N,H,K,V] or NULL
  void* out;             // o (forward) or dv (reverse), [B,T,H,V]
  float* s_fin;          // ht (forward) or dh0 (reverse), or NULL
  float* ckpt;           // [total_chunks,H,K,V] or NULL
  const int* cu_seqlens;
  const int* chunk_offsets;
  int B, T, H, K, V, N, NV;
  float scale;
};

// TIn = uint16_t (bf16 bits) or float; REV = reverse (state-gradient) sweep.
template <typename TIn, bool REV>
hipError_t launch_gla_sweep(const SweepParams& p, hipStream_t s);

struct DqkgParams {
  const void* q;
  const void* k;
  const void* v;
  const float* g;
  const void* dout;
  const float* hs;       // [total, H, K, V] state before each chunk
  const float* dhs;      // [total, H, K, V] gradient w.r.t. the state after each chunk
  void* dq;
  void* dk;
  float* dg;
  const int* cu_seqlens;
  const int* chunk_offsets;
  const int* chunk_map;
  int total, B, T, H, K, V, N;
  float scale;
};

template <typename TIn>
hipError_t launch_gla_dqkg(const DqkgParams& p, hipStream_t s);

}  // namespace tops
