// Internal interfaces of the KDA chunk kernels (kda_prep.hip, kda_wy.hip; the state sweeps
// are the DELTA instances of gla_sweep.hip).
#pragma once
#include <hip/hip_runtime.h>

namespace tops {

// Chunk-parallel forward preparation (one workgroup per (chunk, head)).
struct KdaPrepParams {
  const void* k;
  const void* v;
  const float* g;          // [B,T,H,K] natural-log gates
  const float* beta;       // [B,T,H]
  float* u;                // [B,T,H,V]  T (beta v)
  float* w;                // [B,T,H,K]  T (beta 2^G k)
  float* tt;               // [total,H,C,C]  T transposed (row i holds column i of T), or NULL
  const int* cu_seqlens;
  const int* chunk_offsets;
  const int* chunk_map;
  int total, B, T, H, K, V, N;
};

template <typename TIn>
hipError_t launch_kda_prep(const KdaPrepParams& p, hipStream_t s);

// Chunk-parallel WY backward (one workgroup per (chunk, head)).
struct KdaWyParams {
  const void* k;
  const void* v;
  const float* g;          // [B,T,H,K]
  const float* beta;       // [B,T,H]
  const float* tt;         // [total,H,C,C]  T transposed
  const float* dvnt;       // [total,H,V,C]  dv_new transposed per chunk
  const float* vnew;       // [B,T,H,V]
  const float* hs;         // [total,H,K,V]  state before each chunk
  void* dv;                // [B,T,H,V]  (TIn)
  float* dbeta;            // [B,T,H]
  float* dk_wy;            // [B,T,H,K]  WY part of dk
  float* dg_wy;            // [B,T,H,K]  WY part of dg (reverse in-chunk cumsum applied)
  const int* cu_seqlens;
  const int* chunk_offsets;
  const int* chunk_map;
  int total, B, T, H, K, V, N;
};

template <typename TIn>
hipError_t launch_kda_wy(const KdaWyParams& p, hipStream_t s);

// The bf16 backward's WY stage and dq / dk / dg in one kernel (kda_bwd_fused.hip): one
// 8-wave workgroup per (chunk, head).
struct KdaBwdParams {
  const void* q;
  const void* k;
  const void* v;           // the layer's v (bf16), for dbeta
  const float* g;          // [B,T,H,K] natural-log gates
  const float* beta;       // [B,T,H]
  const float* tt;         // [total,H,C,C]  T transposed
  const float* dvnt;       // [total,H,V,C]  dv_new transposed per chunk
  const float* vnew;       // [B,T,H,V]
  const float* hs;         // [total,H,K,V]  state before each chunk
  const float* dhs;        // [total,H,K,V]  gradient w.r.t. the state after each chunk
  const void* dout;        // dO [B,T,H,V]
  void* dq;
  void* dk;
  void* dv;
  float* dbeta;            // [B,T,H]
  float* dg;               // [B,T,H,K]
  const int* cu_seqlens;
  const int* chunk_offsets;
  const int* chunk_map;
  int total, B, T, H, K, V, N;
  float scale;
  // fp16 checkpoints (SweepParams::ckpt16): hs and dhs point at fp16 [total,H,K,V] values,
  // scaled per (chunk, head, 64-column tile) by hs_scale / dhs_scale [total,H,ceil(V/64)]
  int ckpt16 = 0;
  const float* hs_scale = nullptr;
  const float* dhs_scale = nullptr;
};

hipError_t launch_kda_bwd_fused(const KdaBwdParams& p, hipStream_t s);

}  // namespace tops
