// C-ABI entry points of the chunked KDA (include/tops_hip.h).
//
// Forward (tops_kda_chunk_fwd): the chunk-parallel WY preparation (kda_prep.hip: gate
// cumsum, Akk, T = (I + Akk)^-1, u, w) and the delta-rule state sweep (the DELTA instance of
// gla_sweep.hip: v_new = u - w S, o, S per chunk), replacing chunk_kda_fwd's four stages
// (tops/ops/kda/chunk.py:25-190).
//
// Backward (tops_kda_chunk_bwd): the reverse delta-rule sweep (dv_new, dS per chunk,
// dh0), the WY backward (kda_wy.hip: dv, dbeta and the WY parts of dk, dg), then the
// GLA-shaped dq / dk / dg kernel (gla_dqkg.hip with v := v_new) which adds the WY parts,
// replacing chunk_kda_bwd (tops/ops/kda/chunk_bwd.py:655-832).
#include <stdio.h>

#include "gla_sweep.h"
#include "kda.h"
#include "tops_common.h"
#include "tops_hip.h"

using namespace tops;

static int kda_check(const char* who, int B, int T, int H, int K, int V, int N, int total_chunks,
                     const int32_t* cu_seqlens, const int32_t* chunk_offsets,
                     const int32_t* chunk_map, int dtype) {
  char msg[160];
  if (B <= 0 || T <= 0 || H <= 0 || K <= 0 || V <= 0 || N <= 0) {
    snprintf(msg, sizeof(msg), "%s: non-positive dimension", who);
    return tops_set_error(TOPS_ERR_SHAPE, msg);
  }
  if (K > 128 || V > 128 || (K % 8) || (V % 8)) {
    snprintf(msg, sizeof(msg), "%s: need K, V <= 128 and multiples of 8", who);
    return tops_set_error(TOPS_ERR_SHAPE, msg);
  }
  if ((long long)kChunk * H * (K > V ? K : V) * 4 >= (1LL << 31)) {
    snprintf(msg, sizeof(msg), "%s: H * max(K, V) too large for 32-bit chunk offsets", who);
    return tops_set_error(TOPS_ERR_SHAPE, msg);
  }
  if (cu_seqlens && (B != 1 || !chunk_offsets || !chunk_map)) {
    snprintf(msg, sizeof(msg), "%s: varlen needs B == 1, chunk_offsets and chunk_map", who);
    return tops_set_error(TOPS_ERR_SHAPE, msg);
  }
  if (!cu_seqlens && N != B) {
    snprintf(msg, sizeof(msg), "%s: N must equal B", who);
    return tops_set_error(TOPS_ERR_SHAPE, msg);
  }
  if (!cu_seqlens && total_chunks != B * ((T + kChunk - 1) / kChunk)) {
    snprintf(msg, sizeof(msg), "%s: total_chunks must be B*ceil(T/64)", who);
    return tops_set_error(TOPS_ERR_SHAPE, msg);
  }
  if (total_chunks <= 0) {
    snprintf(msg, sizeof(msg), "%s: total_chunks must be positive", who);
    return tops_set_error(TOPS_ERR_SHAPE, msg);
  }
  if (dtype != TOPS_BF16 && dtype != TOPS_F32) {
    snprintf(msg, sizeof(msg), "%s: dtype must be TOPS_F32 or TOPS_BF16", who);
    return tops_set_error(TOPS_ERR_DTYPE, msg);
  }
  return TOPS_OK;
}

extern "C" int tops_kda_chunk_fwd(const void* q, const void* k, const void* v, const float* g,
                                  const float* beta, const float* h0, void* o, float* ht, float* u,
                                  float* w, float* tt, float* v_new, float* h_ckpt,
                                  const int32_t* cu_seqlens, const int32_t* chunk_offsets,
                                  const int32_t* chunk_map, int total_chunks, int B, int T, int H,
                                  int K, int V, int N, int dtype, float scale, void* stream) {
  if (!q || !k || !v || !g || !beta || !o || !u || !w)
    return tops_set_error(TOPS_ERR_NULL, "kda_chunk_fwd: null tensor");
  int rc = kda_check("kda_chunk_fwd", B, T, H, K, V, N, total_chunks, cu_seqlens, chunk_offsets,
                     chunk_map, dtype);
  if (rc != TOPS_OK) return rc;
  hipStream_t s = (hipStream_t)stream;
  KdaPrepParams pp{k, v, g, beta, u, w, tt, cu_seqlens, chunk_offsets, chunk_map,
                   total_chunks, B, T, H, K, V, N};
  hipError_t e = dtype == TOPS_BF16 ? launch_kda_prep<uint16_t>(pp, s) : launch_kda_prep<float>(pp, s);
  if (e != hipSuccess) return tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
  SweepParams sp{q, k, g, nullptr, h0, o, ht, h_ckpt, cu_seqlens, chunk_offsets,
                 B, T, H, K, V, N, (V + 63) / 64, scale, kGateK, u, w, v_new};
  e = dtype == TOPS_BF16 ? launch_gla_sweep<uint16_t, false, true>(sp, s)
                         : launch_gla_sweep<float, false, true>(sp, s);
  if (e != hipSuccess) return tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
  return TOPS_OK;
}

extern "C" int tops_kda_chunk_bwd(const void* q, const void* k, const void* v, const float* g,
                                  const float* beta, const float* w, const float* tt,
                                  const float* v_new, const float* h_ckpt, const void* do_,
                                  const float* dht, float* dh_work, float* dvn_work, float* dk_work,
                                  float* dg_work, void* dq, void* dk, void* dv, float* dbeta,
                                  float* dg, float* dh0, const int32_t* cu_seqlens,
                                  const int32_t* chunk_offsets, const int32_t* chunk_map,
                                  int total_chunks, int B, int T, int H, int K, int V, int N,
                                  int dtype, float scale, void* stream) {
  if (!q || !k || !v || !g || !beta || !w || !tt || !v_new || !h_ckpt || !do_ || !dh_work ||
      !dvn_work || !dk_work || !dg_work || !dq || !dk || !dv || !dbeta || !dg)
    return tops_set_error(TOPS_ERR_NULL, "kda_chunk_bwd: null tensor");
  int rc = kda_check("kda_chunk_bwd", B, T, H, K, V, N, total_chunks, cu_seqlens, chunk_offsets,
                     chunk_map, dtype);
  if (rc != TOPS_OK) return rc;
  hipStream_t s = (hipStream_t)stream;
  const bool bf = dtype == TOPS_BF16;
  // 1. reverse delta-rule sweep: dv_new (transposed per chunk), dS per chunk, dh0
  SweepParams sp{q, k, g, do_, dht, nullptr, dh0, dh_work, cu_seqlens, chunk_offsets,
                 B, T, H, K, V, N, (V + 63) / 64, scale, kGateK, nullptr, w, dvn_work};
  hipError_t e = bf ? launch_gla_sweep<uint16_t, true, true>(sp, s) : launch_gla_sweep<float, true, true>(sp, s);
  if (e != hipSuccess) return tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
  // 2. WY backward: dv, dbeta, dk_wy, dg_wy
  KdaWyParams wp{k, v, g, beta, tt, dvn_work, v_new, h_ckpt, dv, dbeta, dk_work, dg_work,
                 cu_seqlens, chunk_offsets, chunk_map, total_chunks, B, T, H, K, V, N};
  e = bf ? launch_kda_wy<uint16_t>(wp, s) : launch_kda_wy<float>(wp, s);
  if (e != hipSuccess) return tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
  // 3. dq, dk, dg of the GLA-shaped terms (v := v_new), plus the WY parts
  DqkgParams dp{q, k, v_new, g, do_, h_ckpt, dh_work, dq, dk, dg, cu_seqlens, chunk_offsets,
                chunk_map, total_chunks, B, T, H, K, V, N, scale, kGateK, dk_work, dg_work};
  e = bf ? launch_gla_dqkg<uint16_t, float>(dp, s) : launch_gla_dqkg<float, float>(dp, s);
  if (e != hipSuccess) return tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
  return TOPS_OK;
}
