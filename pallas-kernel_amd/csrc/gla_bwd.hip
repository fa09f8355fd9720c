// C-ABI entry points of the GLA chunked backward (include/tops_hip.h).
//
// Stage 1, tops_gla_chunk_bwd_dh, is the reverse instance of the chunk sweep
// (gla_sweep.hip): dh per chunk, dv and dh0 -- the reference's K8 chunk_bwd_dh
// (tops/ops/common/chunk_h.py:685-878) plus the dv part of K4.  Stage 2,
// tops_gla_chunk_bwd_dqkg, is the chunk-parallel dq / dk / dg kernel (gla_dqkg.hip) --
// the rest of K4 (tops/ops/gla/chunk.py:1447-1581).
#include <stdio.h>

#include "gla_sweep.h"
#include "tops_common.h"
#include "tops_hip.h"

namespace tops {


// Shape checks shared by the backward entry points; returns TOPS_OK or an error code.
static int check_bwd(const char* who, int B, int T, int H, int K, int V, int N, int total_chunks,
                     const int32_t* cu_seqlens, const int32_t* chunk_offsets,
                     const int32_t* chunk_map, bool need_map, int dtype, int ldk = 0,
                     int ldv = 0, bool wide_v = false) {
  char msg[160];
  if (B <= 0 || T <= 0 || H <= 0 || K <= 0 || V <= 0 || N <= 0) {
    snprintf(msg, sizeof(msg), "%s: non-positive dimension", who);
    return tops_set_error(TOPS_ERR_SHAPE, msg);
  }
  if (K > 128 || (V > 128 && !wide_v) || (K % 8) || (V % 8)) {
    snprintf(msg, sizeof(msg), "%s: need K, V <= 128 and multiples of 8", who);
    return tops_set_error(TOPS_ERR_SHAPE, msg);
  }
  const int kw = ldk > 0 ? ldk : K, vw = ldv > 0 ? ldv : V;
  if ((ldk && (ldk < K || (ldk % 8))) || (ldv && (ldv < V || (ldv % 8)))) {
    snprintf(msg, sizeof(msg), "%s: ldk / ldv must be multiples of 8, at least K / V", who);
    return tops_set_error(TOPS_ERR_SHAPE, msg);
  }
  if ((long long)kChunk * H * (kw > vw ? kw : vw) * 4 >= (1LL << 31)) {
    snprintf(msg, sizeof(msg), "%s: H * max(K, V) too large for 32-bit chunk offsets", who);
    return tops_set_error(TOPS_ERR_SHAPE, msg);
  }
  if (cu_seqlens && (B != 1 || !chunk_offsets || (need_map && !chunk_map))) {
    snprintf(msg, sizeof(msg), "%s: varlen needs B == 1, chunk_offsets and chunk_map", who);
    return tops_set_error(TOPS_ERR_SHAPE, msg);
  }
  if (!cu_seqlens && N != B) {
    snprintf(msg, sizeof(msg), "%s: N must equal B", who);
    return tops_set_error(TOPS_ERR_SHAPE, msg);
  }
  if (!cu_seqlens && need_map && total_chunks != B * ((T + kChunk - 1) / kChunk)) {
    snprintf(msg, sizeof(msg), "%s: total_chunks must be B*ceil(T/64)", who);
    return tops_set_error(TOPS_ERR_SHAPE, msg);
  }
  if (need_map && total_chunks <= 0) {
    snprintf(msg, sizeof(msg), "%s: total_chunks must be positive", who);
    return tops_set_error(TOPS_ERR_SHAPE, msg);
  }
  if (dtype != TOPS_BF16 && dtype != TOPS_F32 && dtype != TOPS_F16) {
    snprintf(msg, sizeof(msg), "%s: dtype must be TOPS_F32, TOPS_BF16 or TOPS_F16", who);
    return tops_set_error(TOPS_ERR_DTYPE, msg);
  }
  return TOPS_OK;
}

}  // namespace tops

using namespace tops;

static int bwd_dh_impl(const void* q, const void* k, const float* g, const void* do_,
                       const float* dht, float* dh_work, void* dv, float* dh0,
                       const int32_t* cu_seqlens, const int32_t* chunk_offsets, int B, int T, int H,
                       int K, int V, int N, int dtype, float scale, int gate_mode, void* stream,
                       int ckpt_par = 0, int ldk = 0, float* dv_sum = nullptr, int acc_mode = 0,
                       float* dh_scale = nullptr) {
  if (!q || !k || !g || !do_ || !dh_work || !dv)
    return tops_set_error(TOPS_ERR_NULL, "gla_chunk_bwd_dh: null tensor");
  // (the sweep tiles V by 64, so a channel slice takes the whole V)
  int rc = check_bwd("gla_chunk_bwd_dh", B, T, H, K, V, N, 0, cu_seqlens, chunk_offsets, nullptr,
                     false, dtype, ldk, 0, ldk > 0);
  if (rc != TOPS_OK) return rc;
  if (acc_mode < 0 || acc_mode > 3 || (acc_mode && !dv_sum))
    return tops_set_error(TOPS_ERR_SHAPE, "gla_chunk_bwd_dh: acc_mode 1..3 needs the fp32 sum buffer");
  SweepParams p{q, k, g, do_, dht, dv, dh0, dh_work, cu_seqlens, chunk_offsets,
                B, T, H, K, V, N, (V + 63) / 64, scale, gate_mode};
  p.ckpt_par = ckpt_par;
  p.ldk = ldk;
  p.acc32 = dv_sum;
  p.acc_mode = acc_mode;
  if (dh_scale) {
    if (dtype != TOPS_BF16 || (gate_mode != kGateK && gate_mode != kGateS && gate_mode != kGateGamma) ||
        V > 128 || ldk || ckpt_par)
      return tops_set_error(TOPS_ERR_SHAPE, "chunk_bwd_dh_c16: bf16, per-channel or per-token gates, V <= 128, no slices");
    p.ckpt16 = 1;
    p.ckpt_scale = dh_scale;
  }
  hipStream_t s = (hipStream_t)stream;
  hipError_t e = dtype == TOPS_BF16 ? launch_gla_sweep<uint16_t, true>(p, s)
                 : dtype == TOPS_F16  ? launch_gla_sweep<_Float16, true>(p, s)
                                      : launch_gla_sweep<float, true>(p, s);
  if (e != hipSuccess) return tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
  return TOPS_OK;
}

static int bwd_dqkg_impl(const void* q, const void* k, const void* v, const float* g,
                         const void* do_, const float* h_ckpt, const float* dh_work, void* dq,
                         void* dk, float* dg, const int32_t* cu_seqlens,
                         const int32_t* chunk_offsets, const int32_t* chunk_map, int total_chunks,
                         int B, int T, int H, int K, int V, int N, int dtype, float scale,
                         int gate_mode, void* stream, const float* h0 = nullptr,
                         const float* dht = nullptr, int paired = 0, int ldk = 0, int ldv = 0,
                         float* dq_sum = nullptr, float* dk_sum = nullptr, int acc_mode = 0,
                         int dg_accum = 0, const float* h_scale = nullptr,
                         const float* dh_scale = nullptr) {
  if (!q || !k || !v || !g || !do_ || !h_ckpt || !dh_work || !dq || !dk ||
      ((gate_mode == kGateK || gate_mode == kGateS) && !dg))
    return tops_set_error(TOPS_ERR_NULL, "gla_chunk_bwd_dqkg: null tensor");
  int rc = check_bwd("gla_chunk_bwd_dqkg", B, T, H, K, V, N, total_chunks, cu_seqlens,
                     chunk_offsets, chunk_map, true, dtype, ldk, ldv);
  if (rc != TOPS_OK) return rc;
  if (acc_mode < 0 || acc_mode > 3 || (acc_mode && (!dq_sum || !dk_sum)))
    return tops_set_error(TOPS_ERR_SHAPE, "gla_chunk_bwd_dqkg: acc_mode 1..3 needs the fp32 sum buffers");
  DqkgParams p{q, k, v, g, do_, h_ckpt, dh_work, dq, dk, dg, cu_seqlens, chunk_offsets, chunk_map,
               total_chunks, B, T, H, K, V, N, scale, gate_mode};
  p.paired = paired;
  p.h0 = h0;
  p.dht = dht;
  p.ldk = ldk;
  p.ldv = ldv;
  p.dq32 = dq_sum;
  p.dk32 = dk_sum;
  p.acc_mode = acc_mode;
  p.dg_accum = dg_accum;
  if (h_scale || dh_scale) {
    if (!h_scale || !dh_scale || dtype != TOPS_BF16 ||
        (gate_mode != kGateK && gate_mode != kGateS && gate_mode != kGateGamma) || paired || ldk || ldv)
      return tops_set_error(TOPS_ERR_SHAPE, "chunk_bwd_dqkg_c16: bf16, per-channel or per-token gates, both scales, unpaired, no slices");
    p.ckpt16 = 1;
    p.hs_scale = h_scale;
    p.dhs_scale = dh_scale;
  }
  hipStream_t s = (hipStream_t)stream;
  hipError_t e = dtype == TOPS_BF16 ? launch_gla_dqkg<uint16_t>(p, s)
                 : dtype == TOPS_F16  ? launch_gla_dqkg<_Float16>(p, s)
                                      : launch_gla_dqkg<float>(p, s);
  if (e != hipSuccess) return tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
  return TOPS_OK;
}

extern "C" int tops_gla_chunk_bwd_dh(const void* q, const void* k, const float* g,
                                     const void* do_, const float* dht, float* dh_work, void* dv,
                                     float* dh0, const int32_t* cu_seqlens,
                                     const int32_t* chunk_offsets, int B, int T, int H, int K,
                                     int V, int N, int dtype, float scale, void* stream) {
  return bwd_dh_impl(q, k, g, do_, dht, dh_work, dv, dh0, cu_seqlens, chunk_offsets, B, T, H, K, V,
                     N, dtype, scale, kGateK, stream);
}

extern "C" int tops_gla_chunk_bwd_dqkg(const void* q, const void* k, const void* v, const float* g,
                                       const void* do_, const float* h_ckpt, const float* dh_work,
                                       void* dq, void* dk, float* dg, const int32_t* cu_seqlens,
                                       const int32_t* chunk_offsets, const int32_t* chunk_map,
                                       int total_chunks, int B, int T, int H, int K, int V, int N,
                                       int dtype, float scale, void* stream) {
  return bwd_dqkg_impl(q, k, v, g, do_, h_ckpt, dh_work, dq, dk, dg, cu_seqlens, chunk_offsets,
                       chunk_map, total_chunks, B, T, H, K, V, N, dtype, scale, kGateK, stream);
}

extern "C" int tops_gla_chunk_bwd(const void* q, const void* k, const void* v, const float* g,
                                  const void* do_, const float* dht, const float* h_ckpt,
                                  float* dh_work, void* dq, void* dk, void* dv, float* dg,
                                  float* dh0, const int32_t* cu_seqlens,
                                  const int32_t* chunk_offsets, const int32_t* chunk_map,
                                  int total_chunks, int B, int T, int H, int K, int V, int N,
                                  int dtype, float scale, void* stream) {
  int rc = bwd_dh_impl(q, k, g, do_, dht, dh_work, dv, dh0, cu_seqlens, chunk_offsets, B, T, H, K,
                       V, N, dtype, scale, kGateK, stream);
  if (rc != TOPS_OK) return rc;
  return bwd_dqkg_impl(q, k, v, g, do_, h_ckpt, dh_work, dq, dk, dg, cu_seqlens, chunk_offsets,
                       chunk_map, total_chunks, B, T, H, K, V, N, dtype, scale, kGateK, stream);
}

extern "C" int tops_simple_gla_chunk_bwd(const void* q, const void* k, const void* v,
                                         const float* g, const float* g_gamma, const void* do_,
                                         const float* dht, const float* h_ckpt, float* dh_work,
                                         void* dq, void* dk, void* dv, float* dg, float* dh0,
                                         const int32_t* cu_seqlens, const int32_t* chunk_offsets,
                                         const int32_t* chunk_map, int total_chunks, int B, int T,
                                         int H, int K, int V, int N, int dtype, float scale,
                                         void* stream) {
  if ((g == nullptr) == (g_gamma == nullptr))
    return tops_set_error(TOPS_ERR_NULL, "simple_gla_chunk_bwd: pass exactly one of g, g_gamma");
  const int mode = g ? kGateS : kGateGamma;
  const float* gp = g ? g : g_gamma;
  int rc = bwd_dh_impl(q, k, gp, do_, dht, dh_work, dv, dh0, cu_seqlens, chunk_offsets, B, T, H, K,
                       V, N, dtype, scale, mode, stream);
  if (rc != TOPS_OK) return rc;
  return bwd_dqkg_impl(q, k, v, gp, do_, h_ckpt, dh_work, dq, dk, g ? dg : nullptr, cu_seqlens,
                       chunk_offsets, chunk_map, total_chunks, B, T, H, K, V, N, dtype, scale, mode,
                       stream);
}

extern "C" int tops_simple_gla_chunk_bwd_dh(const void* q, const void* k, const float* g,
                                            const float* g_gamma, const void* do_,
                                            const float* dht, float* dh_work, void* dv,
                                            float* dh0, const int32_t* cu_seqlens,
                                            const int32_t* chunk_offsets, int B, int T, int H,
                                            int K, int V, int N, int dtype, float scale,
                                            void* stream) {
  if ((g == nullptr) == (g_gamma == nullptr))
    return tops_set_error(TOPS_ERR_NULL, "simple_gla_chunk_bwd_dh: pass exactly one of g, g_gamma");
  return bwd_dh_impl(q, k, g ? g : g_gamma, do_, dht, dh_work, dv, dh0, cu_seqlens, chunk_offsets,
                     B, T, H, K, V, N, dtype, scale, g ? kGateS : kGateGamma, stream);
}

extern "C" int tops_simple_gla_chunk_bwd_dqkg(const void* q, const void* k, const void* v,
                                              const float* g, const float* g_gamma,
                                              const void* do_, const float* h_ckpt,
                                              const float* dh_work, void* dq, void* dk, float* dg,
                                              const int32_t* cu_seqlens,
                                              const int32_t* chunk_offsets,
                                              const int32_t* chunk_map, int total_chunks, int B,
                                              int T, int H, int K, int V, int N, int dtype,
                                              float scale, void* stream) {
  if ((g == nullptr) == (g_gamma == nullptr))
    return tops_set_error(TOPS_ERR_NULL, "simple_gla_chunk_bwd_dqkg: pass exactly one of g, g_gamma");
  return bwd_dqkg_impl(q, k, v, g ? g : g_gamma, do_, h_ckpt, dh_work, dq, dk, g ? dg : nullptr,
                       cu_seqlens, chunk_offsets, chunk_map, total_chunks, B, T, H, K, V, N, dtype,
                       scale, g ? kGateS : kGateGamma, stream);
}

extern "C" int tops_simple_gla_chunk_bwd_dh_c16(const void* q, const void* k, const float* g,
                                                const float* g_gamma, const void* do_,
                                                const float* dht, uint16_t* dh16, float* dh_scale,
                                                void* dv, float* dh0, const int32_t* cu_seqlens,
                                                const int32_t* chunk_offsets, int B, int T, int H,
                                                int K, int V, int N, int dtype, float scale,
                                                void* stream) {
  if ((g == nullptr) == (g_gamma == nullptr))
    return tops_set_error(TOPS_ERR_NULL, "simple_gla_chunk_bwd_dh_c16: pass exactly one of g, g_gamma");
  if (!dh16 || !dh_scale) return tops_set_error(TOPS_ERR_NULL, "simple_gla_chunk_bwd_dh_c16: null checkpoint");
  return bwd_dh_impl(q, k, g ? g : g_gamma, do_, dht, (float*)dh16, dv, dh0, cu_seqlens, chunk_offsets,
                     B, T, H, K, V, N, dtype, scale, g ? kGateS : kGateGamma, stream, 0, 0, nullptr, 0,
                     dh_scale);
}

extern "C" int tops_simple_gla_chunk_bwd_dqkg_c16(const void* q, const void* k, const void* v,
                                                  const float* g, const float* g_gamma,
                                                  const void* do_, const uint16_t* h16,
                                                  const float* h_scale, const uint16_t* dh16,
                                                  const float* dh_scale, void* dq, void* dk,
                                                  float* dg, const int32_t* cu_seqlens,
                                                  const int32_t* chunk_offsets,
                                                  const int32_t* chunk_map, int total_chunks,
                                                  int B, int T, int H, int K, int V, int N,
                                                  int dtype, float scale, void* stream) {
  if ((g == nullptr) == (g_gamma == nullptr))
    return tops_set_error(TOPS_ERR_NULL, "simple_gla_chunk_bwd_dqkg_c16: pass exactly one of g, g_gamma");
  if (!h16 || !dh16 || !h_scale || !dh_scale)
    return tops_set_error(TOPS_ERR_NULL, "simple_gla_chunk_bwd_dqkg_c16: null checkpoint");
  return bwd_dqkg_impl(q, k, v, g ? g : g_gamma, do_, (const float*)h16, (const float*)dh16, dq, dk,
                       g ? dg : nullptr, cu_seqlens, chunk_offsets, chunk_map, total_chunks, B, T, H,
                       K, V, N, dtype, scale, g ? kGateS : kGateGamma, stream, nullptr, nullptr, 0,
                       0, 0, nullptr, nullptr, 0, 0, h_scale, dh_scale);
}

extern "C" int tops_gla_chunk_bwd_dh_gamma(const void* q, const void* k, const float* g_gamma,
                                           const void* do_, const float* dht, float* dh_work,
                                           void* dv, float* dh0, const int32_t* cu_seqlens,
                                           const int32_t* chunk_offsets, int B, int T, int H,
                                           int K, int V, int N, int dtype, float scale,
                                           void* stream) {
  return bwd_dh_impl(q, k, g_gamma, do_, dht, dh_work, dv, dh0, cu_seqlens, chunk_offsets, B, T, H,
                     K, V, N, dtype, scale, kGateGammaK, stream);
}

extern "C" int tops_gla_chunk_bwd_dqkg_gamma(const void* q, const void* k, const void* v,
                                             const float* g_gamma, const void* do_,
                                             const float* h_ckpt, const float* dh_work, void* dq,
                                             void* dk, float* dg, const int32_t* cu_seqlens,
                                             const int32_t* chunk_offsets,
                                             const int32_t* chunk_map, int total_chunks, int B,
                                             int T, int H, int K, int V, int N, int dtype,
                                             float scale, void* stream) {
  return bwd_dqkg_impl(q, k, v, g_gamma, do_, h_ckpt, dh_work, dq, dk, dg, cu_seqlens,
                       chunk_offsets, chunk_map, total_chunks, B, T, H, K, V, N, dtype, scale,
                       kGateGammaK, stream);
}

// fp16 checkpoints (bf16 inputs, per-channel gates): the same three stages with h and dh
// stored as fp16 [total,H,K,V] plus one power-of-two factor per (chunk, head, 64-column tile).
extern "C" int tops_gla_chunk_bwd_dh_c16(const void* q, const void* k, const float* g,
                                         const void* do_, const float* dht, uint16_t* dh16,
                                         float* dh_scale, void* dv, float* dh0,
                                         const int32_t* cu_seqlens, const int32_t* chunk_offsets,
                                         int B, int T, int H, int K, int V, int N, int dtype,
                                         float scale, void* stream) {
  if (!dh16 || !dh_scale) return tops_set_error(TOPS_ERR_NULL, "gla_chunk_bwd_dh_c16: null checkpoint");
  return bwd_dh_impl(q, k, g, do_, dht, (float*)dh16, dv, dh0, cu_seqlens, chunk_offsets, B, T, H,
                     K, V, N, dtype, scale, kGateK, stream, 0, 0, nullptr, 0, dh_scale);
}

extern "C" int tops_gla_chunk_bwd_dqkg_c16(const void* q, const void* k, const void* v,
                                           const float* g, const void* do_, const uint16_t* h16,
                                           const float* h_scale, const uint16_t* dh16,
                                           const float* dh_scale, void* dq, void* dk, float* dg,
                                           const int32_t* cu_seqlens, const int32_t* chunk_offsets,
                                           const int32_t* chunk_map, int total_chunks, int B,
                                           int T, int H, int K, int V, int N, int dtype,
                                           float scale, void* stream) {
  if (!h16 || !dh16 || !h_scale || !dh_scale)
    return tops_set_error(TOPS_ERR_NULL, "gla_chunk_bwd_dqkg_c16: null checkpoint");
  return bwd_dqkg_impl(q, k, v, g, do_, (const float*)h16, (const float*)dh16, dq, dk, dg,
                       cu_seqlens, chunk_offsets, chunk_map, total_chunks, B, T, H, K, V, N, dtype,
                       scale, kGateK, stream, nullptr, nullptr, 0, 0, 0, nullptr, nullptr, 0, 0,
                       h_scale, dh_scale);
}

// Channel / value slices of heads wider than one kernel tile (the caller loops over them).
static int check_slice_gate(const char* who, int gate_mode) {
  if (gate_mode < kGateK || gate_mode > kGateGammaK) {
    char msg[160];
    snprintf(msg, sizeof(msg), "%s: gate_mode must be 0..3", who);
    return tops_set_error(TOPS_ERR_SHAPE, msg);
  }
  return TOPS_OK;
}

extern "C" int tops_chunk_bwd_dh_slice(const void* q, const void* k, const float* g,
                                       int gate_mode, const void* do_, const float* dht,
                                       float* dh_work, void* dv, float* dv_sum, int acc_mode,
                                       float* dh0, const int32_t* cu_seqlens,
                                       const int32_t* chunk_offsets, int B, int T, int H, int K,
                                       int V, int N, int ldk, int dtype, float scale,
                                       void* stream) {
  int rc = check_slice_gate("chunk_bwd_dh_slice", gate_mode);
  if (rc != TOPS_OK) return rc;
  if (acc_mode != 1 && acc_mode != 2 && !dv)
    return tops_set_error(TOPS_ERR_NULL, "chunk_bwd_dh_slice: null dv");
  return bwd_dh_impl(q, k, g, do_, dht, dh_work, dv ? dv : (void*)dv_sum, dh0, cu_seqlens,
                     chunk_offsets, B, T, H, K, V, N, dtype, scale, gate_mode, stream, 0,
                     ldk > 0 ? ldk : K, dv_sum, acc_mode);
}

extern "C" int tops_chunk_bwd_dqkg_slice(const void* q, const void* k, const void* v,
                                         const float* g, int gate_mode, const void* do_,
                                         const float* h_ckpt, const float* dh_work, void* dq,
                                         void* dk, float* dg, float* dq_sum, float* dk_sum,
                                         int acc_mode, int dg_accum, const int32_t* cu_seqlens,
                                         const int32_t* chunk_offsets, const int32_t* chunk_map,
                                         int total_chunks, int B, int T, int H, int K, int V,
                                         int N, int ldk, int ldv, int dtype, float scale,
                                         void* stream) {
  int rc = check_slice_gate("chunk_bwd_dqkg_slice", gate_mode);
  if (rc != TOPS_OK) return rc;
  if (gate_mode == kGateGamma) dg = nullptr;
  // dq / dk are written only by acc_mode 0 and 3
  if (acc_mode == 1 || acc_mode == 2) {
    if (!dq) dq = dq_sum;
    if (!dk) dk = dk_sum;
  }
  return bwd_dqkg_impl(q, k, v, g, do_, h_ckpt, dh_work, dq, dk, dg, cu_seqlens, chunk_offsets,
                       chunk_map, total_chunks, B, T, H, K, V, N, dtype, scale, gate_mode, stream,
                       nullptr, nullptr, 0, ldk > 0 ? ldk : K, ldv > 0 ? ldv : V, dq_sum, dk_sum,
                       acc_mode, dg_accum);
}

// Interleaved checkpoints: one [total_chunks, H, K, V] buffer, h before the even global
// chunks (tops_chunk_fwd_paired), dh after the odd ones (stage 1 below); stage 2 rebuilds the
// other state of every chunk from its pair partner.
static int check_paired(const char* who, int gate_mode, int dtype) {
  char msg[160];
  if (gate_mode < kGateK || gate_mode > kGateGammaK) {
    snprintf(msg, sizeof(msg), "%s: gate_mode must be 0..3", who);
    return tops_set_error(TOPS_ERR_SHAPE, msg);
  }
  if (dtype != TOPS_BF16) {
    snprintf(msg, sizeof(msg), "%s: the interleaved layout takes TOPS_BF16", who);
    return tops_set_error(TOPS_ERR_DTYPE, msg);
  }
  return TOPS_OK;
}

extern "C" int tops_chunk_bwd_dh_paired(const void* q, const void* k, const float* g,
                                        int gate_mode, const void* do_, const float* dht,
                                        float* ckpt, void* dv, float* dh0,
                                        const int32_t* cu_seqlens, const int32_t* chunk_offsets,
                                        int B, int T, int H, int K, int V, int N, int dtype,
                                        float scale, void* stream) {
  int rc = check_paired("chunk_bwd_dh_paired", gate_mode, dtype);
  if (rc != TOPS_OK) return rc;
  return bwd_dh_impl(q, k, g, do_, dht, ckpt, dv, dh0, cu_seqlens, chunk_offsets, B, T, H, K, V, N,
                     dtype, scale, gate_mode, stream, 2);
}

extern "C" int tops_chunk_bwd_dqkg_paired(const void* q, const void* k, const void* v,
                                          const float* g, int gate_mode, const void* do_,
                                          const float* h0, const float* dht, const float* ckpt,
                                          void* dq, void* dk, float* dg,
                                          const int32_t* cu_seqlens, const int32_t* chunk_offsets,
                                          const int32_t* chunk_map, int total_chunks, int B,
                                          int T, int H, int K, int V, int N, int dtype,
                                          float scale, void* stream) {
  int rc = check_paired("chunk_bwd_dqkg_paired", gate_mode, dtype);
  if (rc != TOPS_OK) return rc;
  if (gate_mode == kGateGamma) dg = nullptr;
  return bwd_dqkg_impl(q, k, v, g, do_, ckpt, ckpt, dq, dk, dg, cu_seqlens, chunk_offsets,
                       chunk_map, total_chunks, B, T, H, K, V, N, dtype, scale, gate_mode, stream,
                       h0, dht, 1);
}
