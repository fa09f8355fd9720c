// C-ABI entry points of the chunked KDA (include/tops_hip.h).
//
// Forward (tops_kda_chunk_fwd): the chunk-parallel WY preparation (kda_prep.hip: gate
// cumsum, Akk, T = (I + Akk)^-1, u, w) and the delta-rule state sweep (the DELTA instance of
// gla_sweep.hip: v_new = u - w S, o, S per chunk), replacing chunk_kda_fwd's four stages
// (tops/ops/kda/chunk.py:25-190).
//
// Backward (tops_kda_chunk_bwd): the reverse delta-rule sweep (dv_new, dS per chunk,
// dh0), then for bf16 inputs one kernel for the WY backward and the GLA-shaped dq / dk /
// dg (kda_bwd_fused.hip); for fp32 inputs the WY backward (kda_wy.hip: dv, dbeta and the WY
// parts of dk, dg) followed by the dq / dk / dg kernel (gla_dqkg.hip with v := v_new) which
// adds them, replacing chunk_kda_bwd (tops/ops/kda/chunk_bwd.py:655-832).
#include <stdio.h>

#include <mutex>

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

static int kda_fwd_impl(const void* q, const void* k, const void* v, const float* g,
                        const float* beta, const float* h0, void* o, float* ht, float* u,
                        float* w, float* tt, float* v_new, float* h_ckpt, float* h_scale,
                        const int32_t* cu_seqlens, const int32_t* chunk_offsets,
                        const int32_t* chunk_map, int total_chunks, int B, int T, int H,
                        int K, int V, int N, int dtype, float scale, void* stream) {
  if (!q || !k || !v || !g || !beta || !o || !u || !w)
    return tops_set_error(TOPS_ERR_NULL, "kda_chunk_fwd: null tensor");
  int rc = kda_check("kda_chunk_fwd", B, T, H, K, V, N, total_chunks, cu_seqlens, chunk_offsets,
                     chunk_map, dtype);
  if (rc != TOPS_OK) return rc;
  if (h_scale && (dtype != TOPS_BF16 || !h_ckpt))
    return tops_set_error(TOPS_ERR_SHAPE, "kda_chunk_fwd_c16: bf16 inputs and a checkpoint buffer");
  hipStream_t s = (hipStream_t)stream;
  KdaPrepParams pp{k, v, g, beta, u, w, tt, cu_seqlens, chunk_offsets, chunk_map,
                   total_chunks, B, T, H, K, V, N};
  hipError_t e = dtype == TOPS_BF16 ? launch_kda_prep<uint16_t>(pp, s) : launch_kda_prep<float>(pp, s);
  if (e != hipSuccess) return tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
  SweepParams sp{q, k, g, nullptr, h0, o, ht, h_ckpt, cu_seqlens, chunk_offsets,
                 B, T, H, K, V, N, (V + 63) / 64, scale, kGateK, u, w, v_new};
  if (h_scale) {
    sp.ckpt16 = 1;
    sp.ckpt_scale = h_scale;
  }
  e = dtype == TOPS_BF16 ? launch_gla_sweep<uint16_t, false, true>(sp, s)
                         : launch_gla_sweep<float, false, true>(sp, s);
  if (e != hipSuccess) return tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
  return TOPS_OK;
}

extern "C" int tops_kda_chunk_fwd(const void* q, const void* k, const void* v, const float* g,
                                  const float* beta, const float* h0, void* o, float* ht, float* u,
                                  float* w, float* tt, float* v_new, float* h_ckpt,
                                  const int32_t* cu_seqlens, const int32_t* chunk_offsets,
                                  const int32_t* chunk_map, int total_chunks, int B, int T, int H,
                                  int K, int V, int N, int dtype, float scale, void* stream) {
  return kda_fwd_impl(q, k, v, g, beta, h0, o, ht, u, w, tt, v_new, h_ckpt, nullptr, cu_seqlens,
                      chunk_offsets, chunk_map, total_chunks, B, T, H, K, V, N, dtype, scale, stream);
}

extern "C" int tops_kda_chunk_fwd_c16(const void* q, const void* k, const void* v, const float* g,
                                      const float* beta, const float* h0, void* o, float* ht,
                                      float* u, float* w, float* tt, float* v_new,
                                      uint16_t* h_ckpt16, float* h_scale,
                                      const int32_t* cu_seqlens, const int32_t* chunk_offsets,
                                      const int32_t* chunk_map, int total_chunks, int B, int T,
                                      int H, int K, int V, int N, int dtype, float scale,
                                      void* stream) {
  if (!h_ckpt16 || !h_scale) return tops_set_error(TOPS_ERR_NULL, "kda_chunk_fwd_c16: null checkpoint");
  return kda_fwd_impl(q, k, v, g, beta, h0, o, ht, u, w, tt, v_new, (float*)h_ckpt16, h_scale,
                      cu_seqlens, chunk_offsets, chunk_map, total_chunks, B, T, H, K, V, N, dtype,
                      scale, stream);
}

static int kda_bwd_impl(const void* q, const void* k, const void* v, const float* g,
                        const float* beta, const float* w, const float* tt, const float* v_new,
                        const float* h_ckpt, const float* h_scale, const void* do_,
                        const float* dht, float* dh_work, float* dh_scale, float* dvn_work,
                        float* dk_work, float* dg_work, void* dq, void* dk, void* dv,
                        float* dbeta, float* dg, float* dh0, const int32_t* cu_seqlens,
                        const int32_t* chunk_offsets, const int32_t* chunk_map,
                        int total_chunks, int B, int T, int H, int K, int V, int N,
                        int dtype, float scale, void* stream) {
  if (!q || !k || !v || !g || !beta || !w || !tt || !v_new || !h_ckpt || !do_ || !dh_work ||
      !dvn_work || !dq || !dk || !dv || !dbeta || !dg)
    return tops_set_error(TOPS_ERR_NULL, "kda_chunk_bwd: null tensor");
  // bf16: the WY stage and dq / dk / dg run as one kernel and need no dk / dg workspace
  if (dtype != TOPS_BF16 && (!dk_work || !dg_work))
    return tops_set_error(TOPS_ERR_NULL, "kda_chunk_bwd: fp32 inputs need dk_work and dg_work");
  int rc = kda_check("kda_chunk_bwd", B, T, H, K, V, N, total_chunks, cu_seqlens, chunk_offsets,
                     chunk_map, dtype);
  if (rc != TOPS_OK) return rc;
  if ((h_scale || dh_scale) && (!h_scale || !dh_scale || dtype != TOPS_BF16))
    return tops_set_error(TOPS_ERR_SHAPE, "kda_chunk_bwd_c16: bf16 inputs, both checkpoint factor arrays");
  hipStream_t s = (hipStream_t)stream;
  const bool bf = dtype == TOPS_BF16;
  // 1. reverse delta-rule sweep: dv_new (transposed per chunk), dS per chunk, dh0
  SweepParams sp{q, k, g, do_, dht, nullptr, dh0, dh_work, cu_seqlens, chunk_offsets,
                 B, T, H, K, V, N, (V + 63) / 64, scale, kGateK, nullptr, w, dvn_work};
  if (dh_scale) {
    sp.ckpt16 = 1;
    sp.ckpt_scale = dh_scale;
  }
  hipError_t e = bf ? launch_gla_sweep<uint16_t, true, true>(sp, s) : launch_gla_sweep<float, true, true>(sp, s);
  if (e != hipSuccess) return tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
  if (bf) {
    // 2+3. the WY backward and dq, dk, dg in one kernel (the WY parts through LDS)
    KdaBwdParams fp{q, k, v, g, beta, tt, dvn_work, v_new, h_ckpt, dh_work, do_, dq, dk, dv, dbeta, dg,
                    cu_seqlens, chunk_offsets, chunk_map, total_chunks, B, T, H, K, V, N, scale};
    if (h_scale) {
      fp.ckpt16 = 1;
      fp.hs_scale = h_scale;
      fp.dhs_scale = dh_scale;
    }
    e = launch_kda_bwd_fused(fp, s);
    if (e != hipSuccess) return tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
    return TOPS_OK;
  }
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

extern "C" int tops_kda_chunk_bwd(const void* q, const void* k, const void* v, const float* g,
                                  const float* beta, const float* w, const float* tt,
                                  const float* v_new, const float* h_ckpt, const void* do_,
                                  const float* dht, float* dh_work, float* dvn_work, float* dk_work,
                                  float* dg_work, void* dq, void* dk, void* dv, float* dbeta,
                                  float* dg, float* dh0, const int32_t* cu_seqlens,
                                  const int32_t* chunk_offsets, const int32_t* chunk_map,
                                  int total_chunks, int B, int T, int H, int K, int V, int N,
                                  int dtype, float scale, void* stream) {
  return kda_bwd_impl(q, k, v, g, beta, w, tt, v_new, h_ckpt, nullptr, do_, dht, dh_work, nullptr,
                      dvn_work, dk_work, dg_work, dq, dk, dv, dbeta, dg, dh0, cu_seqlens,
                      chunk_offsets, chunk_map, total_chunks, B, T, H, K, V, N, dtype, scale,
                      stream);
}

extern "C" int tops_kda_chunk_bwd_c16(const void* q, const void* k, const void* v, const float* g,
                                      const float* beta, const float* w, const float* tt,
                                      const float* v_new, const uint16_t* h_ckpt16,
                                      const float* h_scale, const void* do_, const float* dht,
                                      uint16_t* dh16_work, float* dh_scale, float* dvn_work,
                                      void* dq, void* dk, void* dv, float* dbeta, float* dg,
                                      float* dh0, const int32_t* cu_seqlens,
                                      const int32_t* chunk_offsets, const int32_t* chunk_map,
                                      int total_chunks, int B, int T, int H, int K, int V, int N,
                                      int dtype, float scale, void* stream) {
  if (!h_ckpt16 || !h_scale || !dh16_work || !dh_scale)
    return tops_set_error(TOPS_ERR_NULL, "kda_chunk_bwd_c16: null checkpoint");
  return kda_bwd_impl(q, k, v, g, beta, w, tt, v_new, (const float*)h_ckpt16, h_scale, do_, dht,
                      (float*)dh16_work, dh_scale, dvn_work, nullptr, nullptr, dq, dk, dv, dbeta,
                      dg, dh0, cu_seqlens, chunk_offsets, chunk_map, total_chunks, B, T, H, K, V,
                      N, dtype, scale, stream);
}

// ---------------------------------------------------------------------------------------
// Allocation-free KDA forward (inference): the WY workspace u [B,T,H,V] and w [B,T,H,K]
// lives in a static device array of kKdaScratchBytes, one copy per GPU, held until the
// process ends.  Its address is taken with hipGetSymbolAddress once per device, with that
// device current, on the first call there; host code never passes the array's name itself
// to a kernel (on the host it is only a stand-in for the symbol).  Nothing in the array has
// to start at zero: kda_prep writes every u / w element that the sweep later reads.  Calls
// that overlap on one GPU share the array and race.
namespace {
constexpr size_t kKdaScratchBytes = size_t(64) << 20;  // 64 MiB: T*H*(K+V) <= 16M floats
constexpr int kMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[kKdaScratchBytes];
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return tops_set_error(TOPS_ERR_SHAPE, "kda_chunk_fwd_noalloc: device index out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return tops_set_error(TOPS_ERR_LAUNCH, e != hipSuccess ? hipGetErrorString(e)
                                                            : "kda_chunk_fwd_noalloc: null scratch");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return TOPS_OK;
}
}  // namespace

extern "C" int64_t tops_kda_chunk_fwd_noalloc_max_bytes(void) { return (int64_t)kKdaScratchBytes; }

extern "C" int tops_kda_chunk_fwd_noalloc(const void* q, const void* k, const void* v,
                                          const float* g, const float* beta, const float* h0,
                                          void* o, float* ht, const int32_t* cu_seqlens,
                                          const int32_t* chunk_offsets, const int32_t* chunk_map,
                                          int total_chunks, int B, int T, int H, int K, int V,
                                          int N, int dtype, float scale, void* stream) {
  if (B <= 0 || T <= 0 || H <= 0 || K <= 0 || V <= 0)
    return tops_set_error(TOPS_ERR_SHAPE, "kda_chunk_fwd_noalloc: non-positive dimension");
  const long long rows = (long long)B * T * H;
  const long long u_bytes = (rows * V * 4 + 255) / 256 * 256;
  const long long need = u_bytes + rows * K * 4;
  if (need > (long long)kKdaScratchBytes) {
    char msg[200];
    snprintf(msg, sizeof(msg),
             "kda_chunk_fwd_noalloc: B*T*H*(K+V)*4 = %lld bytes of workspace exceed the %lld-byte "
             "static scratch (use tops_kda_chunk_fwd with a caller workspace)",
             need, (long long)kKdaScratchBytes);
    return tops_set_error(TOPS_ERR_SHAPE, msg);
  }
  void* base = nullptr;
  int rc = scratch_address(&base);
  if (rc != TOPS_OK) return rc;
  float* u = (float*)base;
  float* w = (float*)((unsigned char*)base + u_bytes);
  return tops_kda_chunk_fwd(q, k, v, g, beta, h0, o, ht, u, w, nullptr, nullptr, nullptr,
                            cu_seqlens, chunk_offsets, chunk_map, total_chunks, B, T, H, K, V, N,
                            dtype, scale, stream);
}
