// Separately callable stages of the chunked KDA forward, for gfx950: the intra-chunk solve
// (tops/ops/kda/chunk_intra.py:91-281, kda_intra_chunk_fwd) and the delta-rule state pass
// (tops/ops/common/chunk_delta_h.py:44-166, 898-993, chunk_gated_delta_rule_fwd_h; the
// oracle tops/cpu/ops/common/chunk_delta_h.py:22-118).  The fused KDA path (kda_prep.hip,
// the DELTA sweeps of gla_sweep.hip) computes the same quantities without writing them in
// these layouts; these kernels serve callers that drive the stages themselves.
//
// Arithmetic is fp32 FMA throughout (the reference's fp32 accumulation), one workgroup of
// 4 wave64 per (batch, head, chunk) for the intra solve and per (sequence, head, 64-column
// V slice) for the state pass.
#include <math.h>
#include <stdio.h>

#include "tops_common.h"
#include "tops_hip.h"

namespace tops {
namespace {

constexpr int kNth = 256;

template <typename T> __device__ __forceinline__ float ld1(const T* p, long long i) {
  return In<T>::ld(p + i);
}
template <typename T> __device__ __forceinline__ void st1(T* p, long long i, float x) {
  In<T>::st(p + i, x);
}

// ------------------------------------------------------------------ intra-chunk solve
// Per chunk of C tokens of one (batch, head), with G the given chunk-local gate cumsum
// (log2 units) and s the segment ids:
//   Aqk[i][j] = scale sum_d q_id k_jd 2^(G_id - G_jd)          (j <= i, s_i == s_j)
//   Akk[i][j] = beta_i sum_d k_id k_jd 2^(G_id - G_jd)         (j <  i, s_i == s_j)
//   [u | w | Akk_inv] = (I + Akk)^-1 [beta v | beta k 2^G | I]  (forward substitution)
//   qg = q 2^G,  kg = k 2^(G_last - G)
// The exponent is taken per (i, j, d) only where j <= i, so it never exceeds 0 for
// non-increasing gates (the reference masks the same entries before its exp2).
struct IntraFwdArgs {
  const void* q;
  const void* k;
  const float* g;
  const float* beta;
  const void* v;
  const int32_t* seg;   // [B, T] or NULL (one segment)
  void* u;
  void* w;
  void* qg;
  void* kg;
  void* Aqk;
  void* Akk_inv;
  int H, T, K, V;
  float scale;
};

template <typename TIn, int C>
__global__ __launch_bounds__(kNth) void kda_intra_fwd_kernel(IntraFwdArgs a) {
  constexpr int DT = 32;              // channels per LDS tile
  constexpr int LT = DT + 1;
  constexpr int TPR = kNth / C;       // threads per row of A
  constexpr int EPT = C / TPR;        // A entries per thread
  constexpr int CB = C <= 64 ? 256 : 128;   // columns per substitution pass
  static_assert(kNth % C == 0 && C % TPR == 0, "C must be 16, 32, 64 or 128");
  // one buffer: the q / k / gate tiles of the A phase, then the columns being solved
  constexpr int NBUF = (3 * C * LT > C * CB) ? 3 * C * LT : C * CB;
  __shared__ float buf[NBUF];
  __shared__ float sA[C][C + 1];
  __shared__ float sb[C];
  __shared__ int ss[C];
  float* const sq = buf;
  float* const sk = buf + C * LT;
  float* const sg = buf + 2 * C * LT;

  const TIn* q = (const TIn*)a.q;
  const TIn* k = (const TIn*)a.k;
  const TIn* v = (const TIn*)a.v;
  const int K = a.K, V = a.V;
  const int NC = a.T / C;
  const int bh = blockIdx.x / NC, ci = blockIdx.x - bh * NC;
  const int b = bh / a.H;
  const long long row0 = (long long)bh * a.T + (long long)ci * C;   // row of [B*H*T, .]
  const int tid = threadIdx.x;
  if (tid < C) {
    sb[tid] = a.beta[row0 + tid];
    ss[tid] = a.seg ? a.seg[(long long)b * a.T + (long long)ci * C + tid] : 0;
  }

  // ---- A entries: thread owns row i, columns j0 + TPR m
  const int i = tid / TPR, j0 = tid - i * TPR;
  float aq[EPT], ak[EPT];
#pragma unroll
  for (int m = 0; m < EPT; ++m) aq[m] = ak[m] = 0.f;
  for (int d0 = 0; d0 < K; d0 += DT) {
    __syncthreads();   // the previous tile is consumed
    for (int e = tid; e < C * DT; e += kNth) {
      const int r = e / DT, c = e - r * DT, d = d0 + c;
      const bool ok = d < K;
      const long long off = (row0 + r) * K + d;
      sq[r * LT + c] = ok ? ld1(q, off) : 0.f;
      sk[r * LT + c] = ok ? ld1(k, off) : 0.f;
      sg[r * LT + c] = ok ? a.g[off] : 0.f;
    }
    __syncthreads();
#pragma unroll 2
    for (int c = 0; c < DT; ++c) {
      const float qi = sq[i * LT + c], ki = sk[i * LT + c], gi = sg[i * LT + c];
#pragma unroll
      for (int m = 0; m < EPT; ++m) {
        const int j = j0 + TPR * m;
        if (j <= i) {
          const float kj = sk[j * LT + c] * fast_exp2(gi - sg[j * LT + c]);
          aq[m] = fmaf(qi, kj, aq[m]);
          ak[m] = fmaf(ki, kj, ak[m]);
        }
      }
    }
  }
  TIn* Aqk = (TIn*)a.Aqk;
  const long long abase = (long long)blockIdx.x * C * C;   // [B, H, NC, C, C]
#pragma unroll
  for (int m = 0; m < EPT; ++m) {
    const int j = j0 + TPR * m;
    const bool same = ss[i] == ss[j];
    st1(Aqk, abase + (long long)i * C + j, (j <= i && same) ? aq[m] * a.scale : 0.f);
    sA[i][j] = (j < i && same) ? ak[m] * sb[i] : 0.f;
  }

  // ---- forward substitution over [beta v | beta k 2^G | I], CB columns at a time, one
  // column per thread, solved in place in LDS (x[r] = b[r] - sum_{j<r} Akk[r][j] x[j])
  TIn* U = (TIn*)a.u;
  TIn* W = (TIn*)a.w;
  TIn* Ainv = (TIn*)a.Akk_inv;
  float* const x = buf;                 // [C][CB]
  const int ncol = V + K + C;
  for (int col0 = 0; col0 < ncol; col0 += CB) {
    __syncthreads();   // sA visible; the tiles (or the previous columns) are consumed
    const int col = col0 + tid;
    const bool own = tid < CB && col < ncol;
    if (own) {
      for (int r = 0; r < C; ++r) {
        float bv;
        if (col < V) {
          bv = sb[r] * ld1(v, (row0 + r) * V + col);
        } else if (col < V + K) {
          const long long off = (row0 + r) * K + (col - V);
          bv = sb[r] * ld1(k, off) * fast_exp2(a.g[off]);
        } else {
          bv = (r == col - V - K) ? 1.f : 0.f;
        }
        float acc = bv;
        for (int jj = 0; jj < r; ++jj) acc = fmaf(-sA[r][jj], x[jj * CB + tid], acc);
        x[r * CB + tid] = acc;
        if (col < V) st1(U, (row0 + r) * V + col, acc);
        else if (col < V + K) st1(W, (row0 + r) * K + (col - V), acc);
        else st1(Ainv, abase + (long long)r * C + (col - V - K), acc);
      }
    }
  }

  // ---- gated q and k
  TIn* QG = (TIn*)a.qg;
  TIn* KG = (TIn*)a.kg;
  for (int e = tid; e < C * K; e += kNth) {
    const int r = e / K, d = e - r * K;
    const long long off = (row0 + r) * K + d;
    const float gr = a.g[off];
    const float gl = a.g[(row0 + C - 1) * K + d];
    st1(QG, off, ld1(q, off) * fast_exp2(gr));
    st1(KG, off, ld1(k, off) * fast_exp2(gl - gr));
  }
}

// ------------------------------------------------------------------ delta-rule state pass
// Per (sequence, head, 64-column V slice), chunk by chunk (S = the state before the chunk):
//   h[chunk] = S;  v_new = u - w S;  S = S 2^(g_last + gk_last) + k^T (v_new 2^(g_last - g))
// with k already gated by the caller, g the scalar and gk the per-channel chunk-local gate
// cumsums (log2 units; either may be absent), "last" the chunk's last token.  The state
// slice lives in LDS; w and k rows of the chunk are staged as fp32.
struct DeltaHArgs {
  const void* k;
  const void* w;
  const void* u;
  const float* g;        // [B, T, H] or NULL
  const float* gk;       // [B, T, H, K] or NULL
  const float* h0;       // [N, H, K, V] or NULL
  void* h;               // [total, H, K, V] (TIn) or NULL
  float* v_new;          // [B, T, H, V] or NULL
  float* ht;             // [N, H, K, V] or NULL
  const int32_t* cu;     // [N + 1] or NULL
  const int32_t* offs;   // [N] first global chunk of each sequence (varlen)
  int T, H, K, V, C;
};

constexpr int kDK = 128, kDC = 64, kDV = 64;

template <typename TIn>
__global__ __launch_bounds__(kNth) void delta_h_kernel(DeltaHArgs a) {
  __shared__ float sS[kDK][kDV + 4];
  __shared__ float sW[kDC][kDK + 4];
  __shared__ float sK[kDC][kDK + 4];
  __shared__ float sV[kDC][kDV + 4];
  __shared__ float sd[kDK];
  const TIn* kp = (const TIn*)a.k;
  const TIn* wp = (const TIn*)a.w;
  const TIn* up = (const TIn*)a.u;
  TIn* hp = (TIn*)a.h;
  const int H = a.H, K = a.K, V = a.V, C = a.C;
  const int n = blockIdx.x / H, hh = blockIdx.x - n * H;
  const int v0 = blockIdx.y * kDV, vw = min(kDV, V - v0);
  long long bos;
  int len, cbase;
  if (a.cu) {
    bos = a.cu[n];
    len = a.cu[n + 1] - a.cu[n];
    cbase = a.offs[n];
  } else {
    bos = (long long)n * a.T;
    len = a.T;
    cbase = n * (a.T / C);
  }
  const int nch = (len + C - 1) / C;
  const int tid = threadIdx.x, j = tid & 63, rg = tid >> 6;
  const bool jok = j < vw;
  const long long sb0 = ((long long)n * H + hh) * K;
  for (int kk = rg; kk < K; kk += 4)
    sS[kk][j] = (a.h0 && jok) ? a.h0[(sb0 + kk) * V + v0 + j] : 0.f;

  for (int c = 0; c < nch; ++c) {
    const long long t0 = bos + (long long)c * C;
    const int nv = min(C, len - c * C);
    const long long tl = t0 + nv - 1;                       // last token of the chunk
    __syncthreads();   // S complete; the previous chunk's rows consumed
    if (hp && jok) {
      const long long hb = ((long long)(cbase + c) * H + hh) * K;
      for (int kk = rg; kk < K; kk += 4) st1(hp, (hb + kk) * V + v0 + j, sS[kk][j]);
    }
    for (int e = tid; e < C * K; e += kNth) {
      const int r = e / K, d = e - r * K;
      const bool ok = r < nv;
      const long long off = ((t0 + r) * H + hh) * K + d;
      sW[r][d] = ok ? ld1(wp, off) : 0.f;
      sK[r][d] = ok ? ld1(kp, off) : 0.f;
    }
    const float glast = a.g ? a.g[tl * H + hh] : 0.f;
    for (int d = tid; d < K; d += kNth)
      sd[d] = fast_exp2(glast + (a.gk ? a.gk[(tl * H + hh) * K + d] : 0.f));
    __syncthreads();
    for (int r = rg; r < C; r += 4) {
      float acc = 0.f;
      for (int kk = 0; kk < K; ++kk) acc = fmaf(sW[r][kk], sS[kk][j], acc);
      float vn = 0.f;
      if (r < nv && jok) {
        const long long vo = ((t0 + r) * H + hh) * V + v0 + j;
        vn = ld1(up, vo) - acc;
        if (a.v_new) a.v_new[vo] = vn;
        if (a.g) vn *= fast_exp2(glast - a.g[(t0 + r) * H + hh]);
      }
      sV[r][j] = vn;
    }
    __syncthreads();
    for (int kk = rg; kk < K; kk += 4) {
      float acc = sS[kk][j] * sd[kk];
      for (int r = 0; r < nv; ++r) acc = fmaf(sK[r][kk], sV[r][j], acc);
      sS[kk][j] = acc;
    }
  }
  __syncthreads();
  if (a.ht && jok)
    for (int kk = rg; kk < K; kk += 4) a.ht[(sb0 + kk) * V + v0 + j] = sS[kk][j];
}

int launch_status() {
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? TOPS_OK : tops_set_error(TOPS_ERR_LAUNCH, hipGetErrorString(err));
}

}  // namespace
}  // namespace tops

using namespace tops;

extern "C" int tops_kda_stage_intra_fwd(const void* q, const void* k, const float* g,
                                        const float* beta, const void* v,
                                        const int32_t* segment_ids, int dtype, void* u, void* w,
                                        void* qg, void* kg, void* Aqk, void* Akk_inv, int B,
                                        int H, int T, int K, int V, int chunk_size, float scale,
                                        void* stream) {
  if (!q || !k || !g || !beta || !v || !u || !w || !qg || !kg || !Aqk || !Akk_inv)
    return tops_set_error(TOPS_ERR_NULL, "kda_stage_intra_fwd: null tensor");
  const int C = chunk_size;
  if (C != 16 && C != 32 && C != 64 && C != 128)
    return tops_set_error(TOPS_ERR_UNSUPPORTED, "kda_stage_intra_fwd: chunk_size must be 16, 32, 64 or 128");
  if (B <= 0 || H <= 0 || T < 0 || K <= 0 || V <= 0 || T % C)
    return tops_set_error(TOPS_ERR_SHAPE, "kda_stage_intra_fwd: need B, H, K, V > 0 and T a multiple of chunk_size");
  if (dtype != TOPS_F32 && dtype != TOPS_BF16)
    return tops_set_error(TOPS_ERR_DTYPE, "kda_stage_intra_fwd: dtype must be TOPS_F32 or TOPS_BF16");
  if ((long long)B * H * (T / C) >= (1LL << 31))
    return tops_set_error(TOPS_ERR_SHAPE, "kda_stage_intra_fwd: too many (batch, head, chunk) triples");
  if (T == 0) return TOPS_OK;
  IntraFwdArgs a{q, k, g, beta, v, segment_ids, u, w, qg, kg, Aqk, Akk_inv, H, T, K, V, scale};
  const int grid = B * H * (T / C);
  hipStream_t s = (hipStream_t)stream;
#define KIF(TI, CC) kda_intra_fwd_kernel<TI, CC><<<grid, kNth, 0, s>>>(a)
  if (dtype == TOPS_F32) {
    if (C == 16) KIF(float, 16); else if (C == 32) KIF(float, 32);
    else if (C == 64) KIF(float, 64); else KIF(float, 128);
  } else {
    if (C == 16) KIF(uint16_t, 16); else if (C == 32) KIF(uint16_t, 32);
    else if (C == 64) KIF(uint16_t, 64); else KIF(uint16_t, 128);
  }
#undef KIF
  return launch_status();
}

extern "C" int tops_delta_rule_fwd_h(const void* k, const void* w, const void* u, const float* g,
                                     const float* gk, int dtype, const float* h0, void* h,
                                     float* v_new, float* ht, const int32_t* cu_seqlens,
                                     const int32_t* chunk_offsets, int B, int T, int H, int K,
                                     int V, int N, int chunk_size, void* stream) {
  if (!k || !w || !u) return tops_set_error(TOPS_ERR_NULL, "delta_rule_fwd_h: null tensor");
  const int C = chunk_size;
  if (C <= 0 || C > kDC)
    return tops_set_error(TOPS_ERR_UNSUPPORTED, "delta_rule_fwd_h: chunk_size must be in 1..64");
  if (K <= 0 || K > kDK || V <= 0 || B <= 0 || H <= 0 || T < 0 || N <= 0)
    return tops_set_error(TOPS_ERR_SHAPE, "delta_rule_fwd_h: need 0 < K <= 128 and positive B, H, V, N");
  if (cu_seqlens && (B != 1 || !chunk_offsets))
    return tops_set_error(TOPS_ERR_SHAPE, "delta_rule_fwd_h: varlen needs B == 1 and chunk_offsets");
  if (!cu_seqlens && (N != B || T % C))
    return tops_set_error(TOPS_ERR_SHAPE, "delta_rule_fwd_h: N must equal B and T be a multiple of chunk_size");
  if (dtype != TOPS_F32 && dtype != TOPS_BF16)
    return tops_set_error(TOPS_ERR_DTYPE, "delta_rule_fwd_h: dtype must be TOPS_F32 or TOPS_BF16");
  DeltaHArgs a{k, w, u, g, gk, h0, h, v_new, ht, cu_seqlens, chunk_offsets, T, H, K, V, C};
  const dim3 grid(N * H, (V + kDV - 1) / kDV);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == TOPS_F32) delta_h_kernel<float><<<grid, kNth, 0, s>>>(a);
  else delta_h_kernel<uint16_t><<<grid, kNth, 0, s>>>(a);
  return launch_status();
}
