/* tops-hip: C ABI of the MI355X (gfx950) GLA hot path.
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t
 * (passed as void*), enqueues its kernels on that stream and returns
 * immediately.  Nothing here allocates, frees or synchronises, and no
 * entry point keeps mutable global state beyond the thread-local error
 * message, so calls are re-entrant.  Return value: TOPS_OK (0) or a
 * negative TOPS_ERR_* code; tops_last_error() gives the message.
 *
 * Layouts follow the reference API: q, k [B,T,H,K]; v, o, do [B,T,H,V];
 * per-channel log-gates g [B,T,H,K] (fp32); states [N,H,K,V] (fp32).
 * Varlen packing (cu_seqlens != NULL) requires B == 1; N = number of
 * sequences, otherwise N == B.  dtype selects the element type of
 * q/k/v/o/do and their gradients: TOPS_F32 or TOPS_BF16 (and TOPS_F16 where stated).
 *
 * Each declaration names the reference interface it replaces
 * (paths relative to the reference repository root).
 */
#ifndef TOPS_HIP_H_
#define TOPS_HIP_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TOPS_F32 0
#define TOPS_BF16 1
/* fp16 inputs: taken by the GLA / simple GLA chunk entry points (tops_gla_chunk_fwd,
 * tops_simple_gla_chunk_fwd, tops_gla_chunk_fwd_gamma, the _bwd, _bwd_dh and _bwd_dqkg
 * stages of all three, tops_chunk_*_slice, tops_chunk_state_pass and
 * tops_chunk_reverse_fwd); every other entry point rejects it (TOPS_ERR_DTYPE).  The
 * kernels read fp16 elements directly and split them into exact bf16 hi / lo halves, as
 * they do fp32 inputs; outputs in the input dtype are written as fp16. */
#define TOPS_F16 2

#define TOPS_OK 0
#define TOPS_ERR_NULL -1
#define TOPS_ERR_SHAPE -2
#define TOPS_ERR_DTYPE -3
#define TOPS_ERR_LAUNCH -4
#define TOPS_ERR_UNSUPPORTED -5

/* Message of the last failing call on this host thread ("" if none). */
const char* tops_last_error(void);
/* Library version string. */
const char* tops_version(void);
/* Internal: record an error message, return code. */
int tops_set_error(int code, const char* msg);

/* Bytes of the per-chunk state checkpoint buffer used between forward and
 * backward: total_chunks * H * K * V * 4. */
int64_t tops_gla_state_bytes(int total_chunks, int H, int K, int V);

/* Host-side varlen chunk map.  Replaces tops.utils.prepare_chunk_indices
 * (tops/utils.py:71-90) and the per-sequence chunk counts of
 * tops/cpu/ops/gla/chunk.py:206-212.  Host pointers.
 *   cu_seqlens [N+1]; chunk_offsets [N+1] (out; chunk_offsets[N] = total);
 *   chunk_indices [capacity][2] (out, may be NULL): (sequence id, chunk id).
 * Returns the total number of chunks, or a negative TOPS_ERR_* code
 * (empty segments are rejected, as tops/cpu/ops/gla/chunk.py:686 does). */
int tops_prepare_chunk_indices(const int32_t* cu_seqlens, int N, int C, int32_t* chunk_offsets,
                               int32_t* chunk_indices, int capacity);

/* Chunked GLA forward (C = 64 tiles).
 * Replaces tops.ops.gla.chunk_gla_fwd (tops/ops/gla/chunk.py:1103-1199), i.e. the
 * pallas_calls K1 chunk_cumsum (chunk.py:176), K7 chunk_fwd_h (ops/common/chunk_h.py:243),
 * K2 fwd_intra_gk (chunk.py:420) and K3 fwd_o_gk (chunk.py:1383).
 *   h0     [N,H,K,V] fp32 or NULL;  o [B,T,H,V] (dtype);  ht [N,H,K,V] fp32 or NULL
 *   h_ckpt [total_chunks,H,K,V] fp32 or NULL: state before every chunk (for backward)
 *   cu_seqlens [N+1] int32 or NULL; chunk_offsets [N+1] int32 (first global chunk of
 *   each sequence; required with cu_seqlens when h_ckpt is given).
 * Limits: K <= 128, K % 8 == 0, V % 8 == 0. */
int tops_gla_chunk_fwd(const void* q, const void* k, const void* v, const float* g,
                       const float* h0, void* o, float* ht, float* h_ckpt,
                       const int32_t* cu_seqlens, const int32_t* chunk_offsets,
                       int B, int T, int H, int K, int V, int N, int dtype, float scale,
                       void* stream);

/* Chunked GLA backward.  Replaces tops.ops.gla.chunk_gla_bwd / chunk_gla_bwd_with_pl
 * (tops/ops/gla/chunk.py:832-1095): K8 chunk_bwd_dh (ops/common/chunk_h.py:864) and the
 * fused K4 (chunk.py:1556), plus the oracle tops/cpu/ops/gla/chunk.py:469-640.
 *   h_ckpt   [total_chunks,H,K,V] fp32 from tops_gla_chunk_fwd (state before each chunk)
 *   dh_work  [total_chunks,H,K,V] fp32 scratch supplied by the caller
 *   do_      [B,T,H,V] (dtype);  dht [N,H,K,V] fp32 or NULL
 *   dq, dk [B,T,H,K] (dtype); dv [B,T,H,V] (dtype); dg [B,T,H,K] fp32; dh0 [N,H,K,V] fp32
 *   or NULL.  chunk_map [total_chunks] int32: sequence id of each global chunk
 *   (varlen only).  Same limits as the forward, plus V <= 128. */
int tops_gla_chunk_bwd(const void* q, const void* k, const void* v, const float* g,
                       const void* do_, const float* dht, const float* h_ckpt, float* dh_work,
                       void* dq, void* dk, void* dv, float* dg, float* dh0,
                       const int32_t* cu_seqlens, const int32_t* chunk_offsets,
                       const int32_t* chunk_map, int total_chunks,
                       int B, int T, int H, int K, int V, int N, int dtype, float scale,
                       void* stream);

/* The two stages of tops_gla_chunk_bwd, callable separately (same arguments and limits).
 * Stage 1 replaces K8 chunk_bwd_dh (tops/ops/common/chunk_h.py:790-878) together with the
 * dv part of K4 (tops/ops/gla/chunk.py:1447-1509): a reverse sweep over the chunks of every
 * (sequence, head) writing dh_work (dL/d(state after each chunk)), dv and dh0.
 * Stage 2 replaces the dq/dk/dg part of K4 (chunk.py:1447-1581) and the oracle's
 * chunk_gla_bwd_dqkg (tops/cpu/ops/gla/chunk.py:396-466): chunk-parallel, reading the
 * forward checkpoints h_ckpt and the stage-1 dh_work. */
int tops_gla_chunk_bwd_dh(const void* q, const void* k, const float* g, const void* do_,
                          const float* dht, float* dh_work, void* dv, float* dh0,
                          const int32_t* cu_seqlens, const int32_t* chunk_offsets,
                          int B, int T, int H, int K, int V, int N, int dtype, float scale,
                          void* stream);
int tops_gla_chunk_bwd_dqkg(const void* q, const void* k, const void* v, const float* g,
                            const void* do_, const float* h_ckpt, const float* dh_work,
                            void* dq, void* dk, float* dg,
                            const int32_t* cu_seqlens, const int32_t* chunk_offsets,
                            const int32_t* chunk_map, int total_chunks,
                            int B, int T, int H, int K, int V, int N, int dtype, float scale,
                            void* stream);

/* GLA with a constant gate: g_gamma [H,K] fp32, the log-decay of every (head, channel),
 * applied at every token (a scalar or per-head g_gamma is passed expanded to [H,K]; no gate
 * at all is g_gamma = 0).  Replaces the g is None branch of chunk_gla_fwd
 * (tops/ops/gla/chunk.py:1134-1163: g = broadcast(g_gamma) or zeros, and the analytic
 * cumsum g_gamma * (i + 1)) without a [B,T,H,K] gate in memory.  Arguments as
 * tops_gla_chunk_fwd / _bwd_dh / _bwd_dqkg; dg (optional, [B,T,H,K] fp32) is the gradient
 * w.r.t. the per-token gate the constant stands for: its sum over (B, T) is the gradient of
 * g_gamma [H,K] (chunk.py:987-995). */
int tops_gla_chunk_fwd_gamma(const void* q, const void* k, const void* v, const float* g_gamma,
                             const float* h0, void* o, float* ht, float* h_ckpt,
                             const int32_t* cu_seqlens, const int32_t* chunk_offsets,
                             int B, int T, int H, int K, int V, int N, int dtype, float scale,
                             void* stream);
int tops_gla_chunk_bwd_dh_gamma(const void* q, const void* k, const float* g_gamma,
                                const void* do_, const float* dht, float* dh_work, void* dv,
                                float* dh0, const int32_t* cu_seqlens,
                                const int32_t* chunk_offsets, int B, int T, int H, int K, int V,
                                int N, int dtype, float scale, void* stream);
int tops_gla_chunk_bwd_dqkg_gamma(const void* q, const void* k, const void* v,
                                  const float* g_gamma, const void* do_, const float* h_ckpt,
                                  const float* dh_work, void* dq, void* dk, float* dg,
                                  const int32_t* cu_seqlens, const int32_t* chunk_offsets,
                                  const int32_t* chunk_map, int total_chunks, int B, int T, int H,
                                  int K, int V, int N, int dtype, float scale, void* stream);

/* The training path of the GLA / simple GLA chunk ops with interleaved state checkpoints
 * (bf16 inputs only; K, V <= 128): the same three stages as tops_gla_chunk_fwd /
 * tops_gla_chunk_bwd_dh / tops_gla_chunk_bwd_dqkg (K7+K2+K3, K8 and K4 of
 * tops/ops/gla/chunk.py:1103-1199, 832-1095 and tops/ops/common/chunk_h.py:685-878), with
 * the residual states kept as one buffer ckpt [total_chunks,H,K,V] fp32:
 *   tops_chunk_fwd_paired     writes the state before every even global chunk;
 *   tops_chunk_bwd_dh_paired  writes dh (the gradient w.r.t. the state after the chunk)
 *                             for every odd global chunk into the same buffer;
 *   tops_chunk_bwd_dqkg_paired takes the chunks in pairs (2i, 2i+1) and rebuilds the
 *                             missing state of each from its partner's (one sweep step);
 *                             h0 / dht (the forward's initial state and the final-state
 *                             gradient, [N,H,K,V] or NULL) stand in where the partner lies
 *                             in another sequence.
 * Half the checkpoint bytes of the unpaired path, written and read.  gate_mode and g as
 * tops_chunk_state_pass (0: g [B,T,H,K]; 1: g [B,T,H]; 2: g_gamma [H]; 3: g_gamma [H,K]);
 * dg as the unpaired entry of that gate (NULL for mode 2).  Other arguments as the
 * unpaired entry points. */
int tops_chunk_fwd_paired(const void* q, const void* k, const void* v, const float* g,
                          int gate_mode, const float* h0, void* o, float* ht, float* ckpt,
                          const int32_t* cu_seqlens, const int32_t* chunk_offsets, int B, int T,
                          int H, int K, int V, int N, int dtype, float scale, void* stream);
int tops_chunk_bwd_dh_paired(const void* q, const void* k, const float* g, int gate_mode,
                             const void* do_, const float* dht, float* ckpt, void* dv,
                             float* dh0, const int32_t* cu_seqlens, const int32_t* chunk_offsets,
                             int B, int T, int H, int K, int V, int N, int dtype, float scale,
                             void* stream);
int tops_chunk_bwd_dqkg_paired(const void* q, const void* k, const void* v, const float* g,
                               int gate_mode, const void* do_, const float* h0, const float* dht,
                               const float* ckpt, void* dq, void* dk, float* dg,
                               const int32_t* cu_seqlens, const int32_t* chunk_offsets,
                               const int32_t* chunk_map, int total_chunks, int B, int T, int H,
                               int K, int V, int N, int dtype, float scale, void* stream);

/* fp16 state checkpoints for the GLA training path (bf16 inputs, per-channel gates,
 * K, V <= 128): tops_gla_chunk_fwd / _bwd_dh / _bwd_dqkg (tops/ops/gla/chunk.py:1103-1199,
 * 832-1095; tops/ops/common/chunk_h.py:685-878) with the forward's h and the reverse sweep's
 * dh kept as fp16 [total_chunks,H,K,V] (h_ckpt16 / dh16) plus one factor per (chunk, head,
 * 64-column tile of V), h_scale / dh_scale [total_chunks,H,ceil(V/64)] fp32: the stored
 * value times its tile's factor is the state (the factor is a power of two chosen from the
 * tile's largest magnitude, so the fp16 values stay below 2^15 and the scaling is exact;
 * the fp16 rounding is 2^-12 of the tile's largest entry).  Half the checkpoint bytes of the
 * fp32 entry points, written by the sweeps and read by dq / dk / dg.  No reference
 * counterpart for the format (the reference keeps h in fp32).  Other arguments as the fp32
 * entry points; dtype TOPS_BF16. */
int tops_gla_chunk_fwd_c16(const void* q, const void* k, const void* v, const float* g,
                           const float* h0, void* o, float* ht, uint16_t* h_ckpt16,
                           float* h_scale, const int32_t* cu_seqlens,
                           const int32_t* chunk_offsets, int B, int T, int H, int K, int V,
                           int N, int dtype, float scale, void* stream);
int tops_gla_chunk_bwd_dh_c16(const void* q, const void* k, const float* g, const void* do_,
                              const float* dht, uint16_t* dh16, float* dh_scale, void* dv,
                              float* dh0, const int32_t* cu_seqlens,
                              const int32_t* chunk_offsets, int B, int T, int H, int K, int V,
                              int N, int dtype, float scale, void* stream);
int tops_gla_chunk_bwd_dqkg_c16(const void* q, const void* k, const void* v, const float* g,
                                const void* do_, const uint16_t* h16, const float* h_scale,
                                const uint16_t* dh16, const float* dh_scale, void* dq, void* dk,
                                float* dg, const int32_t* cu_seqlens,
                                const int32_t* chunk_offsets, const int32_t* chunk_map,
                                int total_chunks, int B, int T, int H, int K, int V, int N,
                                int dtype, float scale, void* stream);

/* Heads wider than one kernel tile (K or V above 128): the reference pads K and V to
 * multiples of 128 and tiles them inside one kernel (tops/ops/gla/chunk.py:1146-1152, the
 * K / V block grid of K7 / K3 / K4).  Here the caller loops over channel slices (K) and, in
 * the dq / dk / dg stage, value slices (V), each at most 128 wide and a multiple of 8, and
 * calls these entry points once per slice on the same stream, with pointers at the slice's
 * first column of the full tensors (no copies):
 *   q, k, g (per-channel gate [B,T,H,ldk], or a constant [H,ldk]), dq, dk, dg (per-channel)
 *     rows of ldk elements; v, dO rows of ldv (the forward and the dh stage take all of V:
 *     their sweeps tile V themselves);
 *   h0 / ht / dht / dh0 / h_ckpt / dh_work [.., ldk, ldv] with the slice's rows (and, for
 *     the dq / dk / dg stage, columns) starting at the pointer.
 * Results that sum over slices are accumulated in fp32: the forward's o and the dh stage's
 * dv over channel slices (o_sum / dv_sum [B,T,H,V]), and dq, dk over value slices (dq_sum,
 * dk_sum [B,T,H,ldk]): acc_mode 0 writes the output directly (one slice), 1 writes the sum
 * buffer, 2 adds into it, 3 writes the output = sum + this slice (the last slice).  The
 * output pointer may be NULL for modes 1 and 2.  dg_accum != 0 adds this call's dg into dg
 * (a per-channel dg over value slices; a per-token dg [B,T,H] over every slice).  Slices
 * add up exactly: the recurrence is separate per state entry, so o and dv are sums over
 * channel slices, and dq, dk, dg sums over value slices.  gate_mode as
 * tops_chunk_fwd_paired.  dtype TOPS_F32 or TOPS_BF16. */
int tops_chunk_fwd_slice(const void* q, const void* k, const void* v, const float* g,
                         int gate_mode, const float* h0, void* o, float* o_sum, int acc_mode,
                         float* ht, float* h_ckpt, const int32_t* cu_seqlens,
                         const int32_t* chunk_offsets, int B, int T, int H, int K, int V, int N,
                         int ldk, int dtype, float scale, void* stream);
int tops_chunk_bwd_dh_slice(const void* q, const void* k, const float* g, int gate_mode,
                            const void* do_, const float* dht, float* dh_work, void* dv,
                            float* dv_sum, int acc_mode, float* dh0, const int32_t* cu_seqlens,
                            const int32_t* chunk_offsets, int B, int T, int H, int K, int V,
                            int N, int ldk, int dtype, float scale, void* stream);
int tops_chunk_bwd_dqkg_slice(const void* q, const void* k, const void* v, const float* g,
                              int gate_mode, const void* do_, const float* h_ckpt,
                              const float* dh_work, void* dq, void* dk, float* dg,
                              float* dq_sum, float* dk_sum, int acc_mode, int dg_accum,
                              const int32_t* cu_seqlens, const int32_t* chunk_offsets,
                              const int32_t* chunk_map, int total_chunks, int B, int T, int H,
                              int K, int V, int N, int ldk, int ldv, int dtype, float scale,
                              void* stream);

/* Reverse-time recurrence, chunked: fused_recurrent_gla_fwd with reverse = True
 * (tops/ops/gla/fused_recurrent.py:380-431; oracle tops/cpu/ops/gla/fused_recurrent.py:116-160,
 * one body iterated from the last token to the first), without gv:
 *     S_t = diag(exp(g_t)) S_(t+1) + k_t v_t^T   (S_T = h0),   o_t = scale S_t^T q_t,
 * ht = S at the first token of each sequence.  Runs on the reverse chunk sweep (the state
 * gradient recurrence has this form with q and k exchanged and the gate read one token
 * later), so it takes no reversed copies of the inputs.  q, k [B,T,H,K], v [B,T,H,V] in dtype;
 * g and gate_mode as tops_chunk_fwd_paired (natural-log gates); h0 [N,H,K,V] fp32 or NULL;
 * o [B,T,H,V] in dtype; ht [N,H,K,V] fp32 or NULL.  Varlen: cu_seqlens [N+1] with B == 1
 * (empty sequences pass h0 through).  K <= 128, K and V multiples of 8.  Inference only:
 * nothing is kept for a backward. */
int tops_chunk_reverse_fwd(const void* q, const void* k, const void* v, const float* g,
                           int gate_mode, const float* h0, void* o, float* ht,
                           const int32_t* cu_seqlens, int B, int T, int H, int K, int V, int N,
                           int dtype, float scale, void* stream);

/* Value-side gate, chunked: fused_recurrent_gla_fwd with gv and without gk
 * (tops/ops/gla/fused_recurrent.py:380-431; oracle tops/cpu/ops/gla/fused_recurrent.py:51-167):
 *     S_t = S_(t-1) diag(exp(gv_t)) + k_t v_t^T   (S_0 = h0),   o_t = scale S_t^T q_t,
 * computed in 64-token chunks on MFMA (the forward sweep with the gate applied per V column:
 * v~ = v 2^(Gm - G) in, 2^(G - Gm) out, per-column state decay).  q, k [B,T,H,K], v [B,T,H,V]
 * bf16; gv [B,T,H,V] fp32 natural-log gates; h0 [N,H,K,V] fp32 or NULL; o [B,T,H,V] bf16;
 * ht [N,H,K,V] fp32 or NULL.  Varlen: cu_seqlens [N+1] with B == 1.  K <= 128, K and V
 * multiples of 8; dtype TOPS_BF16 only.  Inference only: nothing is kept for a backward. */
int tops_gla_chunk_fwd_gv(const void* q, const void* k, const void* v, const float* gv,
                          const float* h0, void* o, float* ht, const int32_t* cu_seqlens, int B,
                          int T, int H, int K, int V, int N, int dtype, float scale, void* stream);

/* The same recurrence with o written in fp32 (o32 [B,T,H,V]) and, when o [B,T,H,V] bf16 is
 * not NULL, in bf16 as well (both rounded from the same fp32 value).  The training forward of
 * fused_recurrent_gla with gv (tops/ops/gla/fused_recurrent.py:496-619) takes both: the bf16
 * output is returned, the fp32 one kept for the gate gradient of the backward. */
int tops_gla_chunk_fwd_gv32(const void* q, const void* k, const void* v, const float* gv,
                            const float* h0, float* o32, void* o, float* ht,
                            const int32_t* cu_seqlens, int B, int T, int H, int K, int V, int N,
                            int dtype, float scale, void* stream);

/* The state-gradient sweep of the value-gated recurrence (the dv of fused_recurrent_gla's
 * backward with gv, tops/ops/gla/fused_recurrent.py:496-619): dS_t = dS_(t+1) diag(exp gv_(t+1))
 * + scale q_t dO_t^T from dS_T = dht + scale q_T dO_T^T, dv_t = dS_t^T k_t written in fp32
 * (dv32 [B,T,H,V]), and dh0 = dS_1 diag(exp gv_1) [N,H,K,V] fp32 or NULL.  q, k [B,T,H,K],
 * dO [B,T,H,V] bf16 (dtype TOPS_BF16), gv [B,T,H,V] fp32 natural-log gates, dht [N,H,K,V]
 * fp32 or NULL.  Chunked on MFMA (the reverse sweep with the gate per V column); K <= 128,
 * K and V multiples of 8; varlen: cu_seqlens [N+1] with B == 1. */
int tops_gla_chunk_bwd_dv_gv32(const void* q, const void* k, const void* do_, const float* gv,
                               const float* dht, float* dv32, float* dh0,
                               const int32_t* cu_seqlens, int B, int T, int H, int K, int V,
                               int N, int dtype, float scale, void* stream);

/* The state-gradient sweep of chunk_gla's backward (tops/ops/gla/chunk.py:1447-1509) without
 * state checkpoints: dv [B,T,H,V] bf16 and dh0 [N,H,K,V] fp32 (or NULL) from q, k, g
 * [B,T,H,K] (g fp32 per-channel natural-log gates), dO [B,T,H,V], dht [N,H,K,V] fp32 or
 * NULL; bf16 (dtype TOPS_BF16), K <= 128, K and V multiples of 8; varlen: cu_seqlens [N+1]
 * with B == 1.  The chunked backward of fused_recurrent_gla with gv uses it on the transposed
 * state gradient, where its dv is dk. */
int tops_gla_chunk_rev_dv(const void* q, const void* k, const float* g, const void* do_,
                          const float* dht, void* dv, float* dh0, const int32_t* cu_seqlens, int B,
                          int T, int H, int K, int V, int N, int dtype, float scale, void* stream);

/* Gate gradient of the value-gated recurrence (the dgv of fused_recurrent_gla's backward with
 * gv, tops/ops/gla/fused_recurrent.py:496-619; oracle tops/cpu/ops/gla/fused_recurrent.py:
 * 171-358 keeps the same running suffix sums):
 *     dgv[t, v] = sum over t' >= t in t's sequence of (o32 dO - v dv32)[t', v] + c[n, v],
 * o32, dv32 [B,T,H,V] fp32; dO, v [B,T,H,V] bf16 (dtype TOPS_BF16); c [N,H,V] fp32 (the
 * final-state term sum_k dht * ht) or NULL; dgv [B,T,H,V] fp32; dv_out [B,T,H,V] bf16 receives
 * dv32 rounded to bf16 (the gradient handed back for v), or NULL.  Varlen: cu_seqlens [N+1],
 * B == 1. */
int tops_gv_gate_grad(const float* o32, const void* dO, const void* v, const float* dv32,
                      const float* c, float* dgv, void* dv_out, const int32_t* cu_seqlens, int B,
                      int T, int H, int V, int N, int dtype, void* stream);

/* Simple GLA: one log-gate per (token, head) -- g [B,T,H] fp32 -- or a constant per-head
 * log-decay g_gamma [H] fp32; pass exactly one.  The state recurrence is GLA's with the
 * gate shared by all K channels.  Replaces tops.ops.simple_gla.chunk_simple_gla_fwd /
 * _varlen (tops/ops/simple_gla/chunk.py:464-577; K9 ops/common/chunk_h.py:887-962,
 * K10 ops/common/chunk_o.py:119-185) and the oracle tops/cpu/ops/simple_gla/chunk.py:53-129.
 * Other arguments as tops_gla_chunk_fwd. */
int tops_simple_gla_chunk_fwd(const void* q, const void* k, const void* v, const float* g,
                              const float* g_gamma, const float* h0, void* o, float* ht,
                              float* h_ckpt, const int32_t* cu_seqlens,
                              const int32_t* chunk_offsets, int B, int T, int H, int K, int V,
                              int N, int dtype, float scale, void* stream);

/* Simple GLA backward: dq, dk, dv, dh0 and, for a per-token g, dg [B,T,H] fp32 (the gate
 * gradient summed over the K channels; dg is ignored with g_gamma).  Replaces
 * tops.ops.simple_gla.chunk_simple_gla_bwd (tops/ops/simple_gla/chunk.py:579-674; K11
 * ops/common/chunk_o.py:277-366) and the oracle tops/cpu/ops/simple_gla/chunk.py:668-788.
 * Arguments as tops_gla_chunk_bwd. */
int tops_simple_gla_chunk_bwd(const void* q, const void* k, const void* v, const float* g,
                              const float* g_gamma, const void* do_, const float* dht,
                              const float* h_ckpt, float* dh_work, void* dq, void* dk, void* dv,
                              float* dg, float* dh0, const int32_t* cu_seqlens,
                              const int32_t* chunk_offsets, const int32_t* chunk_map,
                              int total_chunks, int B, int T, int H, int K, int V, int N,
                              int dtype, float scale, void* stream);

/* The two stages of tops_simple_gla_chunk_bwd, callable separately (arguments as there):
 * the reverse sweep writing dh_work, dv and dh0 (chunk_bwd_dh, tops/ops/common/chunk_h.py:
 * 790-878, as called at tops/ops/simple_gla/chunk.py:653) and the chunk-parallel
 * dq / dk / dg stage (K11, tops/ops/common/chunk_o.py:277-366). */
int tops_simple_gla_chunk_bwd_dh(const void* q, const void* k, const float* g,
                                 const float* g_gamma, const void* do_, const float* dht,
                                 float* dh_work, void* dv, float* dh0, const int32_t* cu_seqlens,
                                 const int32_t* chunk_offsets, int B, int T, int H, int K, int V,
                                 int N, int dtype, float scale, void* stream);
int tops_simple_gla_chunk_bwd_dqkg(const void* q, const void* k, const void* v, const float* g,
                                   const float* g_gamma, const void* do_, const float* h_ckpt,
                                   const float* dh_work, void* dq, void* dk, float* dg,
                                   const int32_t* cu_seqlens, const int32_t* chunk_offsets,
                                   const int32_t* chunk_map, int total_chunks, int B, int T,
                                   int H, int K, int V, int N, int dtype, float scale,
                                   void* stream);

/* Sequence-parallel sweeps (long or few sequences on one device).  The caller cuts each
 * sequence at chunk boundaries into segments, listed in token order as a varlen layout over
 * the same tokens (cu_seqlens of the segments, B == 1), and runs per sweep direction:
 *   1. tops_chunk_state_pass over a list of N pieces, piece i = rows [seg_start[i],
 *      seg_end[i]) (chunk-aligned except at a sequence end): its end state from a zero
 *      state, s_loc [N,H,K,V] fp32, and its summed log2 gates, dec [N,H,K] fp32.
 *      reverse != 0: the state-gradient sweep, z = q, y = dO; else z = k, y = v.  The pieces
 *      cover every segment that hands a state on (all but the last of a sequence forward,
 *      all but the first in reverse), possibly cut finer than the segments so the pass
 *      itself fills the device.
 *   2. tops_chunk_state_combine: real sequence n owns the segments
 *      [seg_first[n], seg_first[n+1]) and the pieces [st_first[n], st_first[n+1]), stored in
 *      sweep order; after piece e the running state enters segment st_dst[e] (-1: none).
 *      Writes every segment's incoming state init [Nseg,H,K,V] from s_in (h0, or dht when
 *      reverse, of the real sequences, [Nreal,H,K,V], or NULL for zero).
 *   3. the usual chunk sweep over the segments with h0 (dht) = init and chunk_offsets = each
 *      segment's first global chunk; its final states per segment give ht (last segment of
 *      each sequence) and dh0 (first segment).
 * No counterpart in the reference, whose K7/K8 state kernels sweep every sequence serially
 * (tops/ops/common/chunk_h.py:160-238, 685-878); results equal those of tops_gla_chunk_fwd
 * and tops_gla_chunk_bwd_dh up to fp32 rounding.  gate_mode: 0 = per-channel g [B,T,H,K],
 * 1 = per-token g [B,T,H], 2 = g_gamma [H], 3 = g_gamma [H,K].  T = rows of the token-major
 * tensors. */
int tops_chunk_state_pass(const void* z, const void* y, const float* g, int gate_mode,
                          float* s_loc, float* dec, const int32_t* seg_start,
                          const int32_t* seg_end, int T, int H, int K, int V, int N, int dtype,
                          float scale, int reverse, void* stream);
int tops_chunk_state_combine(const float* s_loc, const float* dec, const float* s_in,
                             float* init, const int32_t* seg_first, const int32_t* st_first,
                             const int32_t* st_dst, int Nreal, int H, int K, int V, int reverse,
                             void* stream);

/* Fused recurrent GLA forward: the per-token recurrence
 *   h_t = h_{t-1} * exp(gk_t)[:,None] * exp(gv_t)[None,:] + k_t v_t^T,  o_t = h_t^T (scale q_t)
 * over each sequence (reverse != 0: from its last token to its first).  Replaces
 * tops.ops.gla.fused_recurrent_gla_fwd (tops/ops/gla/fused_recurrent.py:236-431, K5 :140-228)
 * and the oracle tops/cpu/ops/gla/fused_recurrent.py:51-167, 362-422.
 *   gk [B,T,H,K] fp32 or NULL; gv [B,T,H,V] fp32 or NULL; h0 [N,H,K,V] fp32 or NULL
 *   o [B,T,H,V] (dtype); o32 [B,T,H,V] fp32 copy of o or NULL; ht [N,H,K,V] fp32 or NULL
 * Limits: K <= 128, K % 4 == 0. */
int tops_gla_fused_recurrent_fwd(const void* q, const void* k, const void* v, const float* gk,
                                 const float* gv, const float* h0, void* o, float* o32, float* ht,
                                 const int32_t* cu_seqlens, int B, int T, int H, int K, int V,
                                 int N, int dtype, float scale, int reverse, void* stream);

/* The same forward for sequences of a few tokens (decode steps against a state cache): one
 * workgroup per (sequence, head, 128 V columns), a wave per 32-column tile, keeps the state in
 * registers, so the launch reads h0 and writes ht once and is bound by those bytes.  Same arguments, semantics and
 * limits as tops_gla_fused_recurrent_fwd, which takes this kernel by itself for fixed-length
 * calls with T <= 4; varlen callers that know every sequence is short call it directly.  Any
 * length is computed correctly; long sequences run one token at a time.  Replaces
 * tops.ops.gla.fused_recurrent_gla_fwd (tops/ops/gla/fused_recurrent.py:380-431) on the
 * decode route of the reference's layer (tops/layers/gla.py:288-297, q_len <= 64). */
int tops_gla_fused_recurrent_fwd_decode(const void* q, const void* k, const void* v,
                                        const float* gk, const float* gv, const float* h0,
                                        void* o, float* o32, float* ht,
                                        const int32_t* cu_seqlens, int B, int T, int H, int K,
                                        int V, int N, int dtype, float scale, int reverse,
                                        void* stream);

/* Decode steps with the GLA layer's output norm fused as the epilogue:
 *   y_t = o_t / sqrt(mean_v(o_t^2) + eps) * weight * silu(g_t)     (per token and head, over V)
 * with o_t the output of tops_gla_fused_recurrent_fwd_decode (same recurrence and arguments).
 * Replaces the decode route of the reference's GLA layer: fused_recurrent_gla followed by
 * FusedRMSNormGated(o, g) (tops/layers/gla.py:288-297, 330-336; tops/modules/fused_norm_gate.py:
 * 6-37); with g NULL, RMSNorm(o) * weight (the layer's g_norm, tops/modules/layernorm.py:6-35).
 *   g [B,T,H,V] (dtype) or NULL; weight [V] fp32 or NULL; eps >= 0
 *   y [B,T,H,V] (dtype); ht [N,H,K,V] fp32 or NULL (o itself is not written)
 * Limits: as tops_gla_fused_recurrent_fwd_decode, and V <= 128 (one workgroup holds a row). */
int tops_gla_fused_recurrent_fwd_decode_norm_gate(const void* q, const void* k, const void* v,
                                                  const float* gk, const float* gv,
                                                  const float* h0, const void* g,
                                                  const float* weight, float eps, void* y,
                                                  float* ht, const int32_t* cu_seqlens, int B,
                                                  int T, int H, int K, int V, int N, int dtype,
                                                  float scale, int reverse, void* stream);

/* The GLA layer's decode route from its projections to the normalised output, one kernel:
 *   q, k, v = act(ShortConvolution(xq, xk, xv)) with the conv caches rolled, then the recurrence
 *   of tops_gla_fused_recurrent_fwd_decode (gk, h0 -> ht), then y = RMSNorm(o) * weight * silu(g).
 * Replaces, on the reference layer's decode route (tops/layers/gla.py:236-262, 288-297,
 * 330-336), the three ShortConvolution calls (tops/modules/convolution.py:44-173),
 * fused_recurrent_gla and FusedRMSNormGated (tops/modules/fused_norm_gate.py:6-37).
 *   xq, xk [B,T,H,K], xv [B,T,H,V] (dtype): the projections before the convolutions
 *   conv_w_* [D,W] fp32 (D = H*K, H*K, H*V), 1 <= W <= 8; conv_b_* [D] fp32 or NULL
 *   cache_* [N,D,W] fp32 or NULL (zeros; pass NULL for a prefill, which reads no cache);
 *   cache_*_out [N,D,W] fp32 or NULL: the last W inputs of each sequence (positions before it
 *   from cache_*); may alias cache_*.  activation 1: SiLU after the convolution
 *   gk [B,T,H,K] fp32 log gates or NULL; h0 [N,H,K,V] fp32 or NULL; g [B,T,H,V] (dtype) or NULL;
 *   weight [V] fp32 or NULL; y [B,T,H,V] (fp32 when y_fp32, else dtype); ht [N,H,K,V] fp32 or NULL
 * Limits: K <= 128, K % 4 == 0, V <= 128; forward time only. */
int tops_gla_decode_conv_norm_gate(const void* xq, const void* xk, const void* xv,
                                   const float* conv_w_q, const float* conv_w_k,
                                   const float* conv_w_v, const float* conv_b_q,
                                   const float* conv_b_k, const float* conv_b_v,
                                   const float* cache_q, const float* cache_k,
                                   const float* cache_v, float* cache_q_out, float* cache_k_out,
                                   float* cache_v_out, int W, int activation, const float* gk,
                                   const float* h0, const void* g, const float* weight, float eps,
                                   void* y, int y_fp32, float* ht, const int32_t* cu_seqlens,
                                   int B, int T, int H, int K, int V, int N, int dtype,
                                   float scale, void* stream);

/* KDA decode steps: the per-token delta rule
 *   S <- diag(exp g_t) S;  S <- S + beta_t k_t (v_t - S^T k_t)^T;  o_t = S^T (scale q_t)
 * on the same register-state kernel, for sequences of a few tokens.  q, k [B,T,H,K] and
 * v [B,T,H,V] (dtype); g [B,T,H,K] natural-log gates fp32; beta [B,T,H] fp32; h0 [N,H,K,V] fp32
 * or NULL; o [B,T,H,V] (dtype); ht [N,H,K,V] fp32 or NULL.  K <= 128, K % 4 == 0; varlen with
 * B == 1.  Replaces the decode use of tops.ops.kda.fused_recurrent_kda
 * (tops/cpu/ops/kda/fused_recurrent.py:71-209; the recurrence of tops/cpu/ops/kda/naive.py:10-118). */
int tops_kda_fused_recurrent_fwd_decode(const void* q, const void* k, const void* v,
                                        const float* g, const float* beta, const float* h0,
                                        void* o, float* ht, const int32_t* cu_seqlens, int B,
                                        int T, int H, int K, int V, int N, int dtype, float scale,
                                        void* stream);

/* Bytes of the workspace tops_gla_fused_recurrent_bwd needs (with_gv: a gv gate is used). */
int64_t tops_gla_fused_recurrent_bwd_workspace(int B, int T, int H, int K, int V, int N,
                                               int with_gv);

/* Fused recurrent GLA backward: dq, dk, dv (dtype), dgk [B,T,H,K] / dgv [B,T,H,V] fp32 (when
 * gk / gv are given; dgv needs the forward output o32 in fp32) and dh0 [N,H,K,V] fp32 or NULL.
 * A forward replay gives dq and the final state, a reverse pass dk, dv and dh0, and the gate
 * gradients are suffix sums of (q dq - k dk) / (o dO - v dv) plus the h_T * dht boundary
 * term.  Replaces tops.ops.gla.fused_recurrent_gla_bwd (tops/ops/gla/fused_recurrent.py:
 * 881-958; K6 :496-619; _compute_gate_grads :800-878) and the oracle
 * tops/cpu/ops/gla/fused_recurrent.py:171-358.  workspace: see the size query above. */
int tops_gla_fused_recurrent_bwd(const void* q, const void* k, const void* v, const float* gk,
                                 const float* gv, const float* o32, const void* do_,
                                 const float* dht, const float* h0, void* dq, void* dk, void* dv,
                                 float* dgk, float* dgv, float* dh0, float* workspace,
                                 const int32_t* cu_seqlens, int B, int T, int H, int K, int V,
                                 int N, int dtype, float scale, int reverse, void* stream);

/* Chunked KDA forward (gated delta rule with per-channel gates, C = 64 tiles).
 * Replaces tops.ops.kda.chunk_kda_fwd (tops/ops/kda/chunk.py:25-190): the gate
 * cumsum (tops/ops/kda/gate.py:19-51), the intra-chunk WY solve
 * kda_intra_chunk_fwd (tops/ops/kda/chunk_intra.py:168-274), the delta-rule
 * state pass chunk_gated_delta_rule_fwd_h (tops/ops/common/chunk_delta_h.py:848-979)
 * and the output kernel chunk_gla_fwd_o_gk (tops/ops/gla/chunk.py:1383-1440).
 *   g [B,T,H,K] natural-log gates, beta [B,T,H] (fp32); h0, ht [N,H,K,V] or NULL.
 *   Workspace (fp32, written): u [B,T,H,V], w [B,T,H,K].
 *   Saved for the backward (fp32, may be NULL for inference): tt [total,H,64,64]
 *   (T = (I + Akk)^-1 transposed per chunk), v_new [B,T,H,V], h_ckpt [total,H,K,V]
 *   (state before each chunk).
 *   chunk_offsets / chunk_map as for tops_gla_chunk_bwd (both required for varlen);
 *   total_chunks = B*ceil(T/64) or the varlen total.  K, V <= 128. */
int tops_kda_chunk_fwd(const void* q, const void* k, const void* v, const float* g,
                       const float* beta, const float* h0, void* o, float* ht, float* u, float* w,
                       float* tt, float* v_new, float* h_ckpt, const int32_t* cu_seqlens,
                       const int32_t* chunk_offsets, const int32_t* chunk_map, int total_chunks,
                       int B, int T, int H, int K, int V, int N, int dtype, float scale,
                       void* stream);

/* Allocation-free KDA forward (inference).  No counterpart in the reference: for callers
 * that cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  As tops_kda_chunk_fwd without the backward's saved
 * tensors; the WY workspace u, w lives in the library's static device scratch of
 * tops_kda_chunk_fwd_noalloc_max_bytes() bytes (64 MiB, one copy per GPU, held until the
 * process ends), so B*T*H*(K+V)*4 must fit in it, else TOPS_ERR_SHAPE before any launch.
 * The call allocates nothing; calls that overlap on one GPU share the scratch and race. */
int64_t tops_kda_chunk_fwd_noalloc_max_bytes(void);
int tops_kda_chunk_fwd_noalloc(const void* q, const void* k, const void* v, const float* g,
                               const float* beta, const float* h0, void* o, float* ht,
                               const int32_t* cu_seqlens, const int32_t* chunk_offsets,
                               const int32_t* chunk_map, int total_chunks, int B, int T, int H,
                               int K, int V, int N, int dtype, float scale, void* stream);

/* Chunked KDA backward.  Replaces tops.ops.kda.chunk_bwd.chunk_kda_bwd
 * (tops/ops/kda/chunk_bwd.py:655-832: the dAv, dhu, WY/dqkg and intra stages)
 * from the tensors saved by tops_kda_chunk_fwd (w, tt, v_new, h_ckpt).
 *   do [B,T,H,V] (dtype); dht [N,H,K,V] or NULL.
 *   Workspace (fp32, written): dh_work [total,H,K,V] (dS per chunk),
 *   dvn_work [total,H,V,64] (dv_new transposed per chunk), dk_work, dg_work [B,T,H,K]
 *   (fp32 inputs only; bf16 runs the WY and dq / dk / dg stages as one kernel that keeps
 *   those parts on chip, and dk_work / dg_work may be NULL).
 *   Outputs: dq, dk [B,T,H,K] and dv [B,T,H,V] (dtype); dbeta [B,T,H], dg [B,T,H,K]
 *   (w.r.t. the natural-log gates) fp32; dh0 [N,H,K,V] fp32 or NULL. */
int tops_kda_chunk_bwd(const void* q, const void* k, const void* v, const float* g,
                       const float* beta, const float* w, const float* tt, const float* v_new,
                       const float* h_ckpt, const void* do_, const float* dht, float* dh_work,
                       float* dvn_work, float* dk_work, float* dg_work, void* dq, void* dk, void* dv,
                       float* dbeta, float* dg, float* dh0, const int32_t* cu_seqlens,
                       const int32_t* chunk_offsets, const int32_t* chunk_map, int total_chunks,
                       int B, int T, int H, int K, int V, int N, int dtype, float scale,
                       void* stream);

/* fp16 state checkpoints for the simple-GLA training path (bf16 inputs, one gate per token
 * g [B,T,H] or a scalar g_gamma [H], K, V <= 128): tops_simple_gla_chunk_fwd / _bwd_dh /
 * _bwd_dqkg (tops/ops/simple_gla/chunk.py:464-577, 579-674) with h
 * and dh per chunk in the format of tops_gla_chunk_fwd_c16 (fp16 [total_chunks,H,K,V] plus
 * one power-of-two factor per (chunk, head, 64-column tile of V), fp32
 * [total_chunks,H,ceil(V/64)]).  Pass exactly one of g, g_gamma.  No reference counterpart for
 * the format.  Other arguments as the fp32 entry points; dtype TOPS_BF16. */
int tops_simple_gla_chunk_fwd_c16(const void* q, const void* k, const void* v, const float* g,
                                  const float* g_gamma, const float* h0, void* o, float* ht,
                                  uint16_t* h_ckpt16, float* h_scale, const int32_t* cu_seqlens,
                                  const int32_t* chunk_offsets, int B, int T, int H, int K, int V,
                                  int N, int dtype, float scale, void* stream);
int tops_simple_gla_chunk_bwd_dh_c16(const void* q, const void* k, const float* g,
                                     const float* g_gamma, const void* do_, const float* dht,
                                     uint16_t* dh16, float* dh_scale, void* dv, float* dh0,
                                     const int32_t* cu_seqlens, const int32_t* chunk_offsets,
                                     int B, int T, int H, int K, int V, int N, int dtype,
                                     float scale, void* stream);
int tops_simple_gla_chunk_bwd_dqkg_c16(const void* q, const void* k, const void* v,
                                       const float* g, const float* g_gamma, const void* do_,
                                       const uint16_t* h16, const float* h_scale,
                                       const uint16_t* dh16, const float* dh_scale, void* dq,
                                       void* dk, float* dg, const int32_t* cu_seqlens,
                                       const int32_t* chunk_offsets, const int32_t* chunk_map,
                                       int total_chunks, int B, int T, int H, int K, int V, int N,
                                       int dtype, float scale, void* stream);

/* fp16 state checkpoints for the KDA training path (bf16 inputs, K, V <= 128):
 * tops_kda_chunk_fwd / _bwd (tops/ops/kda/chunk.py:25-190; chunk_bwd.py:655-832) with the
 * forward's state per chunk (h_ckpt16) and the reverse sweep's dS per chunk (dh16_work)
 * as fp16 [total,H,K,V] plus one power-of-two factor per (chunk, head, 64-column tile of V),
 * h_scale / dh_scale [total,H,ceil(V/64)] fp32, the format of tops_gla_chunk_fwd_c16.  Half
 * the bytes of those two intermediates.  No reference counterpart for the format (the
 * reference recomputes the states in fp32).  The backward's WY and dq / dk / dg stages run as
 * one kernel (bf16), so there is no dk_work / dg_work.  Other arguments as the fp32 entry
 * points; dtype TOPS_BF16. */
int tops_kda_chunk_fwd_c16(const void* q, const void* k, const void* v, const float* g,
                           const float* beta, const float* h0, void* o, float* ht, float* u,
                           float* w, float* tt, float* v_new, uint16_t* h_ckpt16, float* h_scale,
                           const int32_t* cu_seqlens, const int32_t* chunk_offsets,
                           const int32_t* chunk_map, int total_chunks, int B, int T, int H,
                           int K, int V, int N, int dtype, float scale, void* stream);
int tops_kda_chunk_bwd_c16(const void* q, const void* k, const void* v, const float* g,
                           const float* beta, const float* w, const float* tt,
                           const float* v_new, const uint16_t* h_ckpt16, const float* h_scale,
                           const void* do_, const float* dht, uint16_t* dh16_work,
                           float* dh_scale, float* dvn_work, void* dq, void* dk, void* dv,
                           float* dbeta, float* dg, float* dh0, const int32_t* cu_seqlens,
                           const int32_t* chunk_offsets, const int32_t* chunk_map,
                           int total_chunks, int B, int T, int H, int K, int V, int N, int dtype,
                           float scale, void* stream);

/* KDA gate activation modes. */
#define TOPS_KDA_GATE_NONE 0        /* gate already activated (cumsum only) */
#define TOPS_KDA_GATE_SOFTPLUS 1    /* y = -exp(A_log[h]) * softplus(g + dt_bias[h, k]) */
#define TOPS_KDA_GATE_LOWER_BOUND 2 /* y = lower_bound * sigmoid(exp(A_log[h]) * (g + dt_bias[h, k])) */

/* KDA gate activation, y [rows,H,K] fp32 from the raw gate g [rows,H,K] (dtype g_dtype,
 * rows = B*T).  A_log [A_heads] fp32 (A_heads divides H; head h reads A_log[h / (H/A_heads)]);
 * dt_bias [bias_heads*K] fp32 or NULL, bias_heads = A_heads or H.  K % 4 == 0.
 * gate_mode: TOPS_KDA_GATE_SOFTPLUS or TOPS_KDA_GATE_LOWER_BOUND.
 * Replaces fused_kda_gate / kda_gate_fwd / naive_kda_gate / naive_kda_lowerbound_gate
 * (tops/cpu/ops/kda/gate.py:60-115, 161-176) and the head broadcast of
 * _expand_headwise_params (tops/cpu/ops/kda/gate.py:20-57). */
int tops_kda_gate_fwd(const void* g, int g_dtype, const float* A_log, const float* dt_bias,
                      float* y, int rows, int H, int K, int A_heads, int bias_heads,
                      int gate_mode, float lower_bound, void* stream);

/* Chunk-local cumulative sum of (optionally activated) gates, out [B,T,H,K] fp32:
 * out[t] = scale * sum over the tokens of t's chunk up to t of act(g).  Chunks of
 * chunk_size tokens tile each sequence from its start (varlen: cu_seqlens / chunk_offsets /
 * chunk_map of that chunk size, as for tops_gla_chunk_bwd; total_chunks = B*ceil(T/C) or
 * the varlen total).  gate_mode TOPS_KDA_GATE_NONE with scale = 1/ln 2 replaces
 * tops.ops.kda.gate.kda_gate_chunk_cumsum (tops/ops/kda/gate.py:19-51); the activated modes
 * replace the FLA-form kda_gate_chunk_cumsum (tops/cpu/ops/kda/gate.py:179-204). */
int tops_kda_gate_chunk_cumsum(const void* g, int g_dtype, const float* A_log,
                               const float* dt_bias, float* out, const int32_t* cu_seqlens,
                               const int32_t* chunk_offsets, const int32_t* chunk_map,
                               int total_chunks, int B, int T, int H, int K, int A_heads,
                               int bias_heads, int chunk_size, int gate_mode, float lower_bound,
                               float scale, void* stream);

/* Floats of the workspace tops_kda_gate_bwd needs (per-workgroup partials). */
int64_t tops_kda_gate_bwd_workspace(int rows, int H, int K);

/* KDA gate backward: dg [rows,H,K] (g_dtype), dA [A_heads] and dbias [bias_heads*K] (fp32)
 * from dyg [rows,H,K] fp32.  dA / dbias are summed over tokens and over the heads that share
 * a parameter row, in a fixed order (deterministic).  Replaces tops.ops.kda.gate.kda_gate_bwd
 * (tops/ops/kda/gate.py:54-119) and the autodiff backward of tops/cpu/ops/kda/gate.py:117-158. */
int tops_kda_gate_bwd(const void* g, int g_dtype, const float* A_log, const float* dt_bias,
                      const float* dyg, void* dg, float* dA, float* dbias, float* workspace,
                      int64_t workspace_floats, int rows, int H, int K, int A_heads,
                      int bias_heads, int gate_mode, float lower_bound, void* stream);

/* Row L2 normalisation y = x / sqrt(sum x^2 + 1e-6) over the last axis (D <= 256),
 * y fp32 [rows,D].  Replaces _l2_normalize_last_dim (tops/cpu/ops/kda/fused_recurrent.py:14-18)
 * of fused_recurrent_kda(use_qk_l2norm_in_kernel=True). */
int tops_l2norm_fwd(const void* x, int x_dtype, float* y, int rows, int D, void* stream);

/* Its backward: dx = r (dy - y (y . dy)), r = 1 / sqrt(sum x^2 + 1e-6); dy fp32, dx in
 * x_dtype.  (The reference differentiates _l2_normalize_last_dim by autodiff.) */
int tops_l2norm_bwd(const void* x, int x_dtype, const float* dy, void* dx, int rows, int D,
                    void* stream);

/* RMSNorm with an optional SiLU gate, y [rows,D] in x_dtype:
 *   y = x * rsqrt(mean(x^2) + eps) * weight * silu(g), computed in fp32.
 * g [rows,D] (g_dtype) or NULL (plain RMSNorm); weight [D] fp32 or NULL (no affine).
 * D <= 2048.  Replaces FusedRMSNormGated.__call__ (tops/modules/fused_norm_gate.py:28-37)
 * and RMSNorm.__call__ (tops/modules/layernorm.py:28-35). */
int tops_rmsnorm_gated_fwd(const void* x, int x_dtype, const void* g, int g_dtype,
                           const float* weight, void* y, int rows, int D, float eps,
                           void* stream);

/* Floats of the workspace tops_rmsnorm_gated_bwd needs when weight != NULL. */
int64_t tops_rmsnorm_gated_bwd_workspace(int rows, int D);

/* Its backward: dx (x_dtype), dg (g_dtype, when g != NULL) and dweight [D] fp32 (when
 * weight != NULL; per-workgroup partials added in a fixed order) from dy (x_dtype).
 * The reference differentiates the modules above by autodiff. */
int tops_rmsnorm_gated_bwd(const void* x, int x_dtype, const void* g, int g_dtype,
                           const float* weight, const void* dy, void* dx, void* dg,
                           float* dweight, float* workspace, int64_t workspace_floats, int rows,
                           int D, float eps, void* stream);

/* Causal depthwise convolution over time, y [B,T,D] (y_dtype):
 *   y[t, d] = act(sum_j x[t - W + 1 + j, d] * weight[d, j] + bias[d]),
 * zero left padding per sequence (varlen: cu_seqlens [N+1], B == 1).  weight [D,W] fp32
 * (the [D,1,W] depthwise kernel), bias [D] fp32 or NULL, 1 <= W <= 8, activation 0 (none)
 * or 1 (SiLU).  final_state [N,D,W] (x_dtype) or NULL: the last W inputs of each sequence,
 * zero left-padded.  Replaces ShortConvolution._causal_conv1d and the final-state window of
 * ShortConvolution.__call__ (tops/modules/convolution.py:44-80, 128-173). */
int tops_short_conv_fwd(const void* x, int x_dtype, const float* weight, const float* bias,
                        void* y, int y_dtype, void* final_state, const int32_t* cu_seqlens,
                        int B, int T, int D, int W, int N, int activation, void* stream);

/* Floats of the workspace tops_short_conv_bwd needs. */
int64_t tops_short_conv_bwd_workspace(int B, int T, int D, int W);

/* Its backward: dx [B,T,D] (x_dtype), dweight [D,W] and dbias [D] (fp32; dbias may be NULL)
 * from dy (dy_dtype).  Deterministic (fixed-order partial sums).  The reference
 * differentiates ShortConvolution by autodiff. */
int tops_short_conv_bwd(const void* x, int x_dtype, const float* weight, const float* bias,
                        const void* dy, int dy_dtype, void* dx, float* dweight, float* dbias,
                        float* workspace, int64_t workspace_floats, const int32_t* cu_seqlens,
                        int B, int T, int D, int W, int N, int activation, void* stream);

/* One decode step for N sequences: cache_out [N,D,W] fp32 = cache_in rolled by one along W
 * with x [N,D] appended (cache_out may alias cache_in), y [N,D] = act(sum_j cache_out[.., j]
 * * weight[d, j] + bias); without a cache (cache_in NULL) y = act(x * weight[d, W-1] + bias).
 * Replaces ShortConvolution.step (tops/modules/convolution.py:82-126). */
int tops_short_conv_step(const void* x, int x_dtype, const float* cache_in, float* cache_out,
                         const float* weight, const float* bias, void* y, int y_dtype, int N,
                         int D, int W, int activation, void* stream);

/* ---- Stage functions of chunked GLA (csrc/gla_stages.hip) --------------------------------
 * Each computes one intermediate of the chunk algorithm on its own, in fp32, for callers
 * that drive the stages separately (the fused chunk entry points above never write these
 * intermediates).  Layout [B,T,H,D] with T % chunk_size == 0, chunk_size 16, 32, 64 or 128;
 * q/k/v/do in `dtype` (TOPS_F32 / TOPS_BF16), gates, A, states and gradients fp32; K and V
 * positive multiples of 16.  Chunks are those of the flattened [B*T] token axis, which is
 * also the layout of a varlen batch whose cu_seqlens are multiples of chunk_size. */

/* Chunk-local cumsum of g ([B,T,H,S], or [B,H,T,S] when head_first): inclusive prefix sum
 * (suffix sum when reverse) inside each chunk, times scale (pass 1 for none).  g and out
 * each TOPS_F32 or TOPS_BF16; chunk_size any power of two; T need not be a multiple of it.
 * Varlen (B == 1): cu_seqlens [N+1], chunk_offsets [N+1], chunk_map [total_chunks] as for
 * tops_gla_chunk_bwd.  Replaces chunk_local_cumsum_vector (tops/ops/gla/chunk.py:110-198,
 * K1 :55-107; tops/ops/common/cumsum.py:472-540). */
int tops_chunk_local_cumsum(const void* g, int g_dtype, void* out, int out_dtype,
                            const int32_t* cu_seqlens, const int32_t* chunk_offsets,
                            const int32_t* chunk_map, int total_chunks, int B, int T, int H,
                            int S, int chunk_size, int head_first, int reverse, float scale,
                            void* stream);

/* Inter-chunk state recurrence over x [B,T,H,K], y [B,T,H,V] with optional chunk-local gate
 * cumsums gk [B,T,H,K], g [B,T,H] and per-head constant g_gamma [H] (log decay; the gate of
 * row t of a chunk is gk + g + g_gamma * (t + 1)).
 *   reverse == 0 (x = k, y = v): states[c / every] = state before chunk c (c % every == 0),
 *     then S = S * exp(G_last) + (x * exp(G_last - G))^T y; s0 = h0, s_final = ht.
 *     Replaces chunk_fwd_h_ref / chunk_fwd_h_kernel (tops/ops/common/chunk_h.py:100-489,
 *     K7 :22-92; tops/ops/gla/chunk.py:206-292).
 *   reverse == 1 (x = q, y = do): states[c] = gradient w.r.t. the state after chunk c, then
 *     dS = dS * exp(G_last) + (x * scale * exp(G))^T y; s0 = dht, s_final = dh0.  Replaces
 *     chunk_bwd_dh_ref / chunk_bwd_dh_kernel (chunk_h.py:575-884).
 * states [B, NT/every, H, K, V] in states_dtype; s0, s_final [N,H,K,V] fp32 or NULL.
 * cu_seqlens [N+1] (B == 1, every == 1): non-decreasing multiples of chunk_size from 0 to T.
 * K <= 256. */
int tops_chunk_state_recurrence(const void* x, const void* y, int dtype, const float* gk,
                                const float* g, const float* g_gamma, const float* s0,
                                void* states, int states_dtype, float* s_final,
                                const int32_t* cu_seqlens, int B, int T, int H, int K, int V,
                                int N, int chunk_size, int every, int reverse, float scale,
                                void* stream);

/* A [B,T,H,C] fp32 = scale * (q e^{g - gm}) (k e^{gm - g})^T per chunk, full square, gm the
 * mean of the chunk's first and last gate rows.  Replaces chunk_gla_fwd_intra_gk
 * (tops/ops/gla/chunk.py:390-438, K2 :351-387) and its ref (:300-343). */
int tops_gla_stage_attn(const void* q, const void* k, int dtype, const float* g, float* A,
                           int B, int T, int H, int K, int chunk_size, float scale,
                           void* stream);

/* o [B,T,H,V] (dtype) = scale * (q e^{g - gm}) (h_c e^{gm}) + tril(A) v per chunk, with
 * h [B,NT,H,K,V] fp32 and exp2 instead of exp when use_exp2.  Replaces chunk_gla_fwd_o_gk
 * (tops/ops/gla/chunk.py:1411-1440, K3 :1279-1335) and its ref (:446-501). */
int tops_gla_stage_o(const void* q, const void* v, int dtype, const float* g, const float* A,
                     const float* h, void* o, int B, int T, int H, int K, int V, int chunk_size,
                     float scale, int use_exp2, void* stream);

/* dA [B,T,H,C] (dA_dtype) = scale * tril(do v^T) per chunk.  Replaces chunk_gla_bwd_dA_ref
 * (tops/ops/gla/chunk.py:509-549). */
int tops_gla_stage_dattn(const void* v, const void* do_, int dtype, void* dA, int dA_dtype, int B,
                      int T, int H, int V, int chunk_size, float scale, void* stream);

/* dv [B,T,H,V] fp32 = tril(A)^T do + (k e^{g_last - g}) dh_c per chunk, dh [B,NT,H,K,V].
 * Replaces chunk_gla_bwd_dv_ref (tops/ops/gla/chunk.py:552-605). */
int tops_gla_stage_dv(const void* k, const void* do_, int dtype, const float* g, const float* A,
                      const float* dh, float* dv, int B, int T, int H, int K, int V,
                      int chunk_size, void* stream);

/* dq = e^{g - gm} dA (k e^{gm - g}), dk = e^{gm - g} dA^T (q e^{g - gm}) per chunk, dA used as
 * given (no mask); dq, dk [B,T,H,K] fp32.  Replaces chunk_gla_bwd_dqk_intra_ref
 * (tops/ops/gla/chunk.py:608-662). */
int tops_gla_stage_dqk_intra(const void* q, const void* k, int dtype, const float* g,
                             const float* dA, float* dq, float* dk, int B, int T, int H, int K,
                             int chunk_size, void* stream);

/* dq_out = dq + scale e^{g} (do h_c^T), dk_out = dk + e^{g_last - g} (v dh_c^T),
 * dg = reverse-cumsum over the chunk of (q dq_out - k dk_out) + e^{g_last} sum_v(h_c dh_c)
 * + sum over the chunk of the inter dk times k; all [B,T,H,K] fp32.  Replaces
 * chunk_gla_bwd_dqkg_ref (tops/ops/gla/chunk.py:665-760). */
int tops_gla_stage_dqkg(const void* q, const void* k, const void* v, const void* do_, int dtype,
                        const float* g, const float* h, const float* dh, const float* dq,
                        const float* dk, float* dq_out, float* dk_out, float* dg, int B, int T,
                        int H, int K, int V, int chunk_size, float scale, void* stream);

/* kda_intra_chunk_fwd (tops/ops/kda/chunk_intra.py:169-281, kernel :91-166), head-first
 * layout: q, k [B,H,T,K] (dtype), g [B,H,T,K] fp32 (chunk-local gate cumsum, log2 units),
 * beta [B,H,T] fp32, v [B,H,T,V] (dtype), segment_ids [B,T] int32 or NULL (tokens of
 * different segments do not interact).  Writes, in dtype: u [B,H,T,V], w, qg, kg [B,H,T,K],
 * Aqk and Akk_inv [B,H,T/C,C,C] (C = chunk_size: 16, 32, 64 or 128; T % C == 0). */
int tops_kda_stage_intra_fwd(const void* q, const void* k, const float* g, const float* beta,
                             const void* v, const int32_t* segment_ids, int dtype, void* u,
                             void* w, void* qg, void* kg, void* Aqk, void* Akk_inv, int B, int H,
                             int T, int K, int V, int chunk_size, float scale, void* stream);

/* chunk_gated_delta_rule_fwd_h (tops/ops/common/chunk_delta_h.py:898-977; ref :44-166;
 * oracle tops/cpu/ops/common/chunk_delta_h.py:22-118): the delta-rule state pass.
 * k (already gated), w [B,T,H,K] and u [B,T,H,V] in dtype; g [B,T,H] and gk [B,T,H,K] fp32
 * chunk-local gate cumsums in log2 units (either or both NULL); h0 [N,H,K,V] fp32 or NULL.
 * Writes h [total_chunks,H,K,V] (dtype; the state before each chunk), v_new [B,T,H,V] fp32
 * and ht [N,H,K,V] fp32 (each optional).  Varlen: cu_seqlens [N+1] with B == 1 and
 * chunk_offsets [N] (first chunk of each sequence, its chunks counted on their own);
 * otherwise T % chunk_size == 0 and N == B.  K <= 128, chunk_size <= 64. */
int tops_delta_rule_fwd_h(const void* k, const void* w, const void* u, const float* g,
                          const float* gk, int dtype, const float* h0, void* h, float* v_new,
                          float* ht, const int32_t* cu_seqlens, const int32_t* chunk_offsets,
                          int B, int T, int H, int K, int V, int N, int chunk_size, void* stream);

/* KDA intra-chunk backward through Aqk and Akk, with E_ij = 2^{g_i - g_j} per channel (g the
 * chunk-local gate cumsum in log2 units) and dAqk, dAkk [B,T,H,C] used on i >= j:
 *   dq_i = sum_j dAqk_ij k_j E_ij;  row_i = sum_j dAkk_ij k_j E_ij;  db_i = row_i . k_i;
 *   dk = beta_i row_i + sum_i dAqk_ij q_i E_ij + sum_i beta_i dAkk_ij k_i E_ij (column sums);
 *   dg_i = q_i dq_i + k_i beta_i row_i - k_i (column sums)  (no ln 2 factor, as the reference).
 * Writes the intra parts only: dq, dk, dg [B,T,H,K] and db [B,T,H] fp32; beta fp32 [B,T,H].
 * chunk_size 16, 32 or 64.  Replaces chunk_kda_bwd_intra (tops/ops/kda/chunk_intra.py:477-574,
 * K17 :283-386; CPU tier tops/cpu/ops/kda/chunk_intra.py:16-200). */
int tops_kda_stage_intra_bwd(const void* q, const void* k, int dtype, const float* g,
                             const float* beta, const float* dAqk, const float* dAkk, float* dq,
                             float* dk, float* db, float* dg, int B, int T, int H, int K,
                             int chunk_size, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TOPS_HIP_H_ */
