// Internal interfaces of the GLA chunk kernels (gla_sweep.hip, gla_dqkg.hip).
#pragma once
#include <hip/hip_runtime.h>

namespace tops {

// Gate modes of the chunk kernels (runtime, wave-uniform):
//   kGateK     g is [B,T,H,K] per-channel log-gates (GLA)
//   kGateS     g is [B,T,H] one log-gate per (token, head), shared by all K channels
//   kGateGamma g is gamma[H], a constant log-decay per head (simple GLA g_gamma)
//   kGateGammaK g is gamma[H,K], a constant log-decay per head and channel (GLA g_gamma;
//              its gradient is written per token as for kGateK, [B,T,H,K])
enum { kGateK = 0, kGateS = 1, kGateGamma = 2, kGateGammaK = 3 };

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
  int gate_mode;
  // KDA (delta rule) sweeps only:
  const float* u;        // forward: u = T (beta v) [B,T,H,V]
  const float* w;        // w = T (beta 2^G k) [B,T,H,K]
  float* y32;            // forward: v_new [B,T,H,V] or NULL; reverse: dv_new per chunk,
                         // transposed, [total,H,V,C]
  // state-only pass (sequence-parallel segments):
  float* dec_fin;        // [N,H,K] sum of the log2 gates over the sequence, or NULL
  const int* seg_end;    // [N] end row of sequence n (its start is cu_seqlens[n]), or NULL:
                         // sequence n then ends where n + 1 starts
  // checkpoints written: 0 = every chunk, 1 = even global chunks only, 2 = odd only (the
  // interleaved layout: h before the even chunks, dh after the odd ones, in one buffer)
  int ckpt_par;
  // reverse sweep only: gshift = 1 reads the gate of token t - 1 at token t (0 at the first
  // token of a sequence) and starts from s0 decayed by the gate of the sequence's last
  // token; every output element is multiplied by oscale.  With q and k exchanged, v as Y and
  // scale 1 this is the reverse-time recurrence S_t = diag(2^g_t) S_(t+1) + k_t v_t^T,
  // o_t = oscale S_t^T q_t (fused_recurrent with reverse = True).
  int gshift = 0;
  float oscale = 1.f;
  // Channel slices (K beyond one 128-channel tile runs as slices; the caller loops over them):
  // q, k, a per-channel g and the state rows are read with row length ldk (0: K), the pointers
  // at the slice's first channel; s0 / s_fin / ckpt are [.., ldk, V] with this slice's rows
  // starting at their pointers (a constant per-channel gate [H, ldk] likewise).
  int ldk = 0;
  // Output accumulation over the slices, in fp32 acc32 [B,T,H,V]: acc_mode 0 writes out as
  // usual; 1 writes acc32 = result; 2 adds acc32 += result; 3 writes out = acc32 + result.
  float* acc32 = nullptr;
  int acc_mode = 0;
  // fp16 checkpoints (the pipelined bf16 sweep only): ckpt then points at fp16
  // [total, H, K, V] holding the state divided by 2^e, one power of two per (chunk, head,
  // 64-column V tile) chosen from the tile's largest magnitude (at most 2^15 after scaling),
  // and ckpt_scale [total, H, NV] receives the factors 2^e.
  int ckpt16 = 0;
  float* ckpt_scale = nullptr;
  // phase clocks of the pipelined sweep, [grid, 8 waves, 8] (read only by a library built
  // with TOPS_PHASE_CLOCKS; see gla_sweep_pipe.hip)
  unsigned long long* clocks = nullptr;
};

// TIn = uint16_t (bf16 bits) or float; REV = reverse (state-gradient) sweep;
// DELTA = the KDA delta-rule sweep (v_new = u - w S replaces v).
template <typename TIn, bool REV, bool DELTA = false>
hipError_t launch_gla_sweep(const SweepParams& p, hipStream_t s);

// The software-pipelined sweep (gla_sweep_pipe.hip) for bf16 calls with per-channel gates:
// same results as gla_sweep_kernel, the staging of chunk c + 1 overlapped with chunk c's
// matrix products.  launch_gla_sweep routes eligible calls to it.
bool gla_pipe_eligible(const SweepParams& p);
template <bool REV>
hipError_t launch_gla_pipe(const SweepParams& p, hipStream_t s);

// Sweep with the gate on the value side (g = gv [B,T,H,V], bf16 inputs), forward or (REV)
// the state-gradient recurrence: see gla_sweep.hip.
template <bool REV>
hipError_t launch_gla_sweep_gv(const SweepParams& p, hipStream_t s);

// State-only sweep: the end state s_fin of every sequence (from s0, usually zero) and the
// decay sums dec_fin; no output, no checkpoints.
template <typename TIn, bool REV>
hipError_t launch_gla_state_pass(const SweepParams& p, hipStream_t s);

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
  float* dg;             // [B,T,H,K] (kGateK), [B,T,H] (kGateS) or NULL
  const int* cu_seqlens;
  const int* chunk_offsets;
  const int* chunk_map;
  int total, B, T, H, K, V, N;
  float scale;
  int gate_mode;
  // optional fp32 terms added to dk and dg ([B,T,H,K]; the KDA WY part), or NULL
  const float* dk_add;
  const float* dg_add;
  // interleaved checkpoints (bf16 inputs): hs = dhs = one [total, H, K, V] buffer holding h
  // before every even global chunk and dh after every odd one; a workgroup takes a chunk
  // pair and recomputes the missing state of each chunk from its partner's.  h0 / dht
  // [N, H, K, V] (or NULL: zero) stand in where the partner is in another sequence.
  int paired;
  const float* h0;
  const float* dht;
  // Channel / value slices: q, k, g (per-channel), dq, dk, dg (per-channel) have row length
  // ldk (0: K) and v, dO row length ldv (0: V), their pointers at the slice's first column;
  // hs / dhs are [total, H, ldk, ldv] with the slice's (row, column) origin at their pointers.
  int ldk = 0, ldv = 0;
  // Accumulation of dq / dk over value slices, in fp32 dq32 / dk32 [B,T,H,ldk]: acc_mode 0
  // writes dq / dk; 1 writes dq32 / dk32 = result; 2 adds into them; 3 writes dq / dk =
  // dq32 / dk32 + result.  dg_accum != 0 adds this call's dg into dg instead of writing it.
  float* dq32 = nullptr;
  float* dk32 = nullptr;
  int acc_mode = 0;
  int dg_accum = 0;
  // fp16 checkpoints (SweepParams::ckpt16): hs / dhs point at fp16 [total, H, K, V] and
  // hs_scale / dhs_scale [total, H, NV] hold each 64-column tile's factor
  int ckpt16 = 0;
  const float* hs_scale = nullptr;
  const float* dhs_scale = nullptr;
};

// TV = type of v (the KDA backward passes fp32 v_new with bf16 q / k / dO)
template <typename TIn, typename TV = TIn>
hipError_t launch_gla_dqkg(const DqkgParams& p, hipStream_t s);

}  // namespace tops
