// Error plumbing and small host helpers of the tops-hip C ABI.
#include <stdio.h>
#include <string.h>

#include "tops_hip.h"

static thread_local char g_err[512] = "";

extern "C" const char* tops_last_error(void) { return g_err; }

extern "C" const char* tops_version(void) { return "tops-hip 0.1.0 (gfx950)"; }

extern "C" int tops_set_error(int code, const char* msg) {
  snprintf(g_err, sizeof(g_err), "%s", msg ? msg : "");
  return code;
}

extern "C" int64_t tops_gla_state_bytes(int total_chunks, int H, int K, int V) {
  return (int64_t)total_chunks * H * K * V * 4;
}

// Host-side varlen chunk map (replaces tops/utils.py:71-90 prepare_chunk_indices and the
// per-sequence chunk counts of tops/cpu/ops/gla/chunk.py:206-212).
//   cu_seqlens [N+1] (host), chunk_size C.
//   chunk_offsets [N+1] (out): first global chunk of each sequence; chunk_offsets[N] = total.
//   chunk_indices [total][2] (out, optional): (sequence id, chunk id within sequence).
// Returns the total number of chunks, or a negative error code.
extern "C" int tops_prepare_chunk_indices(const int32_t* cu_seqlens, int N, int C,
                                          int32_t* chunk_offsets, int32_t* chunk_indices,
                                          int capacity) {
  if (!cu_seqlens || !chunk_offsets || N <= 0 || C <= 0)
    return tops_set_error(TOPS_ERR_NULL, "prepare_chunk_indices: bad arguments");
  int total = 0;
  chunk_offsets[0] = 0;
  for (int n = 0; n < N; ++n) {
    const int len = cu_seqlens[n + 1] - cu_seqlens[n];
    // an empty sequence has no chunk (tops/utils.py:71-90 gives it none); its state
    // passes through unchanged
    if (len < 0) return tops_set_error(TOPS_ERR_SHAPE, "prepare_chunk_indices: negative segment length");
    const int nc = (len + C - 1) / C;
    if (chunk_indices) {
      if (total + nc > capacity) return tops_set_error(TOPS_ERR_SHAPE, "prepare_chunk_indices: capacity");
      for (int c = 0; c < nc; ++c) {
        chunk_indices[2 * (total + c)] = n;
        chunk_indices[2 * (total + c) + 1] = c;
      }
    }
    total += nc;
    chunk_offsets[n + 1] = total;
  }
  return total;
}
