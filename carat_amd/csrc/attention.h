// Verify / decode attention for gfx950: K+1 query tokens per slot against a per-slot KV cache,
// MFMA QK and PV with wave-level online softmax, split over key chunks and merged by a combine
// kernel.
#pragma once

#include "common.h"
#include "rowops.h"

namespace carat_hip {

enum class AttentionMode : int {
  // Sliding-window verify: the cache is a ring of `capacity` rows holding positions < p (rows of
  // this step's proposals are NOT yet written); query p+t sees keys j in [p+t-window+1, p+t].
  sliding = 0,
  // Global verify: contiguous cache; query p+t sees keys j in [0, p+t]. Keys j < p come from the
  // cache, keys j >= p from this step's new rows.
  global = 1,
  // Single-token decode over the target cache: valid = min(position+1, capacity) physical rows,
  // no new rows (cuda/gemm_attention.cu:88-132).
  decode = 2,
};

struct AttentionArgs {
  AttentionMode mode = AttentionMode::global;
  const bf16_t *q = nullptr;        // [R][T][Hq][D] bf16
  const void *k_cache = nullptr;    // [slots][Hkv][C][D] bf16 or e4m3
  const void *v_cache = nullptr;
  const void *k_new = nullptr;      // [R][T][Hkv][D] (same dtype as the cache); unused in decode
  const void *v_new = nullptr;
  bool fp8_kv = false;
  float k_scale = 1.0f;             // fp8 only: dequantisation scales
  float v_scale = 1.0f;
  const int32_t *slots = nullptr;   // [R] cache slot of each request, < slot_count
  int slot_count = 0;               // cache slots (0: the slots are < requests)
  const int32_t *positions = nullptr;  // [R] first proposal position (decode: context position)
  int requests = 0;
  int tokens = 0;                   // T (1 for decode)
  int query_heads = 0;
  int kv_heads = 0;
  int dimension = 0;
  int capacity = 0;                 // rows per (slot, head) in the cache
  int window = 0;                   // sliding window (sliding mode)
  int max_keys = 0;                 // upper bound on keys per request (sizes the grid)
  bf16_t *out = nullptr;            // [R][T][Hq][D] bf16
  float *out_amax = nullptr;        // optional atomic max of |out|
  int amax_stripes = 1;             // floats of out_amax, see amax_publish
  // split-key workspace (attention_partials_floats); chunks are merged by a second kernel
  float *partials = nullptr;
  int chunk_keys = 0;               // keys per workgroup (multiple of 256; 0 = choose)
  hipEvent_t timing_start = nullptr;  // optional events around the main kernel (timing probes)
  hipEvent_t timing_stop = nullptr;
  // Verify steps: the QKV post-processing of the step (launch_qkv_post's work, `qkv` its
  // arguments over the projection's split-K partials) done by the attention kernel itself, each
  // workgroup for its (request, kv head): the query rows go straight into the workgroup, this
  // step's K/V rows (and a global layer's cache rows) are written before any key is read, and
  // `q` is not read. Decode steps (the assistant): the query-only post-processing, the rows also
  // written to `q` (= qkv.q_out) by the pair's first key chunk. Only where attention_can_fuse_qkv
  // holds.
  bool fuse_qkv = false;
  QkvArgs qkv;
};

size_t attention_partials_floats(int requests, int kv_heads, int max_keys, int chunk_keys,
                                 int query_rows, int dimension);
int attention_default_chunk(AttentionMode mode, int max_keys, int requests, int kv_heads,
                            bool fp8_kv = false, int dimension = 128);
void launch_attention(const AttentionArgs &args, hipStream_t stream);
// Whether launch_attention can run `args` with fuse_qkv: a verify step (sliding or global) at
// D = 128 with bf16 K/V, <= 16 query rows per kv head and <= 8 tokens, one key chunk per
// (request, kv head), and `qkv` the matching QKV post-processing over 1-2 split-K partials of an
// fp8 projection, with no position offset; or a one-row decode step at D = 128 with bf16 K/V
// whose `qkv` is the query-only post-processing (kv_heads 0) of 1-2 partials, bf16 (no scale
// operands) or fp8, writing its rows to `q`.
bool attention_can_fuse_qkv(const AttentionArgs &args);

}  // namespace carat_hip
