/*
 * carat MI355X verify path -- C ABI.
 *
 * Plain pointers and sizes only. Every function returns 0 on success and a non-zero status on
 * failure; carat_hip_last_error() then returns the message (thread-local), whose text matches the
 * reference's std::runtime_error messages for the same condition. Device pointers are HIP device
 * addresses; `stream` is a hipStream_t (NULL = the default stream). Runner calls are synchronous.
 *
 * Reference interfaces replaced (paths inside Gradiated/carat):
 *   runner        include/carat/batch_model_runner.h:22-77 (Gemma4BatchModelRunner)
 *   draft         include/carat/assistant_runner.h:11-27 (Gemma4AssistantRunner::draft_four)
 *   speculation   src/runtime/speculation.h:11-27
 *   ops           include/carat/cuda_ops.h (argmax_bf16_rows, rms_norm_*, embedding_batch_bf16),
 *                 include/carat/linear.h (Fp8Linear::run, Bf16Linear::run, quantize_bf16_to_fp8_*),
 *                 include/carat/prefill_gemm_attention.h (run_uniform_ring_batch / run_uniform_batch),
 *                 include/carat/gemm_attention.h (GemmGroupedDecodeAttention::run_ragged),
 *                 include/carat/qkv.h (Gemma4QkvPostprocessor::run_prefill_uniform_direct)
 */
#ifndef CARAT_HIP_H
#define CARAT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------------------------ */
/* status                                                                                      */
/* ------------------------------------------------------------------------------------------ */
const char *carat_hip_last_error(void);
int carat_hip_device_count(int *count);
int carat_hip_synchronize(void);

/* ------------------------------------------------------------------------------------------ */
/* speculation helpers -- src/runtime/speculation.h:11-27                                      */
/* ------------------------------------------------------------------------------------------ */
/* acceptance_cap (speculation.h:11-12) */
int carat_hip_acceptance_cap(int depth, int remaining, const int32_t *proposals,
                             int proposal_count, const int32_t *stop_ids, int stop_count,
                             int *cap_out);
/* commit_speculation (speculation.h:24-27); resident/emitted hold accepted_count + 1 entries. */
int carat_hip_commit_speculation(int forced_token, const int32_t *accepted_drafts,
                                 int accepted_count, int next_token, const int32_t *stop_ids,
                                 int stop_count, int32_t *resident, int *resident_count,
                                 int32_t *emitted, int *emitted_count, int32_t *next_out,
                                 int *stopped);

/* ------------------------------------------------------------------------------------------ */
/* runner -- Gemma4BatchModelRunner (batch_model_runner.h:22-77)                                */
/* ------------------------------------------------------------------------------------------ */
typedef struct carat_hip_layer_desc {
  int sliding;           /* 1 sliding-window (ring) layer, 0 global layer */
  int query_heads;
  int kv_heads;
  int head_dimension;    /* 128, 256 or 512 */
  int key_equals_value;
} carat_hip_layer_desc;

typedef struct carat_hip_model_desc {
  int hidden;
  int intermediate;
  int vocabulary;
  int sliding_window;
  float rms_norm_epsilon;
  int layer_count;
  const carat_hip_layer_desc *layers;
  int assistant;               /* 1: build the 4-layer MTP assistant */
  int assistant_hidden;
  int assistant_intermediate;
  int assistant_layers;
  int assistant_query_heads;
  uint64_t seed;               /* seeded synthetic weights */
  float weight_std;
  /* AssistantFp8Mode (assistant_runner.cu:29-43): 0 reads CARAT_ASSISTANT_FP8_MODE as the
   * reference's assistant runner does (unset = off), 1 off, 2 lm_head, 3 all. A mode other than
   * off needs quantized assistant weights: the seeded and checkpoint runners quantise the
   * assistant's matrices per tensor themselves (as the reference's loader does when the mode is
   * on, native_runtime_main.cpp:926-933); a runner over device weights takes them from the
   * assistant FP8 arena (segment(..., assistant = 1, fp8 = 1, ...)) and otherwise fails with
   * "assistant FP8 mode requires quantized assistant weights". */
  int assistant_fp8_mode;
  /* Fp8Scaling of the target's e4m3 weights (include/carat/linear.h:27, Fp8WeightArena::quantize
   * device_weights.cu:200-263): 0 tensor, 1 channel, 2 block_128. Under channel / block_128 each
   * projection and the lm_head quantise their activations per row / per 1 x 128 block
   * (run_decode_linear, layer_runner.cu:220-238) and scale inside the GEMM; a runner over device
   * weights copies the arena's scale arrays (n floats, or ceil(n/128) x kbp, kbp = ceil(k/128)
   * rounded up to 4). */
  int fp8_scaling;
} carat_hip_model_desc;

typedef struct carat_hip_runner carat_hip_runner;

/* Fills `desc` with the Gemma-4-31B-shaped benchmark target (60 layers, 5:1 sliding/global,
 * 32/16 heads x 128, hidden 5376, intermediate 21504, vocab 262144). `layers` must hold 60. */
int carat_hip_gemma4_benchmark_desc(carat_hip_model_desc *desc, carat_hip_layer_desc *layers,
                                    int with_assistant);
/* Gemma4BatchModelRunner(config, weights, batch, maximum_context, fp8, assistant...)
 * (batch_model_runner.h:24-28); weights are seeded synthetic tensors. */
int carat_hip_runner_create(const carat_hip_model_desc *desc, int batch, int maximum_context,
                            carat_hip_runner **out);
/* Real-checkpoint weight path (ShardedSafetensors::open + Gemma4Config::load + WeightPlan::gemma4
 * / gemma4_assistant, src/safetensors.cpp, src/gemma4_config.cpp:58-154, src/weight_plan.cpp:37-257).
 * model_dir holds config.json and model.safetensors(.index.json + shards); assistant_dir
 * (nullable) the assistant's safetensors. Weights must be BF16, named as the reference's plan
 * expects; every model.language_model.* tensor must be used.
 * describe: validates without reading weight data or touching the GPU; fills desc (desc->layers =
 * layers, which must hold the checkpoint's layer count; nullable to query the count) and the
 * plans' byte totals (nullable). create: Gemma4BatchModelRunner over the checkpoint's weights
 * (batch_model_runner.h:24-28 with DeviceWeightArena::load + Fp8WeightArena::quantize,
 * device_weights.cu:125-263): fp8 matrices are quantised per tensor on the device and packed. */
int carat_hip_checkpoint_describe(const char *model_dir, const char *assistant_dir,
                                  carat_hip_model_desc *desc, carat_hip_layer_desc *layers,
                                  int layer_capacity, uint64_t *target_bytes,
                                  uint64_t *assistant_bytes);
int carat_hip_runner_create_from_checkpoint(const char *model_dir, const char *assistant_dir,
                                            int batch, int maximum_context,
                                            carat_hip_runner **out);
/* Gemma4BatchModelRunner(config, weights, batch, maximum_context, fp8, assistant, assistant_fp8)
 * (batch_model_runner.h:24-28) over weights already resident on the device (DeviceWeightArena /
 * Fp8WeightArena, include/carat/device_weights.h:15-52): segment(context, assistant, fp8, name,
 * &scale) returns the device address of the execution segment the reference's WeightPlan names
 * `name` ("token_embedding", "layer.3.qkv", ...; weight_plan.cpp:37-189; assistant = 1 selects
 * the assistant's plan) -- bf16 when fp8 == 0; when fp8 == 1 its e4m3 copy with the per-tensor
 * scale's device address stored to *scale, or NULL, and the runner then quantises the bf16
 * segment per tensor (amax/448) itself. *bytes holds the segment size the runner expects on
 * entry: the callback stores the segment's own byte size there when it knows it, and a size
 * that differs fails the construction before anything is copied ("device weight <name> has N
 * bytes, the runner expects M"). Segments are copied device to device during construction (the
 * arenas may be freed afterwards) and packed. desc gives the shapes; its seed and weight_std
 * are unused. */
typedef const void *(*carat_hip_device_segment_fn)(void *context, int assistant, int fp8,
                                                   const char *name, const float **scale,
                                                   uint64_t *bytes);
int carat_hip_runner_create_from_device_weights(const carat_hip_model_desc *desc,
                                                carat_hip_device_segment_fn segment,
                                                void *context, int batch, int maximum_context,
                                                carat_hip_runner **out);
void carat_hip_runner_destroy(carat_hip_runner *runner);
/* Test/benchmark helper, no counterpart in the reference: the target predictions (argmax of every
 * row, [rows]) of the last verify, append or prefill step; *count = rows (min(rows, capacity)
 * copied). A prefill step in which no prompt becomes whole runs no lm_head: its rows read -1. */
int carat_hip_runner_last_predictions(carat_hip_runner *runner, int32_t *out, int capacity,
                                      int *count);
/* prefill_slot (batch_model_runner.h:34, batch_model_runner.cu:1044-1048): resets the slot, makes
 * tokens[count] resident in chunks of chunk_tokens and writes the greedy next token. */
int carat_hip_runner_prefill_slot(carat_hip_runner *runner, int slot, const int32_t *tokens,
                                  int count, int chunk_tokens, int32_t *next_token);
/* prefill_slots_chunks (batch_model_runner.h:40-43): request r's prompt is
 * tokens[offsets[r] .. offsets[r+1]); each advances by up to chunk_tokens tokens from its slot's
 * position. predictions[r] = the greedy next token when the whole prompt is resident, else -1. */
int carat_hip_runner_prefill_slots_chunks(carat_hip_runner *runner, int requests,
                                          const int32_t *slots, const int32_t *offsets,
                                          const int32_t *tokens, int chunk_tokens,
                                          int32_t *predictions);
/* prefill_slot_from_prefix (batch_model_runner.h:36-37, batch_model_runner.cu:1050-1062): the
 * first cached_prefix tokens of tokens[count] must already be resident in the slot; makes the
 * rest resident and writes the greedy next token. */
int carat_hip_runner_prefill_slot_from_prefix(carat_hip_runner *runner, int slot,
                                              const int32_t *tokens, int count, int cached_prefix,
                                              int chunk_tokens, int32_t *next_token);
/* prefill_slot_chunk (batch_model_runner.h:38-39): one chunk of up to chunk_tokens tokens;
 * *next_token = the greedy next token when the whole prompt is resident, else -1. */
int carat_hip_runner_prefill_slot_chunk(carat_hip_runner *runner, int slot, const int32_t *tokens,
                                        int count, int chunk_tokens, int32_t *next_token);
/* prefill_slots_suffix (batch_model_runner.h:44-45, batch_model_runner.cu:1127-1222): every
 * request's whole remaining prompt (layout as prefill_slots_chunks); predictions[requests]. */
int carat_hip_runner_prefill_slots_suffix(carat_hip_runner *runner, int requests,
                                          const int32_t *slots, const int32_t *offsets,
                                          const int32_t *tokens, int32_t *predictions);
/* prefill_slots_suffix_layer_slice (batch_model_runner.h:46-50, batch_model_runner.cu:1356-1496):
 * the same, maximum_layers layers per call; *complete = 1 and predictions[requests] written once
 * the last layer is done (0 and untouched before). The same cohort (slots, prompts) must be
 * passed until complete or aborted. */
int carat_hip_runner_prefill_slots_suffix_layer_slice(carat_hip_runner *runner, int requests,
                                                      const int32_t *slots, const int32_t *offsets,
                                                      const int32_t *tokens, int maximum_layers,
                                                      int *complete, int32_t *predictions);
/* abort_suffix_layer_slices / has_suffix_layer_slices (batch_model_runner.h:51-52). */
int carat_hip_runner_abort_suffix_layer_slices(carat_hip_runner *runner);
int carat_hip_runner_has_suffix_layer_slices(carat_hip_runner *runner, int *out);
/* clone_slot (batch_model_runner.h:53, batch_model_runner.cu:1507-1541): copies the source slot's
 * resident KV rows, hidden hand-off row and position; *copied_bytes = KV bytes copied. */
int carat_hip_runner_clone_slot(carat_hip_runner *runner, int source_slot, int destination_slot,
                                uint64_t *copied_bytes);
/* append (batch_model_runner.h:33, batch_model_runner.cu:1006-1040): tokens[batch], one lock-step
 * decode token for every slot at the shared position; writes next_tokens[batch]. */
int carat_hip_runner_append(carat_hip_runner *runner, const int32_t *tokens, int count,
                            int32_t *next_tokens);
/* verify_greedy_proposals (batch_model_runner.h:56-60): proposals row-major [requests][depth],
 * caps nullable (= empty vector). predictions (nullable) receives the target argmax of every row. */
int carat_hip_runner_verify(carat_hip_runner *runner, int requests, int depth,
                            const int32_t *proposals, const int32_t *target_first,
                            const int32_t *slots, const int32_t *caps, int32_t *accepted_out,
                            int32_t *next_out, int32_t *predictions_out);
/* Gemma4BatchModelRunner::append_ragged (batch_model_runner.h:55, batch_model_runner.cu:1544-1615):
 * one decode step for each (token, slot) at the slot's position; writes next_tokens[rows] and
 * advances each slot by one. */
int carat_hip_runner_append_ragged(carat_hip_runner *runner, int rows, const int32_t *tokens,
                                   const int32_t *slots, int32_t *next_tokens);
/* draft_four (batch_model_runner.h:62-65): forced nullable; proposals_out [rows][depth]. */
int carat_hip_runner_draft(carat_hip_runner *runner, int rows, int depth, const int32_t *last,
                           const int32_t *slots, const int32_t *forced, int32_t *proposals_out);
int carat_hip_runner_has_assistant(carat_hip_runner *runner, int *out);
int carat_hip_runner_batch(carat_hip_runner *runner, int *out);
int carat_hip_runner_position(carat_hip_runner *runner, int *out);
int carat_hip_runner_slot_position(carat_hip_runner *runner, int slot, int *out);
int carat_hip_runner_reset_slot(carat_hip_runner *runner, int slot);
int carat_hip_runner_seed_empty_cache_for_benchmark(carat_hip_runner *runner, int position);
/* No reference counterpart: benchmark/test helpers. */
int carat_hip_runner_seed_random_cache(carat_hip_runner *runner, int position, uint64_t seed,
                                       float stddev);
int carat_hip_runner_set_slot_position(carat_hip_runner *runner, int slot, int position);
int carat_hip_runner_tensor(carat_hip_runner *runner, const char *name, void **device_ptr,
                            size_t *bytes);
/* direction 0: device -> host, 1: host -> device; bytes must equal the tensor size. */
int carat_hip_runner_copy_tensor(carat_hip_runner *runner, const char *name, void *host,
                                 size_t bytes, int direction);
int carat_hip_runner_set_graphs(carat_hip_runner *runner, int enabled);
/* 0 (default): a separate quantisation kernel prepares the next fp8 GEMM's operand; 1: the verify
 * step's layer-end rows write it themselves. Same results bit for bit. 2: fused with a zero bound
 * on the workgroups' wait for the agreed amax, so the step reports the timeout error (a test of
 * that path). Other values are rejected. */
int carat_hip_runner_set_fused_quantization(carat_hip_runner *runner, int enabled);
/* No reference counterpart: 1 (default) lets the verify attention kernel post-process its own
 * (request, kv head)'s QKV rows (Q/K norm, RoPE, this step's K/V rows) where the shape allows,
 * one launch fewer per layer; 0 runs the separate QKV kernel first. Same results bit for bit. */
int carat_hip_runner_set_qkv_fusion(carat_hip_runner *runner, int enabled);
int carat_hip_runner_timing(carat_hip_runner *runner, float *verify_ms, float *draft_ms);
/* Benchmark helper, no counterpart in the reference: one speculative cycle of the reference's
 * scheduler (native_runtime_main.cpp:583-678) in C++ -- draft_four(last, slots, forced, depth),
 * acceptance_cap per request over `planted` [requests][depth] (the benchmark's proposals, row 0
 * = forced, which replace the drafts), verify_greedy_proposals over them with those caps,
 * commit_speculation per
 * request, after one append_ragged of the forced tokens of the requests that accepted nothing
 * (the scheduler's fallback, which gives their next token) -- timed on the host clock from a
 * synchronised device (*seconds_out). Every planted row must start with its forced token. Writes
 * the accepted counts, the next forced token and the last resident token of every request. */
int carat_hip_bench_speculative_cycle(carat_hip_runner *runner, int requests, int depth,
                                      const int32_t *last_tokens, const int32_t *slots,
                                      const int32_t *forced, const int32_t *planted,
                                      int remaining, const int32_t *stop_ids, int stop_count,
                                      int32_t *accepted_out, int32_t *next_out,
                                      int32_t *last_out, double *seconds_out);
/* Timing probes: hip events around every launch of one verify-step kernel kind (0 qkv GEMM, 1 O
 * GEMM, 2 gate/up GEMM, 3 down GEMM, 4 lm_head GEMM, 5 sliding attention, 6 global attention;
 * -1 off). Probing runs the verify step without HIP graphs. read_probe returns and resets the sums. */
int carat_hip_runner_set_probe(carat_hip_runner *runner, int kind);
int carat_hip_runner_read_probe(carat_hip_runner *runner, float *total_ms, int *launches);
/* Benchmark probe, no counterpart in the reference: back-to-back launches of one per-layer kernel
 * kind over every layer of the model that has it, `passes` times, on the last verify's
 * activations, timed with one pair of hip events; *avg_ms = mean time per launch. Kinds: fp8 GEMMs
 * 0 qkv, 1 O, 2 gate/up, 3 down (every layer's weights); 5 sliding and 6 global verify attention
 * (every such layer's cache, with its K/V rows of the last step). Only that kernel's scratch
 * outputs are overwritten. */
int carat_hip_runner_stream_gemm_probe(carat_hip_runner *runner, int kind, int passes,
                                       float *avg_ms, int *launches);

/* ------------------------------------------------------------------------------------------ */
/* op level (device pointers)                                                                   */
/* ------------------------------------------------------------------------------------------ */
/* The op-level calls keep their intermediates (argmax partial keys, the e4m3 activation operand,
 * attention partials and amax stripes) in one workspace per device that the library owns and
 * grows on demand (growing synchronises the device). Calls on one device therefore must not
 * overlap: enqueue them on one stream, or synchronise between streams. */
/* argmax_bf16_rows (cuda_ops.h, ops.cu:1566-1579) over fp32 (compared after bf16 rounding) or bf16
 * logits [requests*tokens][vocabulary], with the greedy acceptance of batch_model_runner.cu:
 * 1738-1759 fused (proposals nullable -> argmax only). caps nullable. */
int carat_hip_argmax_accept(const float *logits_f32, const uint16_t *logits_bf16, int requests,
                            int tokens, int vocabulary, const int32_t *proposals,
                            const int32_t *target_first, const int32_t *caps,
                            int32_t *predictions, int32_t *accepted, int32_t *next_tokens,
                            void *stream);

/* No counterpart in the reference. For callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc): carat_hip_argmax_accept
 * with its partial keys in a fixed per-device scratch array (64 Ki keys, 512 KiB) instead of a
 * library-allocated workspace. Calls no hipMalloc/hipFree. Rejects shapes needing more than 65536
 * keys (ceil(vocabulary / 8192) chunks for fp32 logits, / 16384 for bf16, times requests x tokens).
 * Every call on one device shares that scratch: calls that overlap on one device race. */
int carat_hip_argmax_accept_noalloc(const float *logits_f32, const uint16_t *logits_bf16,
                                    int requests, int tokens, int vocabulary,
                                    const int32_t *proposals, const int32_t *target_first,
                                    const int32_t *caps, int32_t *predictions, int32_t *accepted,
                                    int32_t *next_tokens, void *stream);

/* Fp8Linear::run (linear.h, linear.cu:780-803) with the activation quantisation of
 * quantize_bf16_to_fp8_e4m3_from_amax_values (linear.cu:273-296) fused: x bf16 [m][k], x_amax
 * device float (producer amax), w e4m3 [n][k], w_scale device float.
 * epilogue 0: y bf16 [m][n] (+ y_amax nullable); 1: partial fp32 [splits][m][n];
 * 2: argmax -> predictions [m] (the lm_head); 3: GELU gate over packed [gate|up], y [m][n/2]. */
int carat_hip_fp8_linear(const uint16_t *x, int m, int k, const float *x_amax, const uint8_t *w,
                         int n, const float *w_scale, int epilogue, int splits, uint16_t *y,
                         float *y_amax, float *partial, int32_t *predictions, void *stream);
/* run_decode_linear under Fp8Scaling::channel (1) / ::block_128 (2) (layer_runner.cu:220-238):
 * x bf16 [m][k] quantised per row (quantize_bf16_rows, linear.cu:300-316) or per 1 x 128 block
 * (quantize_activation_block_128_kernel, linear.cu:382-401), then Fp8Linear::run with OUTER_VEC /
 * VEC128 x BLK128x128 scales (linear.cu:706-717): w e4m3 [n][k], w_scales [n] or
 * [ceil(n/128)][kbp] (carat_hip_quantize_weight_fp8). Epilogues as carat_hip_fp8_linear; the
 * partials (epilogue 1) carry the full scale. */
int carat_hip_fp8_linear_scaled(const uint16_t *x, int m, int k, int fp8_scaling, const uint8_t *w,
                                int n, const float *w_scales, int epilogue, int splits, uint16_t *y,
                                float *partial, int32_t *predictions, void *stream);
/* fp8_weight_block_scale_elements (linear.cu:403-409) and its tensor / channel counterparts: the
 * scale floats of an [n][k] weight under fp8_scaling 0 / 1 / 2 (1, n, ceil(n/128) x kbp). */
int carat_hip_fp8_weight_scale_elements(int fp8_scaling, int n, int k, uint64_t *out);
/* Fp8WeightArena::quantize of one bf16 [n][k] segment (device_weights.cu:240-256): e4m3 [n][k]
 * row-major and its scales, per tensor (amax/448), row or 128 x 128 block (max(amax/448, 2^-24)). */
int carat_hip_quantize_weight_fp8(const uint16_t *w, int n, int k, int fp8_scaling, uint8_t *out,
                                  float *scales, void *stream);
/* No reference counterpart (cuBLASLt picks its own algorithm, linear.cu:53-72): the storage layout
 * (tiles per wave, waves per workgroup) and split-K factor the runner uses for an [n][k] weight,
 * so op-level calls can reproduce the runner's exact dispatch. */
int carat_hip_gemm_plan(int n, int k, int fp8, int gate_up, int *tiles_per_wave, int *waves,
                        int *splits);
/* Bf16Linear::run (linear.cu:534-643), same epilogues (no scales). */
int carat_hip_bf16_linear(const uint16_t *x, int m, int k, const uint16_t *w, int n, int epilogue,
                          int splits, uint16_t *y, float *y_amax, float *partial,
                          int32_t *predictions, void *stream);

/* Verify attention: mode 0 sliding ring (run_uniform_ring_batch + the unwrapped direct path,
 * prefill_gemm_attention.cu:552-730), 1 global causal (run_uniform_batch), 2 decode
 * (GemmGroupedDecodeAttention::run_ragged, gemm_attention.cu:618-676).
 * q [R][T][Hq][D] bf16; caches [slots][Hkv][capacity][D] (bf16, or e4m3 when fp8_kv) holding the
 * rows BEFORE this step; k_new/v_new [R][T][Hkv][D] this step's rows; out [R][T][Hq][D] bf16. */
int carat_hip_verify_attention(int mode, const uint16_t *q, const void *k_cache,
                               const void *v_cache, const void *k_new, const void *v_new,
                               int fp8_kv, float k_scale, float v_scale, const int32_t *slots,
                               const int32_t *positions, int requests, int tokens,
                               int query_heads, int kv_heads, int dimension, int capacity,
                               int window, int max_keys, uint16_t *out, float *out_amax,
                               int chunk_keys, void *stream);

/* Row kernel: rms_norm_bf16(_with_row_amax), rms_norm_add_and_norm_bf16, rms_norm_add_scale_bf16,
 * embedding_batch_bf16 (ops.cu:27-217, 321-335) and split-K reduction, one fused kernel.
 * source 0 embedding (tokens, vocabulary, embed_scale), 1 partials (splits, x_amax, w_scale),
 * 2 input x. Stage 1 runs when w1 != NULL, stage 2 when w2 != NULL. */
typedef struct carat_hip_row_args {
  int source;
  int rows;
  int width;
  float eps;
  const uint16_t *embedding;
  const int32_t *tokens;
  int vocabulary;
  float embed_scale;
  const float *partials;
  int splits;
  const float *x_amax;
  const float *w_scale;
  const uint16_t *x;
  uint16_t *v_out;
  const uint16_t *w1;
  const uint16_t *residual;
  const uint16_t *scalar;
  uint16_t *r1_out;
  const uint16_t *w2;
  uint16_t *y_out;
  float *y_amax;
} carat_hip_row_args;
int carat_hip_row_op(const carat_hip_row_args *args, void *stream);

/* Gemma4QkvPostprocessor::run_prefill_uniform_direct (qkv.cu:824-869; kernels :387-530) on packed
 * bf16 rows [rows][packed_width]: q_out [rows][Hq][D], k_new/v_new [rows][Hkv][D]; caches
 * nullable. cos/sin tables [positions][D] bf16 (carat_hip_rope_table). */
int carat_hip_qkv_post(const uint16_t *packed, int rows, int tokens, int query_heads,
                       int kv_heads, int dimension, int key_equals_value, float eps,
                       const uint16_t *q_norm, const uint16_t *k_norm, const uint16_t *cosine,
                       const uint16_t *sine, const int32_t *positions, const int32_t *slots,
                       uint16_t *q_out, uint16_t *k_new, uint16_t *v_new, uint16_t *k_cache,
                       uint16_t *v_cache, int capacity, void *stream);
/* rope_cache_kernel (qkv.cu:44-64) tables, host memory [positions][dimension] bf16. */
int carat_hip_rope_table(int dimension, int proportional, int positions, uint16_t *cosine,
                         uint16_t *sine);
/* f32 -> e4m3 with the kernels' conversion (RNE, saturating); device arrays. */
int carat_hip_f32_to_e4m3(const float *in, uint8_t *out, int64_t n, void *stream);

#ifdef __cplusplus
}
#endif
#endif
