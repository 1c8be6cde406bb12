// MI355X batch model runner: the speculative-decoding verify step and the assistant draft loop of
// Gradiated/carat behind the reference's own runner interface
// (include/carat/batch_model_runner.h:22-77, include/carat/assistant_runner.h:11-27).
//
// One HIP stream per runner; every call is synchronous on return, like the reference. All device
// memory (weights, KV arenas, workspaces) is allocated in the constructor; the verify and draft
// paths allocate nothing.
#pragma once

#include "common.h"
#include "gemm.h"

#include <map>
#include <memory>
#include <optional>
#include <string>
#include <vector>

namespace carat_hip {

struct LayerSpec {
  bool sliding = true;
  int query_heads = 32;
  int kv_heads = 16;
  int head_dimension = 128;
  bool key_equals_value = false;
};

struct AssistantSpec {
  bool enabled = false;
  int hidden = 1024;
  int intermediate = 8192;
  int layers = 4;          // layers 0..layers-2 sliding, the last global (assistant_runner.cu:162-169)
  int query_heads = 32;
  // AssistantFp8Mode (assistant_runner.cu:29-43): 0 off (bf16 projections), 1 lm_head (the
  // draft lm_head in e4m3), 2 all (every projection in e4m3, inputs quantised per tensor);
  // -1 reads CARAT_ASSISTANT_FP8_MODE as the reference does (unset: off).
  int fp8_mode = -1;
};

struct ModelSpec {
  int hidden = 5376;
  int intermediate = 21504;
  int vocabulary = 262144;
  int sliding_window = 1024;
  float eps = 1e-6f;
  std::vector<LayerSpec> layers;
  AssistantSpec assistant;
  uint64_t seed = 1;
  float weight_std = 0.02f;
  // Fp8Scaling of the target's e4m3 weights (include/carat/linear.h:27): 0 tensor, 1 channel,
  // 2 block_128 (Fp8WeightArena::quantize, device_weights.cu:200-263).
  int fp8_scaling = 0;
};

// Gemma-4-31B-shaped target at the benchmark's attention shapes: 60 layers, 5 sliding : 1 global,
// 32 query heads / 16 KV heads, head_dim 128, hidden 5376, intermediate 21504, vocab 262144.
ModelSpec gemma4_31b_benchmark_spec(bool with_assistant);

// Kernel kinds of the verify step that timing probes can bracket.
enum ProbeKind : int {
  probe_none = -1,
  probe_qkv_gemm = 0,
  probe_o_gemm = 1,
  probe_gate_up_gemm = 2,
  probe_down_gemm = 3,
  probe_lm_head_gemm = 4,
  probe_sliding_attention = 5,
  probe_global_attention = 6,
};

struct GreedyVerificationResult {
  std::vector<int> accepted_tokens;
  std::vector<int> next_tokens;
};

struct LayerSlicedSuffixPrefillResult {
  bool complete = false;
  std::vector<int> predictions;
};

struct Checkpoint;

class BatchModelRunner {
public:
  // Seeded random weights of the described shape (benchmarks, tests).
  BatchModelRunner(const ModelSpec &spec, int batch, int maximum_context);
  // Weights streamed from a checkpoint (the model shape is the checkpoint's): bf16 execution
  // segments are uploaded, fp8 matrices quantised per tensor on the device (amax/448,
  // device_weights.cu:200-263) and packed. The checkpoint is only read during construction.
  BatchModelRunner(const Checkpoint &checkpoint, int batch, int maximum_context);
  // Weights already on the device (the reference's DeviceWeightArena / Fp8WeightArena,
  // device_weights.h:15-52): segment(context, assistant, fp8, name, &scale) returns the device
  // address of the execution segment the reference's WeightPlan names `name`
  // (weight_plan.cpp:37-189), laid out as that plan lays it out: bf16 when fp8 == 0; e4m3 with
  // its per-tensor scale (a device float stored to *scale) when fp8 == 1, or null, in which
  // case the runner quantises the bf16 segment per tensor (amax/448) itself. *bytes holds the
  // size the runner expects on entry; the source stores the segment's own size there when it
  // knows it, and a different size is an error (nothing is copied). Segments are copied device
  // to device and packed; they are only read during construction.
  using DeviceSegmentFn = const void *(*)(void *context, int assistant, int fp8, const char *name,
                                          const float **scale, uint64_t *bytes);
  BatchModelRunner(const ModelSpec &spec, DeviceSegmentFn segment, void *context, int batch,
                   int maximum_context);
  ~BatchModelRunner();
  BatchModelRunner(const BatchModelRunner &) = delete;
  BatchModelRunner &operator=(const BatchModelRunner &) = delete;

  // batch_model_runner.h:33-50. Prompts become resident from each slot's current position through
  // the verify kernels as forced steps (every row committed); a step holds all the cohort's
  // active slots, up to max(batch x 8, min(1024, context)) rows and never more rows than the
  // smallest sliding ring. The fp8 activation scales are per step, not per reference chunk.
  // prefill_slot resets the slot and returns the greedy token after the whole prompt;
  // prefill_slot_from_prefix requires the first cached_prefix_tokens to be resident already.
  int prefill_slot(int slot, const std::vector<int> &token_ids, int chunk_tokens = 1024);
  int prefill_slot_from_prefix(int slot, const std::vector<int> &token_ids, int cached_prefix_tokens,
                               int chunk_tokens = 1024);
  // The greedy next token only when the complete prompt is resident.
  std::optional<int> prefill_slot_chunk(int slot, const std::vector<int> &token_ids,
                                        int chunk_tokens);
  std::vector<std::optional<int>> prefill_slots_chunks(
      const std::vector<int> &slots, const std::vector<const std::vector<int> *> &token_ids,
      int chunk_tokens);
  // Each slot's whole remaining prompt; the greedy next token of every request.
  std::vector<int> prefill_slots_suffix(const std::vector<int> &slots,
                                        const std::vector<const std::vector<int> *> &token_ids);
  // The same computation, maximum_layers layers per call; the hidden states live in buffers of
  // their own between calls, so verify / draft / append calls on other slots may run in between.
  // complete (and the predictions) once the last layer is done; the same cohort (slots and
  // prompts) must be passed until then, or the state aborted.
  LayerSlicedSuffixPrefillResult prefill_slots_suffix_layer_slice(
      const std::vector<int> &slots, const std::vector<const std::vector<int> *> &token_ids,
      int maximum_layers);
  void abort_suffix_layer_slices();
  bool has_suffix_layer_slices() const;
  // Copies the source slot's resident KV rows, hidden hand-off row and position; returns the KV
  // bytes copied (K and V).
  uint64_t clone_slot(int source_slot, int destination_slot);
  // One lock-step decode token for every slot at the shared position (batch_model_runner.cu:
  // 1006-1040); every slot is then at the next position.
  std::vector<int> append(const std::vector<int> &token_ids);
  // cuda/batch_model_runner.cu:1617-1810 semantics.
  // batch_model_runner.h:55: one decode step for each (token, slot); returns the next tokens.
  std::vector<int> append_ragged(const std::vector<int> &token_ids, const std::vector<int> &slots);
  GreedyVerificationResult verify_greedy_proposals(
      const std::vector<std::vector<int>> &proposals, const std::vector<int> &target_first_tokens,
      const std::vector<int> &slots, const std::vector<int> &maximum_accepted_tokens = {});
  // cuda/batch_model_runner.cu:1812-1836 + cuda/assistant_runner.cu:218-338 semantics.
  std::vector<std::vector<int>> draft_four(const std::vector<int> &last_tokens,
                                           const std::vector<int> &slots,
                                           const std::vector<int> &forced_first_tokens = {},
                                           int depth = 4);
  bool has_assistant() const;
  void reset_slot(int slot);
  void seed_empty_cache_for_benchmark(int position);
  int batch() const;
  int position() const;
  int slot_position(int slot) const;

  // ---- benchmark / test helpers (no reference counterpart)
  // Fills every KV arena with seeded N(0, stddev) bf16 values and sets all slot positions.
  void seed_random_cache_for_benchmark(int position, uint64_t seed, float stddev);
  void set_slot_position(int slot, int position);
  // Target predictions (argmax of every verified row, [R*T]) of the last verify call.
  const std::vector<int> &last_predictions() const;
  // Named device tensors for inspection by tests ("layer.3.qkv", "cache.0.k", ...). Weights are
  // held in the GEMM's packed order; `layout` (optional) receives it (n = 0 for other tensors).
  void *tensor(const std::string &name, size_t *bytes, WeightLayout *layout = nullptr) const;
  hipStream_t stream() const;
  // Optional HIP-graph replay of the verify step (keyed by batch shape).
  void set_graphs_enabled(bool enabled);
  // Whether the verify step's layer-end rows quantise the next GEMM's operand themselves (1) or a
  // separate prepare kernel does (0, the default: faster in the step); the results are the same
  // bit for bit. 2 fuses
  // with a zero bound on the workgroups' wait for the agreed amax, so that every waiting
  // workgroup reports a timeout and the step raises (a test of that error path).
  void set_fused_quantization(int mode);
  // Whether verify attention post-processes its own QKV rows (true, the default: one launch fewer
  // per layer) or the separate QKV kernel runs first; the results are the same bit for bit.
  void set_qkv_fusion(bool enabled);
  // Milliseconds of the last verify / draft call's device work (hip events on the runner stream).
  float last_verify_ms() const;
  float last_draft_ms() const;
  // Timing probes: hip events around every launch of one kernel kind of the verify step
  // (ProbeKind); accumulated over calls until read. Probes force eager (non-graph) launches.
  void set_probe(int kind);
  void read_probe(float *total_ms, int *launches);
  // Back-to-back timing of one per-layer fp8 GEMM kind (probe_qkv_gemm .. probe_down_gemm) over
  // every layer's weights, `passes` times, on the last verify's activations (prepared once):
  // hip events around the whole sequence, so dispatch latency overlaps as it does in a step.
  // Overwrites only that GEMM's scratch outputs. Returns the mean kernel time per launch.
  float stream_gemm_probe(int kind, int passes, int *launches);

private:
  struct Implementation;
  std::unique_ptr<Implementation> implementation_;
};

}  // namespace carat_hip
