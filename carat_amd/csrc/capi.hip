// extern "C" boundary of the MI355X verify path (declarations and reference citations in
// include/carat_hip.h). Exceptions never cross the boundary: they become a non-zero status and a
// thread-local message.
#include "carat_hip.h"

#include "attention.h"
#include "gemm.h"
#include "init.h"
#include "rowops.h"
#include "checkpoint.h"
#include "runner.h"
#include "speculation.h"

#include <chrono>
#include <cstring>
#include <unordered_set>
#include <map>
#include <mutex>
#include <string>

using namespace carat_hip;

struct carat_hip_runner {
  std::unique_ptr<BatchModelRunner> runner;
};

namespace {

thread_local std::string last_error;

template <typename F> int guarded(F &&body) {
  try {
    body();
    return 0;
  } catch (const std::exception &error) {
    last_error = error.what();
    return 1;
  } catch (...) {
    last_error = "unknown error";
    return 1;
  }
}

// Op-level workspaces (argmax partial keys, GEMM activation operands, attention partials), one
// set per device, grown on demand. Growing synchronises the device first so no launch still
// reads the old buffer.
struct OpWorkspace {
  void *keys = nullptr;
  size_t key_bytes = 0;
  void *partials = nullptr;
  size_t partial_bytes = 0;
  void *xprep = nullptr;          // e4m3 activation operand of a standalone linear
  size_t xprep_bytes = 0;
  void *packed_weight = nullptr;  // the row-major weight of a standalone linear, packed
  size_t packed_weight_bytes = 0;
  void *amax = nullptr;           // striped amax of a split attention call
  size_t amax_bytes = 0;
  void *x_scales = nullptr;       // activation scales of a channel / block_128 linear
  size_t x_scale_bytes = 0;
};
constexpr int kOpAmaxStripes = 64;
std::mutex workspace_mutex;
std::map<int, OpWorkspace> workspaces;

OpWorkspace &workspace_for_current_device() {
  int device = 0;
  hip_check(hipGetDevice(&device), "get device");
  return workspaces[device];
}

void ensure(void *&buffer, size_t &have, size_t need, const char *what) {
  if (need <= have) return;
  hip_check(hipDeviceSynchronize(), "synchronise before workspace growth");
  if (buffer != nullptr) (void)hipFree(buffer);
  buffer = nullptr;
  hip_check(hipMalloc(&buffer, need), what);
  have = need;
}

ModelSpec spec_from_desc(const carat_hip_model_desc *d) {
  if (d == nullptr || d->layers == nullptr || d->layer_count <= 0)
    throw std::runtime_error("invalid model description");
  ModelSpec spec;
  spec.hidden = d->hidden;
  spec.intermediate = d->intermediate;
  spec.vocabulary = d->vocabulary;
  spec.sliding_window = d->sliding_window;
  spec.eps = d->rms_norm_epsilon;
  for (int i = 0; i < d->layer_count; ++i) {
    LayerSpec l;
    l.sliding = d->layers[i].sliding != 0;
    l.query_heads = d->layers[i].query_heads;
    l.kv_heads = d->layers[i].kv_heads;
    l.head_dimension = d->layers[i].head_dimension;
    l.key_equals_value = d->layers[i].key_equals_value != 0;
    spec.layers.push_back(l);
  }
  spec.assistant.enabled = d->assistant != 0;
  spec.assistant.hidden = d->assistant_hidden;
  spec.assistant.intermediate = d->assistant_intermediate;
  spec.assistant.layers = d->assistant_layers;
  spec.assistant.query_heads = d->assistant_query_heads;
  if (d->assistant_fp8_mode < 0 || d->assistant_fp8_mode > 3)
    throw std::runtime_error("assistant_fp8_mode must be 0 (environment), 1 off, 2 lm_head or 3 all");
  spec.assistant.fp8_mode = d->assistant_fp8_mode - 1;
  if (d->fp8_scaling < 0 || d->fp8_scaling > 2)
    throw std::runtime_error("fp8_scaling must be 0 tensor, 1 channel or 2 block_128");
  spec.fp8_scaling = d->fp8_scaling;
  spec.seed = d->seed;
  spec.weight_std = d->weight_std;
  return spec;
}

BatchModelRunner &runner_of(carat_hip_runner *r) {
  if (r == nullptr || !r->runner) throw std::runtime_error("null runner handle");
  return *r->runner;
}

__global__ void convert_e4m3_kernel(const float *in, uint8_t *out, int64_t n) {
  const int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  if (i < n) out[i] = static_cast<uint8_t>(f32x2_to_e4m3x2(in[i], 0.0f) & 0xffu);
}

}  // namespace

extern "C" {

const char *carat_hip_last_error(void) { return last_error.c_str(); }

int carat_hip_device_count(int *count) {
  return guarded([&] { hip_check(hipGetDeviceCount(count), "count devices"); });
}

int carat_hip_synchronize(void) {
  return guarded([&] { hip_check(hipDeviceSynchronize(), "synchronize device"); });
}

int carat_hip_acceptance_cap(int depth, int remaining, const int32_t *proposals,
                             int proposal_count, const int32_t *stop_ids, int stop_count,
                             int *cap_out) {
  return guarded([&] {
    if (cap_out == nullptr || proposal_count < 0 || stop_count < 0 ||
        (proposal_count > 0 && proposals == nullptr) || (stop_count > 0 && stop_ids == nullptr))
      throw std::runtime_error("invalid acceptance cap arguments");
    const std::unordered_set<int> stops(stop_ids, stop_ids + stop_count);
    *cap_out = acceptance_cap(depth, remaining,
                              std::span<const int>(proposals, static_cast<size_t>(proposal_count)),
                              stops);
  });
}

int carat_hip_commit_speculation(int forced_token, const int32_t *accepted_drafts,
                                 int accepted_count, int next_token, const int32_t *stop_ids,
                                 int stop_count, int32_t *resident, int *resident_count,
                                 int32_t *emitted, int *emitted_count, int32_t *next_out,
                                 int *stopped) {
  return guarded([&] {
    if (accepted_count < 0 || stop_count < 0 || resident == nullptr || emitted == nullptr ||
        resident_count == nullptr || emitted_count == nullptr || next_out == nullptr ||
        stopped == nullptr)
      throw std::runtime_error("invalid speculative commit arguments");
    const std::unordered_set<int> stops(stop_ids, stop_ids + stop_count);
    const SpeculativeCommit commit = commit_speculation(
        forced_token, std::span<const int>(accepted_drafts, static_cast<size_t>(accepted_count)),
        next_token, stops);
    std::copy(commit.resident_tokens.begin(), commit.resident_tokens.end(), resident);
    std::copy(commit.emitted_tokens.begin(), commit.emitted_tokens.end(), emitted);
    *resident_count = static_cast<int>(commit.resident_tokens.size());
    *emitted_count = static_cast<int>(commit.emitted_tokens.size());
    *next_out = commit.next_token;
    *stopped = commit.stopped ? 1 : 0;
  });
}

int carat_hip_gemma4_benchmark_desc(carat_hip_model_desc *desc, carat_hip_layer_desc *layers,
                                    int with_assistant) {
  return guarded([&] {
    if (desc == nullptr || layers == nullptr) throw std::runtime_error("null description");
    const ModelSpec spec = gemma4_31b_benchmark_spec(with_assistant != 0);
    for (size_t i = 0; i < spec.layers.size(); ++i) {
      layers[i].sliding = spec.layers[i].sliding ? 1 : 0;
      layers[i].query_heads = spec.layers[i].query_heads;
      layers[i].kv_heads = spec.layers[i].kv_heads;
      layers[i].head_dimension = spec.layers[i].head_dimension;
      layers[i].key_equals_value = spec.layers[i].key_equals_value ? 1 : 0;
    }
    desc->hidden = spec.hidden;
    desc->intermediate = spec.intermediate;
    desc->vocabulary = spec.vocabulary;
    desc->sliding_window = spec.sliding_window;
    desc->rms_norm_epsilon = spec.eps;
    desc->layer_count = static_cast<int>(spec.layers.size());
    desc->layers = layers;
    desc->assistant = spec.assistant.enabled ? 1 : 0;
    desc->assistant_hidden = spec.assistant.hidden;
    desc->assistant_intermediate = spec.assistant.intermediate;
    desc->assistant_layers = spec.assistant.layers;
    desc->assistant_query_heads = spec.assistant.query_heads;
    desc->seed = spec.seed;
    desc->weight_std = spec.weight_std;
    desc->fp8_scaling = spec.fp8_scaling;
  });
}

int carat_hip_runner_create(const carat_hip_model_desc *desc, int batch, int maximum_context,
                            carat_hip_runner **out) {
  return guarded([&] {
    if (out == nullptr) throw std::runtime_error("null output handle");
    auto handle = std::make_unique<carat_hip_runner>();
    handle->runner = std::make_unique<BatchModelRunner>(spec_from_desc(desc), batch, maximum_context);
    *out = handle.release();
  });
}

int carat_hip_runner_create_from_device_weights(const carat_hip_model_desc *desc,
                                                carat_hip_device_segment_fn segment,
                                                void *context, int batch, int maximum_context,
                                                carat_hip_runner **out) {
  return guarded([&] {
    if (out == nullptr) throw std::runtime_error("null output handle");
    if (segment == nullptr) throw std::runtime_error("missing device weight lookup");
    auto handle = std::make_unique<carat_hip_runner>();
    handle->runner = std::make_unique<BatchModelRunner>(spec_from_desc(desc), segment, context,
                                                        batch, maximum_context);
    *out = handle.release();
  });
}

int carat_hip_checkpoint_describe(const char *model_dir, const char *assistant_dir,
                                  carat_hip_model_desc *desc, carat_hip_layer_desc *layers,
                                  int layer_capacity, uint64_t *target_bytes,
                                  uint64_t *assistant_bytes) {
  return guarded([&] {
    if (model_dir == nullptr || desc == nullptr) throw std::runtime_error("null checkpoint argument");
    const Checkpoint checkpoint =
        Checkpoint::open(model_dir, assistant_dir == nullptr ? std::string() : assistant_dir);
    ModelSpec spec;
    checkpoint.describe(spec);
    const int count = static_cast<int>(spec.layers.size());
    if (layers != nullptr && layer_capacity < count)
      throw std::runtime_error("layer array too small: checkpoint has " + std::to_string(count) +
                               " layers");
    *desc = carat_hip_model_desc{};
    desc->hidden = spec.hidden;
    desc->intermediate = spec.intermediate;
    desc->vocabulary = spec.vocabulary;
    desc->sliding_window = spec.sliding_window;
    desc->rms_norm_epsilon = spec.eps;
    desc->layer_count = count;
    desc->layers = layers;
    desc->assistant = spec.assistant.enabled ? 1 : 0;
    desc->assistant_hidden = spec.assistant.hidden;
    desc->assistant_intermediate = spec.assistant.intermediate;
    desc->assistant_layers = spec.assistant.layers;
    desc->assistant_query_heads = spec.assistant.query_heads;
    if (layers != nullptr)
      for (int i = 0; i < count; ++i) {
        const LayerSpec &l = spec.layers[static_cast<size_t>(i)];
        layers[i] = carat_hip_layer_desc{l.sliding ? 1 : 0, l.query_heads, l.kv_heads,
                                         l.head_dimension, l.key_equals_value ? 1 : 0};
      }
    if (target_bytes != nullptr) *target_bytes = checkpoint.target_plan.bytes();
    if (assistant_bytes != nullptr)
      *assistant_bytes = checkpoint.has_assistant ? checkpoint.assistant_plan.bytes() : 0;
  });
}

int carat_hip_runner_create_from_checkpoint(const char *model_dir, const char *assistant_dir,
                                            int batch, int maximum_context,
                                            carat_hip_runner **out) {
  return guarded([&] {
    if (out == nullptr || model_dir == nullptr) throw std::runtime_error("null checkpoint argument");
    const Checkpoint checkpoint =
        Checkpoint::open(model_dir, assistant_dir == nullptr ? std::string() : assistant_dir);
    auto handle = std::make_unique<carat_hip_runner>();
    handle->runner = std::make_unique<BatchModelRunner>(checkpoint, batch, maximum_context);
    *out = handle.release();
  });
}

void carat_hip_runner_destroy(carat_hip_runner *runner) { delete runner; }

int carat_hip_runner_last_predictions(carat_hip_runner *runner, int32_t *out, int capacity,
                                      int *count) {
  return guarded([&] {
    const auto &p = runner_of(runner).last_predictions();
    if (count == nullptr || (out == nullptr && capacity > 0)) throw std::runtime_error("null output");
    *count = static_cast<int>(p.size());
    std::copy(p.begin(), p.begin() + std::min<size_t>(p.size(), static_cast<size_t>(std::max(capacity, 0))), out);
  });
}

int carat_hip_runner_prefill_slot(carat_hip_runner *runner, int slot, const int32_t *tokens,
                                  int count, int chunk_tokens, int32_t *next_token) {
  return guarded([&] {
    if (count < 0 || (count > 0 && tokens == nullptr) || next_token == nullptr)
      throw std::runtime_error("invalid slot prefill shape");
    const std::vector<int> prompt(tokens, tokens + count);
    *next_token = runner_of(runner).prefill_slot(slot, prompt, chunk_tokens);
  });
}

int carat_hip_runner_prefill_slots_chunks(carat_hip_runner *runner, int requests,
                                          const int32_t *slots, const int32_t *offsets,
                                          const int32_t *tokens, int chunk_tokens,
                                          int32_t *predictions) {
  return guarded([&] {
    if (requests <= 0 || slots == nullptr || offsets == nullptr || tokens == nullptr ||
        predictions == nullptr)
      throw std::runtime_error("invalid slot prefill chunk shape");
    std::vector<std::vector<int>> prompts(static_cast<size_t>(requests));
    std::vector<const std::vector<int> *> pointers;
    for (int r = 0; r < requests; ++r) {
      if (offsets[r + 1] < offsets[r]) throw std::runtime_error("invalid slot prefill chunk shape");
      prompts[static_cast<size_t>(r)].assign(tokens + offsets[r], tokens + offsets[r + 1]);
      pointers.push_back(&prompts[static_cast<size_t>(r)]);
    }
    const std::vector<int> s(slots, slots + requests);
    const auto result = runner_of(runner).prefill_slots_chunks(s, pointers, chunk_tokens);
    for (int r = 0; r < requests; ++r)
      predictions[r] = result[static_cast<size_t>(r)] ? *result[static_cast<size_t>(r)] : -1;
  });
}

namespace {
// Request r's prompt is tokens[offsets[r] .. offsets[r+1]).
void unpack_prompts(int requests, const int32_t *slots, const int32_t *offsets,
                    const int32_t *tokens, const char *message, std::vector<int> &slot_list,
                    std::vector<std::vector<int>> &prompts,
                    std::vector<const std::vector<int> *> &pointers) {
  if (requests <= 0 || slots == nullptr || offsets == nullptr || tokens == nullptr)
    throw std::runtime_error(message);
  prompts.assign(static_cast<size_t>(requests), {});
  pointers.clear();
  for (int r = 0; r < requests; ++r) {
    if (offsets[r] < 0 || offsets[r + 1] < offsets[r]) throw std::runtime_error(message);
    prompts[static_cast<size_t>(r)].assign(tokens + offsets[r], tokens + offsets[r + 1]);
    pointers.push_back(&prompts[static_cast<size_t>(r)]);
  }
  slot_list.assign(slots, slots + requests);
}
}  // namespace

int carat_hip_runner_prefill_slot_from_prefix(carat_hip_runner *runner, int slot,
                                              const int32_t *tokens, int count, int cached_prefix,
                                              int chunk_tokens, int32_t *next_token) {
  return guarded([&] {
    if (count < 0 || (count > 0 && tokens == nullptr) || next_token == nullptr)
      throw std::runtime_error("invalid slot prefill shape");
    const std::vector<int> prompt(tokens, tokens + count);
    *next_token = runner_of(runner).prefill_slot_from_prefix(slot, prompt, cached_prefix, chunk_tokens);
  });
}

int carat_hip_runner_prefill_slot_chunk(carat_hip_runner *runner, int slot, const int32_t *tokens,
                                        int count, int chunk_tokens, int32_t *next_token) {
  return guarded([&] {
    if (count < 0 || (count > 0 && tokens == nullptr) || next_token == nullptr)
      throw std::runtime_error("invalid slot prefill chunk shape");
    const std::vector<int> prompt(tokens, tokens + count);
    const auto result = runner_of(runner).prefill_slot_chunk(slot, prompt, chunk_tokens);
    *next_token = result ? *result : -1;
  });
}

int carat_hip_runner_prefill_slots_suffix(carat_hip_runner *runner, int requests,
                                          const int32_t *slots, const int32_t *offsets,
                                          const int32_t *tokens, int32_t *predictions) {
  return guarded([&] {
    std::vector<int> slot_list;
    std::vector<std::vector<int>> prompts;
    std::vector<const std::vector<int> *> pointers;
    if (predictions == nullptr) throw std::runtime_error("invalid batched suffix prefill shape");
    unpack_prompts(requests, slots, offsets, tokens, "invalid batched suffix prefill shape",
                   slot_list, prompts, pointers);
    const auto result = runner_of(runner).prefill_slots_suffix(slot_list, pointers);
    std::copy(result.begin(), result.end(), predictions);
  });
}

int carat_hip_runner_prefill_slots_suffix_layer_slice(carat_hip_runner *runner, int requests,
                                                      const int32_t *slots, const int32_t *offsets,
                                                      const int32_t *tokens, int maximum_layers,
                                                      int *complete, int32_t *predictions) {
  return guarded([&] {
    std::vector<int> slot_list;
    std::vector<std::vector<int>> prompts;
    std::vector<const std::vector<int> *> pointers;
    if (complete == nullptr || predictions == nullptr)
      throw std::runtime_error("invalid layer-sliced suffix prefill shape");
    unpack_prompts(requests, slots, offsets, tokens, "invalid layer-sliced suffix prefill shape",
                   slot_list, prompts, pointers);
    const auto result =
        runner_of(runner).prefill_slots_suffix_layer_slice(slot_list, pointers, maximum_layers);
    *complete = result.complete ? 1 : 0;
    if (result.complete) std::copy(result.predictions.begin(), result.predictions.end(), predictions);
  });
}

int carat_hip_runner_abort_suffix_layer_slices(carat_hip_runner *runner) {
  return guarded([&] { runner_of(runner).abort_suffix_layer_slices(); });
}

int carat_hip_runner_has_suffix_layer_slices(carat_hip_runner *runner, int *out) {
  return guarded([&] {
    if (out == nullptr) throw std::runtime_error("null output");
    *out = runner_of(runner).has_suffix_layer_slices() ? 1 : 0;
  });
}

int carat_hip_runner_clone_slot(carat_hip_runner *runner, int source_slot, int destination_slot,
                                uint64_t *copied_bytes) {
  return guarded([&] {
    const uint64_t copied = runner_of(runner).clone_slot(source_slot, destination_slot);
    if (copied_bytes != nullptr) *copied_bytes = copied;
  });
}

int carat_hip_runner_append(carat_hip_runner *runner, const int32_t *tokens, int count,
                            int32_t *next_tokens) {
  return guarded([&] {
    if (count < 0 || (count > 0 && tokens == nullptr) || next_tokens == nullptr)
      throw std::runtime_error("token batch has the wrong size");
    const std::vector<int> next = runner_of(runner).append(std::vector<int>(tokens, tokens + count));
    std::copy(next.begin(), next.end(), next_tokens);
  });
}

int carat_hip_runner_verify(carat_hip_runner *runner, int requests, int depth,
                            const int32_t *proposals, const int32_t *target_first,
                            const int32_t *slots, const int32_t *caps, int32_t *accepted_out,
                            int32_t *next_out, int32_t *predictions_out) {
  return guarded([&] {
    auto &r = runner_of(runner);
    if (requests < 0 || depth < 0 || (requests > 0 && (proposals == nullptr ||
                                                       target_first == nullptr || slots == nullptr)))
      throw std::runtime_error("invalid greedy verification batch");
    std::vector<std::vector<int>> rows(static_cast<size_t>(requests));
    for (int i = 0; i < requests; ++i)
      rows[static_cast<size_t>(i)].assign(proposals + static_cast<size_t>(i) * depth,
                                          proposals + static_cast<size_t>(i + 1) * depth);
    const std::vector<int> first(target_first, target_first + requests);
    const std::vector<int> slot_list(slots, slots + requests);
    std::vector<int> cap_list;
    if (caps != nullptr) cap_list.assign(caps, caps + requests);
    const GreedyVerificationResult result = r.verify_greedy_proposals(rows, first, slot_list, cap_list);
    if (accepted_out != nullptr) std::copy(result.accepted_tokens.begin(), result.accepted_tokens.end(), accepted_out);
    if (next_out != nullptr) std::copy(result.next_tokens.begin(), result.next_tokens.end(), next_out);
    if (predictions_out != nullptr) std::copy(r.last_predictions().begin(), r.last_predictions().end(), predictions_out);
  });
}

int carat_hip_bench_speculative_cycle(carat_hip_runner *runner, int requests, int depth,
                                      const int32_t *last_tokens, const int32_t *slots,
                                      const int32_t *forced, const int32_t *planted,
                                      int remaining, const int32_t *stop_ids, int stop_count,
                                      int32_t *accepted_out, int32_t *next_out,
                                      int32_t *last_out, double *seconds_out) {
  return guarded([&] {
    auto &r = runner_of(runner);
    if (requests <= 0 || depth <= 0 || last_tokens == nullptr || slots == nullptr ||
        forced == nullptr || planted == nullptr || accepted_out == nullptr ||
        next_out == nullptr || last_out == nullptr || seconds_out == nullptr ||
        (stop_count > 0 && stop_ids == nullptr))
      throw std::runtime_error("invalid speculative cycle arguments");
    const std::unordered_set<int> stops(stop_ids, stop_ids + std::max(stop_count, 0));
    const std::vector<int> last(last_tokens, last_tokens + requests);
    const std::vector<int> slot_list(slots, slots + requests);
    const std::vector<int> first(forced, forced + requests);
    std::vector<std::vector<int>> proposals(static_cast<size_t>(requests));
    for (int i = 0; i < requests; ++i) {
      proposals[static_cast<size_t>(i)].assign(planted + static_cast<size_t>(i) * depth,
                                               planted + static_cast<size_t>(i + 1) * depth);
      // the scheduler's proposals start with the token it forces (native_runtime_main.cpp:597-604)
      if (planted[static_cast<size_t>(i) * depth] != forced[i])
        throw std::runtime_error("planted proposals must start with the forced token");
    }
    hip_check(hipDeviceSynchronize(), "synchronise before the speculative cycle");
    const auto start = std::chrono::steady_clock::now();
    // native_runtime_main.cpp:583-678: draft, caps from the proposals, verify, commit. The
    // proposals verified are the planted ones (they replace the drafts), so the caps are taken
    // from them, as the reference takes them from the drafts it verifies.
    const auto drafts = r.draft_four(last, slot_list, first, depth);
    if (drafts.size() != static_cast<size_t>(requests))
      throw std::runtime_error("draft returned the wrong number of rows");
    std::vector<int> caps(static_cast<size_t>(requests));
    for (int i = 0; i < requests; ++i)
      caps[static_cast<size_t>(i)] = acceptance_cap(depth, remaining, proposals[static_cast<size_t>(i)], stops);
    const GreedyVerificationResult result = r.verify_greedy_proposals(proposals, first, slot_list, caps);
    // Rows that accepted nothing append their forced token in one ragged decode step
    // (native_runtime_main.cpp:636-646), which also yields their next token.
    std::vector<int> fallback_slots, fallback_tokens;
    for (int i = 0; i < requests; ++i)
      if (result.accepted_tokens[static_cast<size_t>(i)] == 0) {
        fallback_slots.push_back(slot_list[static_cast<size_t>(i)]);
        fallback_tokens.push_back(first[static_cast<size_t>(i)]);
      }
    std::vector<int> fallback_next;
    if (!fallback_slots.empty()) fallback_next = r.append_ragged(fallback_tokens, fallback_slots);
    size_t fallback_index = 0;
    for (int i = 0; i < requests; ++i) {
      const int a = result.accepted_tokens[static_cast<size_t>(i)];
      const auto &row = proposals[static_cast<size_t>(i)];
      const std::span<const int> accepted_drafts(row.data() + 1, a > 1 ? static_cast<size_t>(a - 1) : 0);
      const int next_token =
          a == 0 ? fallback_next.at(fallback_index++) : result.next_tokens[static_cast<size_t>(i)];
      const SpeculativeCommit commit =
          commit_speculation(first[static_cast<size_t>(i)], accepted_drafts, next_token, stops);
      accepted_out[i] = a;
      next_out[i] = commit.next_token;
      last_out[i] = commit.resident_tokens.back();
    }
    *seconds_out = std::chrono::duration<double>(std::chrono::steady_clock::now() - start).count();
  });
}

int carat_hip_runner_append_ragged(carat_hip_runner *runner, int rows, const int32_t *tokens,
                                   const int32_t *slots, int32_t *next_tokens) {
  return guarded([&] {
    if (rows < 0 || (rows > 0 && (tokens == nullptr || slots == nullptr || next_tokens == nullptr)))
      throw std::runtime_error("invalid ragged token batch");
    const std::vector<int> token_ids(tokens, tokens + rows);
    const std::vector<int> slot_ids(slots, slots + rows);
    const std::vector<int> next = runner_of(runner).append_ragged(token_ids, slot_ids);
    std::copy(next.begin(), next.end(), next_tokens);
  });
}

int carat_hip_runner_draft(carat_hip_runner *runner, int rows, int depth, const int32_t *last,
                           const int32_t *slots, const int32_t *forced, int32_t *proposals_out) {
  return guarded([&] {
    auto &r = runner_of(runner);
    if (rows < 0 || (rows > 0 && (last == nullptr || slots == nullptr)) || proposals_out == nullptr)
      throw std::runtime_error("assistant is not configured or draft batch is invalid");
    const std::vector<int> last_list(last, last + rows);
    const std::vector<int> slot_list(slots, slots + rows);
    std::vector<int> forced_list;
    if (forced != nullptr) forced_list.assign(forced, forced + rows);
    const auto proposals = r.draft_four(last_list, slot_list, forced_list, depth);
    for (size_t i = 0; i < proposals.size(); ++i)
      std::copy(proposals[i].begin(), proposals[i].end(), proposals_out + i * static_cast<size_t>(depth));
  });
}

int carat_hip_runner_has_assistant(carat_hip_runner *runner, int *out) {
  return guarded([&] { *out = runner_of(runner).has_assistant() ? 1 : 0; });
}
int carat_hip_runner_batch(carat_hip_runner *runner, int *out) {
  return guarded([&] { *out = runner_of(runner).batch(); });
}
int carat_hip_runner_position(carat_hip_runner *runner, int *out) {
  return guarded([&] { *out = runner_of(runner).position(); });
}
int carat_hip_runner_slot_position(carat_hip_runner *runner, int slot, int *out) {
  return guarded([&] { *out = runner_of(runner).slot_position(slot); });
}
int carat_hip_runner_reset_slot(carat_hip_runner *runner, int slot) {
  return guarded([&] { runner_of(runner).reset_slot(slot); });
}
int carat_hip_runner_seed_empty_cache_for_benchmark(carat_hip_runner *runner, int position) {
  return guarded([&] { runner_of(runner).seed_empty_cache_for_benchmark(position); });
}
int carat_hip_runner_seed_random_cache(carat_hip_runner *runner, int position, uint64_t seed,
                                       float stddev) {
  return guarded([&] { runner_of(runner).seed_random_cache_for_benchmark(position, seed, stddev); });
}
int carat_hip_runner_set_slot_position(carat_hip_runner *runner, int slot, int position) {
  return guarded([&] { runner_of(runner).set_slot_position(slot, position); });
}
int carat_hip_runner_tensor(carat_hip_runner *runner, const char *name, void **device_ptr,
                            size_t *bytes) {
  return guarded([&] {
    if (name == nullptr || device_ptr == nullptr) throw std::runtime_error("invalid tensor query");
    *device_ptr = runner_of(runner).tensor(name, bytes);
  });
}
int carat_hip_runner_copy_tensor(carat_hip_runner *runner, const char *name, void *host,
                                 size_t bytes, int direction) {
  return guarded([&] {
    auto &r = runner_of(runner);
    size_t size = 0;
    WeightLayout layout;
    void *device = r.tensor(name, &size, &layout);
    if (host == nullptr || bytes != size) throw std::runtime_error("tensor copy size mismatch");
    hip_check(hipStreamSynchronize(r.stream()), "synchronize runner");
    if (layout.n == 0) {
      if (direction == 0)
        hip_check(hipMemcpy(host, device, bytes, hipMemcpyDeviceToHost), "copy tensor to host");
      else
        hip_check(hipMemcpy(device, host, bytes, hipMemcpyHostToDevice), "copy tensor to device");
      return;
    }
    // Packed weights travel in their logical row-major [n][row_bytes] order.
    void *row_major = nullptr;
    hip_check(hipMalloc(&row_major, bytes), "allocate weight staging");
    try {
      if (direction == 0) {
        unpack_weight(device, row_major, layout, r.stream());
        hip_check(hipStreamSynchronize(r.stream()), "unpack weight");
        hip_check(hipMemcpy(host, row_major, bytes, hipMemcpyDeviceToHost), "copy tensor to host");
      } else {
        hip_check(hipMemcpy(row_major, host, bytes, hipMemcpyHostToDevice), "copy tensor to device");
        pack_weight(row_major, device, layout, r.stream());
        hip_check(hipStreamSynchronize(r.stream()), "pack weight");
      }
    } catch (...) {
      (void)hipFree(row_major);
      throw;
    }
    hip_check(hipFree(row_major), "free weight staging");
  });
}
int carat_hip_runner_set_graphs(carat_hip_runner *runner, int enabled) {
  return guarded([&] { runner_of(runner).set_graphs_enabled(enabled != 0); });
}

int carat_hip_runner_set_qkv_fusion(carat_hip_runner *runner, int enabled) {
  return guarded([&] { runner_of(runner).set_qkv_fusion(enabled != 0); });
}
int carat_hip_runner_set_fused_quantization(carat_hip_runner *runner, int enabled) {
  return guarded([&] { runner_of(runner).set_fused_quantization(enabled); });
}
int carat_hip_runner_set_probe(carat_hip_runner *runner, int kind) {
  return guarded([&] { runner_of(runner).set_probe(kind); });
}
int carat_hip_runner_stream_gemm_probe(carat_hip_runner *runner, int kind, int passes,
                                       float *avg_ms, int *launches) {
  return guarded([&] {
    if (avg_ms == nullptr || launches == nullptr) throw std::runtime_error("null probe output");
    *avg_ms = runner_of(runner).stream_gemm_probe(kind, passes, launches);
  });
}
int carat_hip_runner_read_probe(carat_hip_runner *runner, float *total_ms, int *launches) {
  return guarded([&] {
    if (total_ms == nullptr || launches == nullptr) throw std::runtime_error("null probe output");
    runner_of(runner).read_probe(total_ms, launches);
  });
}
int carat_hip_runner_timing(carat_hip_runner *runner, float *verify_ms, float *draft_ms) {
  return guarded([&] {
    auto &r = runner_of(runner);
    if (verify_ms != nullptr) *verify_ms = r.last_verify_ms();
    if (draft_ms != nullptr) *draft_ms = r.last_draft_ms();
  });
}

int carat_hip_argmax_accept(const float *logits_f32, const uint16_t *logits_bf16, int requests,
                            int tokens, int vocabulary, const int32_t *proposals,
                            const int32_t *target_first, const int32_t *caps,
                            int32_t *predictions, int32_t *accepted, int32_t *next_tokens,
                            void *stream) {
  return guarded([&] {
    std::lock_guard<std::mutex> lock(workspace_mutex);
    OpWorkspace &w = workspace_for_current_device();
    const size_t keys = static_cast<size_t>(argmax_accept_chunks(vocabulary, logits_f32 != nullptr)) *
                        static_cast<size_t>(std::max(requests, 0)) * static_cast<size_t>(std::max(tokens, 0));
    ensure(w.keys, w.key_bytes, keys * sizeof(uint64_t), "allocate argmax partials");
    ArgmaxAcceptArgs a;
    a.logits_f32 = logits_f32;
    a.logits_bf16 = logits_bf16;
    a.requests = requests;
    a.tokens = tokens;
    a.vocabulary = vocabulary;
    a.proposals = proposals;
    a.target_first = target_first;
    a.caps = caps;
    a.predictions = predictions;
    a.accepted = accepted;
    a.next_tokens = next_tokens;
    a.partials = static_cast<uint64_t *>(w.keys);
    a.partial_capacity = w.key_bytes / sizeof(uint64_t);
    launch_argmax_accept(a, static_cast<hipStream_t>(stream));
  });
}

// Allocation-free argmax + acceptance: the partial keys live in a file-scope device array of
// fixed size instead of a workspace the library allocates. Each device holds its own copy;
// host code reaches it only through the address hipGetSymbolAddress returns on that device
// (the array's name is a host-side stand-in, not a device address). Every call on one device
// shares the array, so calls that overlap on one device race. The partial kernel writes every
// key the final kernel reads, so nothing needs clearing between calls.
constexpr size_t kNoAllocArgmaxKeys = 65536;  // 512 KiB: e.g. 256 requests x 8 rows x 32 chunks
static __device__ __align__(256) uint64_t scratch[kNoAllocArgmaxKeys];
constexpr int kNoAllocMaxDevices = 64;
std::mutex scratch_mutex;
uint64_t *scratch_by_device[kNoAllocMaxDevices] = {};

uint64_t *scratch_for_current_device() {
  int device = 0;
  hip_check(hipGetDevice(&device), "get device");
  if (device < 0 || device >= kNoAllocMaxDevices)
    throw std::runtime_error("allocation-free argmax: device index out of range");
  std::lock_guard<std::mutex> lock(scratch_mutex);
  if (scratch_by_device[device] == nullptr) {
    void *address = nullptr;
    hip_check(hipGetSymbolAddress(&address, HIP_SYMBOL(scratch)),
              "resolve the allocation-free argmax scratch");
    scratch_by_device[device] = static_cast<uint64_t *>(address);
  }
  return scratch_by_device[device];
}

int carat_hip_argmax_accept_noalloc(const float *logits_f32, const uint16_t *logits_bf16,
                                    int requests, int tokens, int vocabulary,
                                    const int32_t *proposals, const int32_t *target_first,
                                    const int32_t *caps, int32_t *predictions, int32_t *accepted,
                                    int32_t *next_tokens, void *stream) {
  return guarded([&] {
    if (requests <= 0 || tokens <= 0 || vocabulary <= 0)
      throw std::runtime_error("invalid argmax arguments");
    const size_t keys = static_cast<size_t>(argmax_accept_chunks(vocabulary, logits_f32 != nullptr)) *
                        static_cast<size_t>(requests) * static_cast<size_t>(tokens);
    if (keys > kNoAllocArgmaxKeys)
      throw std::runtime_error("allocation-free argmax: " + std::to_string(keys) +
                               " partial keys exceed the fixed scratch of " +
                               std::to_string(kNoAllocArgmaxKeys));
    ArgmaxAcceptArgs a;
    a.logits_f32 = logits_f32;
    a.logits_bf16 = logits_bf16;
    a.requests = requests;
    a.tokens = tokens;
    a.vocabulary = vocabulary;
    a.proposals = proposals;
    a.target_first = target_first;
    a.caps = caps;
    a.predictions = predictions;
    a.accepted = accepted;
    a.next_tokens = next_tokens;
    a.partials = scratch_for_current_device();
    a.partial_capacity = kNoAllocArgmaxKeys;
    launch_argmax_accept(a, static_cast<hipStream_t>(stream));
  });
}

static int linear_common(bool fp8, const uint16_t *x, int m, int k, const float *x_amax,
                         const void *w, int n, const float *w_scale, int epilogue, int splits,
                         uint16_t *y, float *y_amax, float *partial, int32_t *predictions,
                         void *stream, int scaling = 0) {
  return guarded([&] {
    if (epilogue < 0 || epilogue > 3) throw std::runtime_error("invalid GEMM epilogue");
    if (scaling < 0 || scaling > 2) throw std::runtime_error("fp8_scaling must be 0, 1 or 2");
    GemmArgs g;
    g.x = x;
    g.ldx = k;
    g.m = m;
    g.k = k;
    g.x_amax = x_amax;
    g.n = n;
    g.w_scale = w_scale;
    g.k_splits = splits <= 0 ? 1 : splits;
    g.epilogue = static_cast<GemmEpilogue>(epilogue);
    g.y = y;
    g.ldy = g.epilogue == GemmEpilogue::gelu_gate ? n / 2 : n;
    g.y_amax = y_amax;
    g.partial = partial;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (m <= 0 || n <= 0 || k <= 0) throw std::runtime_error("invalid skinny GEMM shape");
    std::lock_guard<std::mutex> lock(workspace_mutex);
    OpWorkspace &ws = workspace_for_current_device();
    // The reference interface passes a row-major [n][k] weight; the kernels read the packed
    // storage layout, so the weight is packed into a workspace first (the runner packs once at
    // load time instead).
    if (fp8) {
      ensure(ws.xprep, ws.xprep_bytes, gemm_xprep_bytes(m, k), "allocate GEMM activation workspace");
      g.xprep = static_cast<unsigned char *>(ws.xprep);
      g.xprep_capacity = ws.xprep_bytes;
    }
    if (scaling != 0) {
      if (w_scale == nullptr) throw std::runtime_error("scaled FP8 linear needs weight scales");
      ensure(ws.x_scales, ws.x_scale_bytes, sizeof(float) * gemm_x_scale_floats(m, k),
             "allocate activation scale workspace");
      g.scaling = scaling;
      g.w_scales = w_scale;
      g.w_scale_kblocks = static_cast<int>(fp8_weight_scale_elements(2, n, k) / ((n + 127) / 128));
      g.x_scales = static_cast<float *>(ws.x_scales);
      g.x_scales_capacity = ws.x_scale_bytes / sizeof(float);
      g.w_scale = nullptr;
    }
    g.w_layout = gemm_weight_layout(n, k * (fp8 ? 1 : 2), g.epilogue == GemmEpilogue::gelu_gate);
    ensure(ws.packed_weight, ws.packed_weight_bytes,
           static_cast<size_t>(n) * k * (fp8 ? 1 : 2), "allocate packed weight workspace");
    pack_weight(w, ws.packed_weight, g.w_layout, s);
    g.w = ws.packed_weight;
    if (g.epilogue == GemmEpilogue::argmax) {
      if (predictions == nullptr) throw std::runtime_error("argmax GEMM needs predictions");
      ensure(ws.keys, ws.key_bytes, gemm_argmax_partials(m, g.w_layout) * sizeof(uint64_t),
             "allocate argmax partials");
      g.argmax_partials = static_cast<uint64_t *>(ws.keys);
      g.argmax_partial_capacity = ws.key_bytes / sizeof(uint64_t);
      g.argmax_out = predictions;
    }
    if (fp8) launch_fp8_gemm(g, s); else launch_bf16_gemm(g, s);
  });
}

int carat_hip_gemm_plan(int n, int k, int fp8, int gate_up, int *tiles_per_wave, int *waves,
                        int *splits) {
  return guarded([&] {
    if (n <= 0 || k <= 0) throw std::runtime_error("invalid skinny GEMM shape");
    const WeightLayout l = gemm_weight_layout(n, k * (fp8 ? 1 : 2), gate_up != 0);
    if (tiles_per_wave != nullptr) *tiles_per_wave = l.tiles_per_wave;
    if (waves != nullptr) *waves = l.waves;
    // gate/up feeds the GELU epilogue, which needs whole sums: it never splits K
    if (splits != nullptr)
      *splits = gate_up ? 1 : gemm_choose_splits(gemm_blocks_n(l), l.row_bytes / 128);
  });
}

int carat_hip_fp8_linear(const uint16_t *x, int m, int k, const float *x_amax, const uint8_t *w,
                         int n, const float *w_scale, int epilogue, int splits, uint16_t *y,
                         float *y_amax, float *partial, int32_t *predictions, void *stream) {
  return linear_common(true, x, m, k, x_amax, w, n, w_scale, epilogue, splits, y, y_amax, partial,
                       predictions, stream);
}

int carat_hip_fp8_linear_scaled(const uint16_t *x, int m, int k, int fp8_scaling, const uint8_t *w,
                                int n, const float *w_scales, int epilogue, int splits, uint16_t *y,
                                float *partial, int32_t *predictions, void *stream) {
  if (fp8_scaling != 1 && fp8_scaling != 2)
    return guarded([] { throw std::runtime_error("fp8_scaling must be 1 (channel) or 2 (block_128)"); });
  return linear_common(true, x, m, k, nullptr, w, n, w_scales, epilogue, splits, y, nullptr, partial,
                       predictions, stream, fp8_scaling);
}

int carat_hip_fp8_weight_scale_elements(int fp8_scaling, int n, int k, uint64_t *out) {
  return guarded([&] {
    if (out == nullptr || n <= 0 || k <= 0) throw std::runtime_error("invalid FP8 weight shape");
    *out = fp8_weight_scale_elements(fp8_scaling, n, k);
  });
}

int carat_hip_quantize_weight_fp8(const uint16_t *w, int n, int k, int fp8_scaling, uint8_t *out,
                                  float *scales, void *stream) {
  return guarded([&] {
    if (w == nullptr || out == nullptr || scales == nullptr)
      throw std::runtime_error("invalid FP8 weight quantization arguments");
    std::lock_guard<std::mutex> lock(workspace_mutex);
    OpWorkspace &ws = workspace_for_current_device();
    ensure(ws.amax, ws.amax_bytes, sizeof(float) * kOpAmaxStripes * 64, "allocate amax workspace");
    quantize_weight_bf16_to_fp8_scaled(w, reinterpret_cast<fp8_t *>(out), n, k, fp8_scaling, scales,
                                       static_cast<float *>(ws.amax), static_cast<hipStream_t>(stream));
  });
}

int carat_hip_bf16_linear(const uint16_t *x, int m, int k, const uint16_t *w, int n, int epilogue,
                          int splits, uint16_t *y, float *y_amax, float *partial,
                          int32_t *predictions, void *stream) {
  return linear_common(false, x, m, k, nullptr, w, n, nullptr, epilogue, splits, y, y_amax,
                       partial, predictions, stream);
}

int carat_hip_verify_attention(int mode, const uint16_t *q, const void *k_cache,
                               const void *v_cache, const void *k_new, const void *v_new,
                               int fp8_kv, float k_scale, float v_scale, const int32_t *slots,
                               const int32_t *positions, int requests, int tokens,
                               int query_heads, int kv_heads, int dimension, int capacity,
                               int window, int max_keys, uint16_t *out, float *out_amax,
                               int chunk_keys, void *stream) {
  return guarded([&] {
    if (mode < 0 || mode > 2) throw std::runtime_error("invalid attention mode");
    AttentionArgs a;
    a.mode = static_cast<AttentionMode>(mode);
    a.q = q;
    a.k_cache = k_cache;
    a.v_cache = v_cache;
    a.k_new = k_new;
    a.v_new = v_new;
    a.fp8_kv = fp8_kv != 0;
    a.k_scale = k_scale;
    a.v_scale = v_scale;
    a.slots = slots;
    a.positions = positions;
    a.requests = requests;
    a.tokens = tokens;
    a.query_heads = query_heads;
    a.kv_heads = kv_heads;
    a.dimension = dimension;
    a.capacity = capacity;
    a.window = window;
    a.max_keys = max_keys;
    a.out = out;
    a.out_amax = out_amax;
    a.chunk_keys = chunk_keys > 0 ? chunk_keys
                                  : attention_default_chunk(a.mode, max_keys, requests, kv_heads, a.fp8_kv,
                                                            dimension);
    std::lock_guard<std::mutex> lock(workspace_mutex);
    OpWorkspace &w = workspace_for_current_device();
    if (kv_heads <= 0 || requests <= 0 || max_keys <= 0)
      throw std::runtime_error("invalid verify attention shape");
    const int qrows = query_heads / kv_heads * tokens;
    ensure(w.partials, w.partial_bytes,
           sizeof(float) * attention_partials_floats(requests, kv_heads, max_keys, a.chunk_keys,
                                                     qrows, dimension),
           "allocate attention partials");
    a.partials = static_cast<float *>(w.partials);
    // A split range ends in a merge kernel whose workgroups all finish at once: their amax updates
    // go to striped slots (zeroed first), folded into the caller's float afterwards, instead of
    // queueing on one address.
    const bool split = (max_keys + a.chunk_keys - 1) / a.chunk_keys > 1;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (split && out_amax != nullptr) {
      ensure(w.amax, w.amax_bytes, sizeof(float) * kOpAmaxStripes * kAmaxStripeFloats,
             "allocate attention amax stripes");
      a.out_amax = static_cast<float *>(w.amax);
      a.amax_stripes = kOpAmaxStripes;
      launch_step_init(a.out_amax, kOpAmaxStripes, s);
    }
    launch_attention(a, s);
    if (split && out_amax != nullptr) launch_amax_fold(a.out_amax, kOpAmaxStripes, out_amax, s);
  });
}

int carat_hip_row_op(const carat_hip_row_args *args, void *stream) {
  return guarded([&] {
    if (args == nullptr) throw std::runtime_error("null row arguments");
    if (args->source < 0 || args->source > 2) throw std::runtime_error("invalid row source");
    RowArgs r;
    r.source = static_cast<RowSource>(args->source);
    r.rows = args->rows;
    r.width = args->width;
    r.eps = args->eps;
    r.embedding = args->embedding;
    r.tokens = args->tokens;
    r.vocabulary = args->vocabulary;
    r.embed_scale = args->embed_scale;
    r.partials = args->partials;
    r.splits = args->splits;
    r.x_amax = args->x_amax;
    r.w_scale = args->w_scale;
    r.x = args->x;
    r.v_out = args->v_out;
    r.w1 = args->w1;
    r.residual = args->residual;
    r.scalar = args->scalar;
    r.r1_out = args->r1_out;
    r.w2 = args->w2;
    r.y_out = args->y_out;
    r.y_amax = args->y_amax;
    launch_row_kernel(r, static_cast<hipStream_t>(stream));
  });
}

int carat_hip_qkv_post(const uint16_t *packed, int rows, int tokens, int query_heads,
                       int kv_heads, int dimension, int key_equals_value, float eps,
                       const uint16_t *q_norm, const uint16_t *k_norm, const uint16_t *cosine,
                       const uint16_t *sine, const int32_t *positions, const int32_t *slots,
                       uint16_t *q_out, uint16_t *k_new, uint16_t *v_new, uint16_t *k_cache,
                       uint16_t *v_cache, int capacity, void *stream) {
  return guarded([&] {
    QkvArgs a;
    a.packed = packed;
    a.rows = rows;
    a.tokens = tokens;
    a.query_heads = query_heads;
    a.kv_heads = kv_heads;
    a.dimension = dimension;
    a.key_equals_value = key_equals_value != 0;
    a.eps = eps;
    a.q_norm = q_norm;
    a.k_norm = k_norm;
    a.cosine = cosine;
    a.sine = sine;
    a.positions = positions;
    a.slots = slots;
    a.q_out = q_out;
    a.k_new = k_new;
    a.v_new = v_new;
    a.k_cache = k_cache;
    a.v_cache = v_cache;
    a.capacity = capacity;
    launch_qkv_post(a, static_cast<hipStream_t>(stream));
  });
}

int carat_hip_rope_table(int dimension, int proportional, int positions, uint16_t *cosine,
                         uint16_t *sine) {
  return guarded([&] {
    if (dimension <= 0 || dimension % 8 != 0 || positions <= 0 || cosine == nullptr || sine == nullptr)
      throw std::runtime_error("invalid RoPE table shape");
    std::vector<bf16_t> c, s;
    rope_table(dimension, proportional != 0, positions, c, s);
    std::memcpy(cosine, c.data(), c.size() * sizeof(bf16_t));
    std::memcpy(sine, s.data(), s.size() * sizeof(bf16_t));
  });
}

int carat_hip_f32_to_e4m3(const float *in, uint8_t *out, int64_t n, void *stream) {
  return guarded([&] {
    if (n <= 0) return;
    convert_e4m3_kernel<<<static_cast<unsigned>((n + 255) / 256), 256, 0,
                          static_cast<hipStream_t>(stream)>>>(in, out, n);
    hip_check(hipGetLastError(), "launch e4m3 conversion");
  });
}

}  // extern "C"
