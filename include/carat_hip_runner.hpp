// C++ drop-in for the reference's runner interface, header-only over the C ABI in carat_hip.h
// (the speculation helpers are in carat_hip_speculation.hpp). Class, method and type names,
// argument meaning and error behaviour follow include/carat/batch_model_runner.h:10-77 of the
// reference:
// every failure is rethrown as std::runtime_error carrying the library's message, which is the
// reference's own text (batch_model_runner.cu:1006-1810), so CHECK_THROWS(expr, fragment) style
// tests keep working. The reference's serving loop (native_runtime_main.cpp:583-678) calls these
// unchanged.
//
// Construction: the reference's own constructor (config + device weight arenas) is declared here
// and defined in carat_amd/binding/batch_model_runner_binding.cpp, which compiles against the
// reference's Gemma4Config / DeviceWeightArena / Fp8WeightArena headers. A runner can also be
// built from a Gemma-4 checkpoint directory (config.json + safetensors, weights quantised and
// packed on the device) or from a carat_hip_model_desc of seeded synthetic weights.
#pragma once

#include "carat_hip.h"

#include <cstdint>
#include <optional>
#include <stdexcept>
#include <string>
#include <vector>

namespace carat {

struct Gemma4Config;
class DeviceWeightArena;
class Fp8WeightArena;

inline void hip_ok(int status) {
  if (status != 0) throw std::runtime_error(carat_hip_last_error());
}

// ------------------------------------------------------------------ batch_model_runner.h:10-77
struct GreedyVerificationResult {
  std::vector<int> accepted_tokens;
  std::vector<int> next_tokens;
};

struct LayerSlicedSuffixPrefillResult {
  bool complete{false};
  std::vector<int> predictions;
};

class Gemma4BatchModelRunner {
public:
  // batch_model_runner.h:24-28. Defined in carat_amd/binding/batch_model_runner_binding.cpp
  // (built with the reference's headers): the arenas' bf16 segments, and the FP8 arena's e4m3
  // segments and scales when given, are copied into the runner during construction.
  Gemma4BatchModelRunner(const Gemma4Config &config, const DeviceWeightArena &weights, int batch,
                         int maximum_context, const Fp8WeightArena *fp8_weights = nullptr,
                         const DeviceWeightArena *assistant_weights = nullptr,
                         const Fp8WeightArena *assistant_fp8_weights = nullptr);
  // Seeded synthetic weights of the described shape.
  Gemma4BatchModelRunner(const carat_hip_model_desc &desc, int batch, int maximum_context) {
    hip_ok(carat_hip_runner_create(&desc, batch, maximum_context, &runner_));
  }
  // A Gemma-4 checkpoint (and optionally its assistant) read from disk.
  Gemma4BatchModelRunner(const std::string &model_dir, const std::string &assistant_dir, int batch,
                         int maximum_context) {
    hip_ok(carat_hip_runner_create_from_checkpoint(
        model_dir.c_str(), assistant_dir.empty() ? nullptr : assistant_dir.c_str(), batch,
        maximum_context, &runner_));
  }
  ~Gemma4BatchModelRunner() { carat_hip_runner_destroy(runner_); }
  Gemma4BatchModelRunner(const Gemma4BatchModelRunner &) = delete;
  Gemma4BatchModelRunner &operator=(const Gemma4BatchModelRunner &) = delete;

  std::vector<int> append(const std::vector<int> &token_ids) {
    std::vector<int> next(token_ids.size());
    hip_ok(carat_hip_runner_append(runner_, token_ids.data(), static_cast<int>(token_ids.size()),
                                   next.data()));
    return next;
  }

  int prefill_slot(int slot, const std::vector<int> &token_ids, int chunk_tokens = 1024) {
    int32_t next = 0;
    hip_ok(carat_hip_runner_prefill_slot(runner_, slot, token_ids.data(),
                                         static_cast<int>(token_ids.size()), chunk_tokens, &next));
    return next;
  }

  int prefill_slot_from_prefix(int slot, const std::vector<int> &token_ids,
                               int cached_prefix_tokens, int chunk_tokens = 1024) {
    int32_t next = 0;
    hip_ok(carat_hip_runner_prefill_slot_from_prefix(runner_, slot, token_ids.data(),
                                                     static_cast<int>(token_ids.size()),
                                                     cached_prefix_tokens, chunk_tokens, &next));
    return next;
  }

  std::optional<int> prefill_slot_chunk(int slot, const std::vector<int> &token_ids,
                                        int chunk_tokens) {
    int32_t next = -1;
    hip_ok(carat_hip_runner_prefill_slot_chunk(runner_, slot, token_ids.data(),
                                               static_cast<int>(token_ids.size()), chunk_tokens,
                                               &next));
    return next < 0 ? std::nullopt : std::optional<int>(next);
  }

  std::vector<std::optional<int>>
  prefill_slots_chunks(const std::vector<int> &slots,
                       const std::vector<const std::vector<int> *> &token_ids, int chunk_tokens) {
    std::vector<int32_t> offsets, flat;
    pack(slots, token_ids, offsets, flat, "invalid batched chunk prefill shape");
    std::vector<int32_t> predictions(slots.size());
    hip_ok(carat_hip_runner_prefill_slots_chunks(runner_, static_cast<int>(slots.size()),
                                                 slots.data(), offsets.data(), flat.data(),
                                                 chunk_tokens, predictions.data()));
    std::vector<std::optional<int>> out;
    for (const int32_t p : predictions) out.push_back(p < 0 ? std::nullopt : std::optional<int>(p));
    return out;
  }

  std::vector<int> prefill_slots_suffix(const std::vector<int> &slots,
                                        const std::vector<const std::vector<int> *> &token_ids) {
    std::vector<int32_t> offsets, flat;
    pack(slots, token_ids, offsets, flat, "invalid batched suffix prefill shape");
    std::vector<int> predictions(slots.size());
    hip_ok(carat_hip_runner_prefill_slots_suffix(runner_, static_cast<int>(slots.size()),
                                                 slots.data(), offsets.data(), flat.data(),
                                                 predictions.data()));
    return predictions;
  }

  LayerSlicedSuffixPrefillResult
  prefill_slots_suffix_layer_slice(const std::vector<int> &slots,
                                   const std::vector<const std::vector<int> *> &token_ids,
                                   int maximum_layers) {
    std::vector<int32_t> offsets, flat;
    pack(slots, token_ids, offsets, flat, "invalid layer-sliced suffix prefill shape");
    LayerSlicedSuffixPrefillResult out;
    std::vector<int> predictions(slots.size());
    int complete = 0;
    hip_ok(carat_hip_runner_prefill_slots_suffix_layer_slice(
        runner_, static_cast<int>(slots.size()), slots.data(), offsets.data(), flat.data(),
        maximum_layers, &complete, predictions.data()));
    out.complete = complete != 0;
    if (out.complete) out.predictions = std::move(predictions);
    return out;
  }

  void abort_suffix_layer_slices() { hip_ok(carat_hip_runner_abort_suffix_layer_slices(runner_)); }

  [[nodiscard]] bool has_suffix_layer_slices() const {
    int v = 0;
    hip_ok(carat_hip_runner_has_suffix_layer_slices(runner_, &v));
    return v != 0;
  }

  std::uint64_t clone_slot(int source_slot, int destination_slot) {
    uint64_t bytes = 0;
    hip_ok(carat_hip_runner_clone_slot(runner_, source_slot, destination_slot, &bytes));
    return bytes;
  }

  std::vector<int> append_ragged(const std::vector<int> &token_ids, const std::vector<int> &slots) {
    if (token_ids.size() != slots.size()) throw std::runtime_error("invalid ragged token batch");
    std::vector<int> next(token_ids.size());
    hip_ok(carat_hip_runner_append_ragged(runner_, static_cast<int>(token_ids.size()),
                                          token_ids.data(), slots.data(), next.data()));
    return next;
  }

  GreedyVerificationResult verify_greedy_proposals(
      const std::vector<std::vector<int>> &proposals, const std::vector<int> &target_first_tokens,
      const std::vector<int> &slots, const std::vector<int> &maximum_accepted_tokens = {}) {
    const int requests = static_cast<int>(proposals.size());
    if (target_first_tokens.size() != proposals.size() || slots.size() != proposals.size())
      throw std::runtime_error("invalid greedy verification batch");
    if (!maximum_accepted_tokens.empty() && maximum_accepted_tokens.size() != proposals.size())
      throw std::runtime_error("speculative acceptance caps do not match request count");
    const int depth = requests ? static_cast<int>(proposals[0].size()) : 0;
    std::vector<int32_t> flat;
    for (const auto &row : proposals) {
      if (static_cast<int>(row.size()) != depth)
        throw std::runtime_error("invalid or repeated speculative slot");
      flat.insert(flat.end(), row.begin(), row.end());
    }
    GreedyVerificationResult out{std::vector<int>(proposals.size()),
                                 std::vector<int>(proposals.size())};
    hip_ok(carat_hip_runner_verify(
        runner_, requests, depth, flat.data(), target_first_tokens.data(), slots.data(),
        maximum_accepted_tokens.empty() ? nullptr : maximum_accepted_tokens.data(),
        out.accepted_tokens.data(), out.next_tokens.data(), nullptr));
    return out;
  }

  [[nodiscard]] bool has_assistant() const {
    int v = 0;
    hip_ok(carat_hip_runner_has_assistant(runner_, &v));
    return v != 0;
  }

  std::vector<std::vector<int>> draft_four(const std::vector<int> &last_tokens,
                                           const std::vector<int> &slots,
                                           const std::vector<int> &forced_first_tokens = {},
                                           int depth = 4) {
    if (last_tokens.size() != slots.size() || last_tokens.empty() || depth <= 0)
      throw std::runtime_error("assistant is not configured or draft batch is invalid");
    if (!forced_first_tokens.empty() && forced_first_tokens.size() != last_tokens.size())
      throw std::runtime_error("forced assistant first tokens do not match draft batch");
    const int rows = static_cast<int>(last_tokens.size());
    std::vector<int32_t> table(static_cast<size_t>(rows) * static_cast<size_t>(depth));
    hip_ok(carat_hip_runner_draft(runner_, rows, depth, last_tokens.data(), slots.data(),
                                  forced_first_tokens.empty() ? nullptr : forced_first_tokens.data(),
                                  table.data()));
    std::vector<std::vector<int>> out(static_cast<size_t>(rows));
    for (int r = 0; r < rows; ++r)
      out[static_cast<size_t>(r)].assign(table.begin() + r * depth, table.begin() + (r + 1) * depth);
    return out;
  }

  void reset_slot(int slot) { hip_ok(carat_hip_runner_reset_slot(runner_, slot)); }

  void seed_empty_cache_for_benchmark(int position) {
    hip_ok(carat_hip_runner_seed_empty_cache_for_benchmark(runner_, position));
  }

  [[nodiscard]] int batch() const {
    int v = 0;
    hip_ok(carat_hip_runner_batch(runner_, &v));
    return v;
  }

  [[nodiscard]] int position() const {
    int v = 0;
    hip_ok(carat_hip_runner_position(runner_, &v));
    return v;
  }

  [[nodiscard]] int slot_position(int slot) const {
    int v = 0;
    hip_ok(carat_hip_runner_slot_position(runner_, slot, &v));
    return v;
  }

  // The C ABI handle, for the entry points without a reference counterpart (timing, tensors).
  [[nodiscard]] carat_hip_runner *handle() const { return runner_; }

private:
  // Request r's prompt becomes flat[offsets[r] .. offsets[r + 1]).
  static void pack(const std::vector<int> &slots, const std::vector<const std::vector<int> *> &prompts,
                   std::vector<int32_t> &offsets, std::vector<int32_t> &flat, const char *message) {
    if (prompts.size() != slots.size() || slots.empty()) throw std::runtime_error(message);
    offsets.assign(1, 0);
    for (const auto *prompt : prompts) {
      if (prompt != nullptr) flat.insert(flat.end(), prompt->begin(), prompt->end());
      offsets.push_back(static_cast<int32_t>(flat.size()));
    }
    if (flat.empty()) flat.push_back(0);  // keep the token pointer non-null
  }

  carat_hip_runner *runner_ = nullptr;
};

}  // namespace carat
