// Reference-side binding of the MI355X runner: Gemma4BatchModelRunner's own constructor
// (include/carat/batch_model_runner.h:24-28), built inside the reference's tree against its
// Gemma4Config (include/carat/gemma4_config.h:25-40), DeviceWeightArena / Fp8WeightArena
// (include/carat/device_weights.h:15-52) and assistant shape (include/carat/weight_plan.h:25-37).
// Compile with carat_amd/binding and this repository's include/ ahead of the reference's
// include/, and link libcarat_hip.so. The arenas must hold device memory the HIP runtime can
// read (a HIP build of DeviceWeightArena::load / Fp8WeightArena::quantize).
#include "carat/batch_model_runner.h"

#include "carat/device_weights.h"
#include "carat/gemma4_config.h"
#include "carat/weight_plan.h"

#include <stdexcept>
#include <string>
#include <vector>

namespace carat {
namespace {

struct ArenaSet {
  const DeviceWeightArena *weights[2];
  const Fp8WeightArena *fp8[2];
};

// carat_hip_device_segment_fn over the reference's arenas: index 0 target, 1 assistant. The
// arenas do not expose per-segment sizes, so *bytes is left as the runner's own figure; the
// runner's description comes from the same Gemma4Config the arenas' WeightPlan was built from.
const void *arena_segment(void *context, int assistant, int fp8, const char *name,
                          const float **scale, uint64_t * /*bytes*/) {
  const auto &arenas = *static_cast<const ArenaSet *>(context);
  const int which = assistant != 0 ? 1 : 0;
  try {
    if (fp8 != 0) {
      const Fp8WeightArena *arena = arenas.fp8[which];
      if (arena == nullptr) return nullptr;
      const void *data = arena->at(name);
      *scale = arena->scale(name);
      return data;
    }
    const DeviceWeightArena *arena = arenas.weights[which];
    return arena == nullptr ? nullptr : arena->at(name);
  } catch (const std::exception &) {
    return nullptr;  // absent segment: the runner reports it by name
  }
}

}  // namespace

Gemma4BatchModelRunner::Gemma4BatchModelRunner(const Gemma4Config &config,
                                               const DeviceWeightArena &weights, int batch,
                                               int maximum_context,
                                               const Fp8WeightArena *fp8_weights,
                                               const DeviceWeightArena *assistant_weights,
                                               const Fp8WeightArena *assistant_fp8_weights) {
  // The target arena may be quantised per tensor, channel or 128 x 128 block; the assistant's
  // Fp8Linear is per tensor (assistant_runner.cu:123-125), so its arena must be too.
  if (assistant_fp8_weights != nullptr && assistant_fp8_weights->scaling() != Fp8Scaling::tensor)
    throw std::runtime_error("assistant FP8 weights must be quantized per tensor");
  std::vector<carat_hip_layer_desc> layers;
  layers.reserve(config.layers.size());
  for (const Gemma4LayerConfig &layer : config.layers)
    layers.push_back({layer.attention == AttentionKind::sliding ? 1 : 0,
                      static_cast<int>(layer.query_heads), static_cast<int>(layer.kv_heads),
                      static_cast<int>(layer.head_dimension), layer.key_equals_value ? 1 : 0});
  constexpr Gemma4AssistantShape assistant = gemma4_assistant_shape;
  carat_hip_model_desc desc{};
  desc.hidden = static_cast<int>(config.hidden_size);
  desc.intermediate = static_cast<int>(config.intermediate_size);
  desc.vocabulary = static_cast<int>(config.vocabulary_size);
  desc.sliding_window = static_cast<int>(config.sliding_window);
  desc.rms_norm_epsilon = static_cast<float>(config.rms_norm_epsilon);
  desc.layer_count = static_cast<int>(layers.size());
  desc.layers = layers.data();
  desc.assistant = assistant_weights != nullptr ? 1 : 0;
  desc.assistant_hidden = static_cast<int>(assistant.hidden);
  desc.assistant_intermediate = static_cast<int>(assistant.intermediate);
  desc.assistant_layers = static_cast<int>(assistant.layers);
  desc.assistant_query_heads = static_cast<int>(assistant.query_heads);
  // The assistant's FP8 mode comes from CARAT_ASSISTANT_FP8_MODE, as in the reference's
  // assistant runner (assistant_runner.cu:31-44); lm_head and all read the assistant FP8 arena
  // and fail without it.
  desc.assistant_fp8_mode = 0;
  desc.fp8_scaling = fp8_weights == nullptr ? 0
                     : fp8_weights->scaling() == Fp8Scaling::channel ? 1
                     : fp8_weights->scaling() == Fp8Scaling::block_128 ? 2
                                                                     : 0;
  ArenaSet arenas{{&weights, assistant_weights}, {fp8_weights, assistant_fp8_weights}};
  hip_ok(carat_hip_runner_create_from_device_weights(&desc, arena_segment, &arenas, batch,
                                                     maximum_context, &runner_));
}

}  // namespace carat
