// MI355X batch model runner (see runner.h).
//
// Verify step, per layer (reference: cuda/layer_runner.cu:241-354, 730-1041):
//   QKV fp8 GEMM (split-K partials) -> QKV reduce + per-head norm + RoPE (K/V to this step's rows;
//   global layers also to the cache) -> fused verify attention (sliding ring read before any
//   proposal is written, so no backup copy) -> O fp8 GEMM -> reduce + post-attention norm +
//   residual + pre-MLP norm -> gate/up fp8 GEMM with the GELU gate in the epilogue -> down fp8 GEMM
//   -> reduce + post-MLP norm + residual + layer scalar + the NEXT layer's input norm.
// Then the fp8 lm_head with the vocabulary argmax in its epilogue, and one kernel for greedy
// acceptance + committing the accepted proposal rows into the sliding rings + the hidden hand-off.
// Activation amaxes are produced by the kernel that writes the activation and consumed by the next
// GEMM's prologue, so no separate quantisation pass runs.
#include "runner.h"

#include "attention.h"
#include "checkpoint.h"
#include "gemm.h"
#include "init.h"
#include "rowops.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>
#include <numeric>
#include <stdexcept>
#include <tuple>

namespace carat_hip {

ModelSpec gemma4_31b_benchmark_spec(bool with_assistant) {
  ModelSpec spec;
  spec.hidden = 5376;
  spec.intermediate = 21504;
  spec.vocabulary = 262144;
  spec.sliding_window = 1024;
  spec.eps = 1e-6f;
  for (int layer = 0; layer < 60; ++layer) {
    LayerSpec l;
    l.sliding = (layer % 6) != 5;
    l.query_heads = 32;
    l.kv_heads = 16;
    l.head_dimension = 128;
    l.key_equals_value = false;
    spec.layers.push_back(l);
  }
  spec.assistant.enabled = with_assistant;
  return spec;
}

namespace {

constexpr int kMaximumDepth = 8;  // batch_model_runner.cu:33 speculative_depth
// Rows of one forced prefill step (bounded further by the context and the sliding ring): enough
// for the skinny GEMMs' token blocks to share each weight block through L2.
constexpr int kPrefillStepRows = 1024;
constexpr int kAmaxStripes = 64;  // stripes per per-tensor amax (see amax_publish)
constexpr int kAmaxSlotFloats = kAmaxStripes * kAmaxStripeFloats;  // storage per amax
static_assert(kAmaxStripes >= kFusedSyncWords, "a sync slot holds the fused quantisation's words");

class DeviceBuffer {
public:
  DeviceBuffer() = default;
  explicit DeviceBuffer(size_t bytes) { allocate(bytes); }
  ~DeviceBuffer() {
    if (pointer_ != nullptr) (void)hipFree(pointer_);
  }
  DeviceBuffer(const DeviceBuffer &) = delete;
  DeviceBuffer &operator=(const DeviceBuffer &) = delete;
  DeviceBuffer(DeviceBuffer &&other) noexcept : pointer_(other.pointer_), bytes_(other.bytes_) {
    other.pointer_ = nullptr;
    other.bytes_ = 0;
  }
  void allocate(size_t bytes) {
    if (pointer_ != nullptr) throw std::runtime_error("device buffer already allocated");
    bytes_ = bytes;
    if (bytes == 0) return;
    hip_check(hipMalloc(&pointer_, bytes), "allocate device memory");
  }
  void release() {
    if (pointer_ != nullptr) (void)hipFree(pointer_);
    pointer_ = nullptr;
    bytes_ = 0;
  }
  template <typename T> T *as() const { return static_cast<T *>(pointer_); }
  void *get() const { return pointer_; }
  size_t bytes() const { return bytes_; }

private:
  void *pointer_ = nullptr;
  size_t bytes_ = 0;
};

// A weight in the GEMM's packed storage order (gemm.h WeightLayout); logical shape [n][row_bytes].
struct PackedWeight {
  DeviceBuffer data;
  WeightLayout layout;
  // e4m3 weights under Fp8Scaling channel (1) or block_128 (2): their scales in the
  // Fp8WeightArena layout ([n], or [ceil(n/128)][scale_kblocks]); tensor-scaled weights keep their
  // one float with the caller.
  int scaling = 0;
  int scale_kblocks = 0;
  DeviceBuffer scale_table;
  template <typename T> T *as() const { return data.as<T>(); }
  void *get() const { return data.get(); }
};

struct TargetLayer {
  LayerSpec spec;
  int capacity = 0;
  DeviceBuffer input_norm, q_norm, k_norm, post_attention_norm, pre_mlp_norm, post_mlp_norm, scalar;
  PackedWeight qkv, o, gate_up, down;  // e4m3
  DeviceBuffer scales;                 // [4] floats: qkv, o, gate_up, down
  DeviceBuffer k_cache, v_cache;       // [batch][Hkv][C][D]
  DeviceBuffer k_new, v_new;           // [batch*8][Hkv][D] this step's rows
  int query_width() const { return spec.query_heads * spec.head_dimension; }
  int kv_width() const { return spec.kv_heads * spec.head_dimension; }
  int packed_width() const { return query_width() + kv_width() * (spec.key_equals_value ? 1 : 2); }
};

struct AssistantLayer {
  bool global = false;
  int kv_heads = 0;
  int head_dimension = 0;
  int attention_chunk = 0;  // keys per workgroup of its decode attention over the target cache
  DeviceBuffer input_norm, q_norm, post_attention_norm, pre_mlp_norm, post_mlp_norm, scalar;
  PackedWeight q, o, gate_up, down;  // bf16
  // AssistantFp8Mode::all: e4m3 copies (per-tensor scales: q, o, gate_up, down)
  PackedWeight q8, o8, gate_up8, down8;
  DeviceBuffer scales8;
};

// The assistant's input row of one draft step: the token's embedding row times bf16(sqrt(H)) |
// the previous hidden row (embedding_batch_bf16 + concatenate_rows_bf16,
// assistant_runner.cu:279-283). The token is given, or (the steps after an lm_head pass) reduced
// here from that pass's per-workgroup argmax keys (argmax_bf16_rows, :316; the reduction of
// argmax_reduce_kernel), the row's block 0 writing it to the proposals table. The previous hidden
// row is gathered from the target's hand-off rows by slot (gather_rows_bf16, :271; the first
// step), or summed here from the post-projection's split-K partials and rounded as the row kernel
// would (:320; the later steps). Every thread owns 8 consecutive elements of the 2H-wide row;
// `amax` (the `all` fp8 mode: the pre-projection input's per-tensor quantisation) gets the row's
// maximum magnitude.
struct AssistantInputArgs {
  const bf16_t *embedding = nullptr;
  int vocabulary = 0;
  float embed_scale = 1.0f;
  const int32_t *tokens = nullptr;             // or:
  const uint64_t *argmax_partials = nullptr;   // [row][argmax_parts] keys
  int argmax_parts = 0;
  int32_t *table = nullptr;                    // optional: table[row * stride + column] = token
  int table_stride = 0, table_column = 0;
  const bf16_t *gather_src = nullptr;          // [slot][hidden], rows gather_rows[row]; or:
  const int32_t *gather_rows = nullptr;
  const float *partials = nullptr;             // [splits][rows][hidden]
  int splits = 1;
  const float *x_amax = nullptr;               // partials' fp8 output scale operands (or null)
  const float *w_scale = nullptr;
  bf16_t *out = nullptr;                       // [rows][2 hidden]
  int rows = 0, hidden = 0;
  float *amax = nullptr;
  int stripes = 1;
};

__global__ __launch_bounds__(256) void assistant_input_kernel(const AssistantInputArgs a) {
  const int row = blockIdx.y;
  const int c0 = (blockIdx.x * 256 + threadIdx.x) * 8;
  const bool live = c0 < 2 * a.hidden;
  const bool previous = live && c0 >= a.hidden;
  // the previous-hidden half first: its loads do not wait for the token
  float pv[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  u32x4_t gathered = {0u, 0u, 0u, 0u};
  float amax_part = 0.0f, w_scale = 1.0f;
  if (a.partials != nullptr) {
    if (a.x_amax != nullptr) amax_part = amax_lane(a.x_amax, a.stripes);
    if (a.w_scale != nullptr) w_scale = *a.w_scale;
  }
  if (previous) {
    const int c = c0 - a.hidden;
    if (a.partials != nullptr) {
      for (int k = 0; k < a.splits; ++k) {
        const float *src = a.partials + (static_cast<size_t>(k) * a.rows + row) * a.hidden + c;
        const f32x4_t lo = *reinterpret_cast<const f32x4_t *>(src);
        const f32x4_t hi = *reinterpret_cast<const f32x4_t *>(src + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          pv[e] += lo[e];
          pv[4 + e] += hi[e];
        }
      }
    } else {
      gathered = *reinterpret_cast<const u32x4_t *>(
          a.gather_src + static_cast<size_t>(a.gather_rows[row]) * a.hidden + c);
    }
  }
  int token;
  if (a.argmax_partials != nullptr) {
    uint64_t best = kArgmaxInitialKey;
    for (int i = threadIdx.x; i < a.argmax_parts; i += 256) {
      const uint64_t k = a.argmax_partials[static_cast<size_t>(row) * a.argmax_parts + i];
      best = k > best ? k : best;
    }
    best = wave_max_u64(best);
    __shared__ uint64_t wave_best[4];
    if ((threadIdx.x & 63) == 0) wave_best[threadIdx.x >> 6] = best;
    __syncthreads();
    best = wave_best[0];
#pragma unroll
    for (int w = 1; w < 4; ++w) best = wave_best[w] > best ? wave_best[w] : best;
    token = static_cast<int>(argmax_key_index(best));
  } else {
    token = a.tokens[row];
  }
  if (a.table != nullptr && blockIdx.x == 0 && threadIdx.x == 0)
    a.table[row * a.table_stride + a.table_column] = token;
  float scale = w_scale;
  if (a.partials != nullptr && a.x_amax != nullptr) scale *= fp8_scale_from_amax(wave_max(amax_part));
  if (!live) return;
  u32x4_t value;
  if (!previous) {
    value = u32x4_t{0u, 0u, 0u, 0u};
    if (token >= 0 && token < a.vocabulary) {
      const float s = round_bf16(a.embed_scale);
      const u32x4_t e = *reinterpret_cast<const u32x4_t *>(a.embedding + static_cast<size_t>(token) * a.hidden + c0);
#pragma unroll
      for (int q = 0; q < 4; ++q)
        value[q] = f32x2_to_bf16x2(__uint_as_float(e[q] << 16) * s, __uint_as_float(e[q] & 0xffff0000u) * s);
    }
  } else if (a.partials != nullptr) {
#pragma unroll
    for (int q = 0; q < 4; ++q) value[q] = f32x2_to_bf16x2(pv[2 * q] * scale, pv[2 * q + 1] * scale);
  } else {
    value = gathered;
  }
  *reinterpret_cast<u32x4_t *>(a.out + static_cast<size_t>(row) * 2 * a.hidden + c0) = value;
  if (a.amax == nullptr) return;
  float maximum = 0.0f;
#pragma unroll
  for (int q = 0; q < 4; ++q)
    maximum = fmaxf(maximum, fmaxf(fabsf(__uint_as_float(value[q] << 16)), fabsf(__uint_as_float(value[q] & 0xffff0000u))));
  maximum = wave_max(maximum);
  if ((threadIdx.x & (kWave - 1)) == 0) amax_publish(a.amax, a.stripes, maximum);
}

__global__ void copy_tokens_kernel(const int32_t *src, int32_t *dst, int32_t *table, int rows,
                                   int stride, int column) {
  const int row = blockIdx.x * blockDim.x + threadIdx.x;
  if (row >= rows) return;
  dst[row] = src[row];
  table[row * stride + column] = src[row];
}


}  // namespace

struct BatchModelRunner::Implementation {
  ModelSpec spec;
  int batch_size;
  int maximum_context;
  int maximum_rows;  // batch * kMaximumDepth: rows of a verify step
  int step_rows;     // rows of a forced (prefill) step: >= maximum_rows, sizes the step buffers
  int current_position = 0;
  std::vector<int> slot_positions;
  std::vector<int> predictions;
  hipStream_t stream = nullptr;
  hipEvent_t start_event = nullptr, stop_event = nullptr;
  float verify_ms = 0.0f, draft_ms = 0.0f;
  bool graphs_enabled = false;
  int probe_kind = probe_none;
  // Construction-time weight source (null: seeded weights) and its staging.
  const Checkpoint *checkpoint = nullptr;
  // device-resident bf16 segments (the reference's DeviceWeightArena) when constructing from them
  BatchModelRunner::DeviceSegmentFn device_segment = nullptr;
  void *device_segment_context = nullptr;
  DeviceBuffer load_staging;
  std::unique_ptr<void, void (*)(void *)> pinned{nullptr, [](void *p) {
    if (p != nullptr) (void)hipHostFree(p);
  }};
  int last_rows = 0;  // rows of the last verify step (the stream probe's activation shape)
  int last_requests = 0, last_depth = 0;
  std::vector<std::pair<hipEvent_t, hipEvent_t>> probe_pool;
  size_t probe_used = 0;
  double probe_total_ms = 0.0;
  int probe_launches = 0;
  std::map<std::tuple<int, int, bool>, hipGraphExec_t> verify_graphs;

  std::vector<TargetLayer> layers;
  DeviceBuffer embedding_bf16, embedding_scale, final_norm;
  PackedWeight lm_head;  // e4m3 copy of the tied embedding
  DeviceBuffer staging;  // row-major weights before packing (freed after load)
  DeviceBuffer rope_sliding_cos, rope_sliding_sin, rope_global_cos, rope_global_sin;
  int rope_sliding_dim = 0, rope_global_dim = 0;

  // workspaces
  DeviceBuffer hidden_a, hidden_b, normalized, first_residual, pre_mlp, activated, queries,
      attention_out, final_hidden, partials, amax, argmax_partials, xprep, x_scales, attention_partials,
      target_hidden, sliding_table, init_scratch;
  size_t attention_partial_floats = 0;
  int attention_chunk_sliding = 256, attention_chunk_global = 256;
  // device inputs / outputs and their pinned host staging
  DeviceBuffer device_io;
  int32_t *d_tokens = nullptr, *d_positions = nullptr, *d_slots = nullptr, *d_first = nullptr,
          *d_caps = nullptr, *d_accepted = nullptr, *d_next = nullptr, *d_predictions = nullptr,
          *d_fault = nullptr;
  int32_t *host_io = nullptr;  // pinned mirror of device_io
  int32_t *a_host_io = nullptr;  // pinned mirror of a_io (the draft's inputs and proposals)
  // verify steps quantise the layer-end rows' outputs in the row kernels (RowArgs::xprep)
  // 0 (default): separate prepare kernels, measured faster in the step than the fused
  // quantisation (1); 2: fused with a zero wait bound (error-path test)
  int fused_quantize_mode = 0;
  // verify attention post-processes the QKV rows itself where it can (attention_can_fuse_qkv)
  bool qkv_fusion = true;
  bool last_input_prepared = false;
  size_t io_ints = 0;
  int sliding_layer_count = 0;
  int last_sliding = -1, last_global = -1;

  // assistant
  bool has_assistant = false;
  std::vector<AssistantLayer> assistant_layers;
  PackedWeight a_embedding, a_pre_projection, a_post_projection;  // bf16
  DeviceBuffer a_final_norm;
  // AssistantFp8Mode (assistant_runner.cu:29-43): 0 off, 1 lm_head, 2 all. The e4m3 copies of
  // the lm_head (both fp8 modes) and of the pre/post projections (all), per-tensor scales
  // [lm_head, pre, post]; per-draft-step striped amaxes of the projections' inputs.
  int assistant_fp8 = 0;
  PackedWeight a_embedding8, a_pre_projection8, a_post_projection8;
  DeviceBuffer a_scales8, a_amax;
  DeviceBuffer a_input, a_hidden_a, a_hidden_b, a_normalized, a_first_residual, a_pre_mlp,
      a_activated, a_queries, a_attention_out, a_final_hidden, a_previous_hidden;
  DeviceBuffer a_io;
  int32_t *a_tokens = nullptr, *a_outputs = nullptr, *a_forced = nullptr, *a_context = nullptr,
          *a_slots = nullptr, *a_proposals = nullptr;

  Implementation(const ModelSpec &model, int batch, int context, const Checkpoint *source = nullptr,
                 BatchModelRunner::DeviceSegmentFn segment = nullptr, void *segment_context = nullptr)
      : spec(model), batch_size(batch), maximum_context(context),
        maximum_rows(batch * kMaximumDepth),
        step_rows(std::max(batch * kMaximumDepth, std::min(kPrefillStepRows, context))),
        slot_positions(static_cast<size_t>(batch), 0) {
    checkpoint = source;
    device_segment = segment;
    device_segment_context = segment_context;
    if (batch <= 0 || batch > 64 || context <= 0 || spec.layers.empty() || spec.hidden <= 0 ||
        spec.intermediate <= 0 || spec.vocabulary <= 0)
      throw std::runtime_error("invalid runner shape");
    if (maximum_rows > 192) throw std::runtime_error("runner batch exceeds 192 verify rows");
    try {
      hip_check(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking), "create runner stream");
      hip_check(hipEventCreate(&start_event), "create event");
      hip_check(hipEventCreate(&stop_event), "create event");
      init_scratch.allocate(256);
      allocate_target();
      if (spec.assistant.enabled) allocate_assistant();
      allocate_workspaces();
      hip_check(hipStreamSynchronize(stream), "initialise runner");
    } catch (...) {
      // a failed construction releases the handles the destructor would have (device buffers
      // free themselves)
      if (stream != nullptr) (void)hipStreamSynchronize(stream);
      release_handles();
      throw;
    }
    staging.release();
    load_staging.release();
    pinned.reset();
    checkpoint = nullptr;
    device_segment = nullptr;
    device_segment_context = nullptr;
  }

  // Next probe event pair when `kind` is being probed (else a null pair).
  std::pair<hipEvent_t, hipEvent_t> probe(int kind) {
    if (kind == probe_none || kind != probe_kind) return {nullptr, nullptr};
    if (probe_used == probe_pool.size()) {
      hipEvent_t a = nullptr, b = nullptr;
      hip_check(hipEventCreate(&a), "create probe event");
      if (hipEventCreate(&b) != hipSuccess) {
        (void)hipEventDestroy(a);
        throw std::runtime_error("create probe event failed");
      }
      probe_pool.emplace_back(a, b);
    }
    return probe_pool[probe_used++];
  }

  void collect_probes() {
    for (size_t i = 0; i < probe_used; ++i) {
      float ms = 0.0f;
      hip_check(hipEventElapsedTime(&ms, probe_pool[i].first, probe_pool[i].second), "probe time");
      probe_total_ms += ms;
      ++probe_launches;
    }
    probe_used = 0;
  }

  void set_qkv_fusion(bool enabled) {
    qkv_fusion = enabled;
    for (auto &entry : verify_graphs) (void)hipGraphExecDestroy(entry.second);
    verify_graphs.clear();  // captured steps hold the previous choice
  }

  void set_fused_quantization(int mode) {
    if (mode < 0 || mode > 2) throw std::runtime_error("fused quantisation mode must be 0, 1 or 2");
    fused_quantize_mode = mode;
    for (auto &entry : verify_graphs) (void)hipGraphExecDestroy(entry.second);
    verify_graphs.clear();  // captured steps hold the previous choice
  }

  void release_handles() {
    for (auto &entry : probe_pool) {
      (void)hipEventDestroy(entry.first);
      (void)hipEventDestroy(entry.second);
    }
    probe_pool.clear();
    for (auto &entry : verify_graphs) (void)hipGraphExecDestroy(entry.second);
    verify_graphs.clear();
    if (host_io != nullptr) (void)hipHostFree(host_io);
    host_io = nullptr;
    if (a_host_io != nullptr) (void)hipHostFree(a_host_io);
    a_host_io = nullptr;
    if (start_event != nullptr) (void)hipEventDestroy(start_event);
    if (stop_event != nullptr) (void)hipEventDestroy(stop_event);
    start_event = stop_event = nullptr;
    if (stream != nullptr) (void)hipStreamDestroy(stream);
    stream = nullptr;
  }

  ~Implementation() {
    if (stream != nullptr) (void)hipStreamSynchronize(stream);
    release_handles();
  }

  uint64_t seed_for(uint64_t tensor) const { return spec.seed * 1000003ull + tensor * 7919ull; }

  // ---- weight sources: a checkpoint segment or a device-resident segment when loading one,
  // else seeded values. Segment names are the execution plan's ("layer.3.qkv"; "assistant."
  // selects the assistant's plan).
  bool has_source() const { return checkpoint != nullptr || device_segment != nullptr; }

  // A device segment whose owner reported a size other than the runner's (a description that
  // disagrees with the arena) would be read out of bounds: refuse it before any copy.
  static void check_segment_bytes(const std::string &name, uint64_t reported, size_t expected) {
    if (reported != expected)
      throw std::runtime_error("device weight " + name + " has " + std::to_string(reported) +
                               " bytes, the runner expects " + std::to_string(expected));
  }

  void upload_segment(const std::string &name, void *device, size_t bytes) {
    const bool assistant = name.rfind("assistant.", 0) == 0;
    const std::string segment = assistant ? name.substr(10) : name;
    if (device_segment != nullptr) {
      uint64_t source_bytes = bytes;
      const void *source = device_segment(device_segment_context, assistant ? 1 : 0, 0,
                                          segment.c_str(), nullptr, &source_bytes);
      if (source == nullptr)
        throw std::runtime_error(std::string(assistant ? "assistant" : "target") +
                                 " device weights have no segment " + segment);
      check_segment_bytes(name, source_bytes, bytes);
      hip_check(hipMemcpyAsync(device, source, bytes, hipMemcpyDeviceToDevice, stream),
                "copy device weight segment");
      return;
    }
    const WeightSegment &s = (assistant ? checkpoint->assistant_plan : checkpoint->target_plan).at(segment);
    if (s.bytes != bytes)
      throw std::runtime_error("checkpoint weight " + name + " has " + std::to_string(s.bytes) +
                               " bytes, the runner expects " + std::to_string(bytes));
    constexpr size_t kPinned = 64u << 20;
    if (pinned == nullptr) {
      void *p = nullptr;
      hip_check(hipHostMalloc(&p, kPinned), "allocate pinned staging");
      pinned.reset(p);
    }
    checkpoint->read_segment(assistant, segment, [&](uint64_t offset, const void *data, size_t n) {
      for (size_t done = 0; done < n;) {
        const size_t chunk = std::min(kPinned, n - done);
        std::memcpy(pinned.get(), static_cast<const unsigned char *>(data) + done, chunk);
        hip_check(hipMemcpyAsync(static_cast<unsigned char *>(device) + offset + done, pinned.get(), chunk,
                                 hipMemcpyHostToDevice, stream),
                  "copy weight to device");
        hip_check(hipStreamSynchronize(stream), "copy weight to device");
        done += chunk;
      }
    });
  }

  void fill_norm(DeviceBuffer &buffer, int n, uint64_t tensor, const std::string &segment) {
    buffer.allocate(sizeof(bf16_t) * static_cast<size_t>(n));
    if (has_source()) {
      upload_segment(segment, buffer.get(), buffer.bytes());
      return;
    }
    fill_normal_bf16(buffer.as<bf16_t>(), static_cast<size_t>(n), seed_for(tensor), 1.0f, 0.05f,
                     stream);
  }

  // The device source's own e4m3 copy of a segment (Fp8WeightArena) into `dst` and its scale
  // into `scale`; false when the source has none (the bf16 segment is quantised instead).
  bool copy_device_fp8(const std::string &name, void *dst, size_t bytes, float *scale,
                       size_t scale_floats = 1) {
    if (device_segment == nullptr) return false;
    const bool assistant = name.rfind("assistant.", 0) == 0;
    const std::string segment = assistant ? name.substr(10) : name;
    const float *source_scale = nullptr;
    uint64_t source_bytes = bytes;
    const void *source = device_segment(device_segment_context, assistant ? 1 : 0, 1,
                                        segment.c_str(), &source_scale, &source_bytes);
    if (source == nullptr) return false;
    check_segment_bytes(name + " (e4m3)", source_bytes, bytes);
    if (source_scale == nullptr)
      throw std::runtime_error("device fp8 weight " + segment + " has no scale");
    hip_check(hipMemcpyAsync(dst, source, bytes, hipMemcpyDeviceToDevice, stream),
              "copy device fp8 weight segment");
    hip_check(hipMemcpyAsync(scale, source_scale, sizeof(float) * scale_floats,
                             hipMemcpyDeviceToDevice, stream),
              "copy device fp8 weight scale");
    return true;
  }

  void *staging_for(size_t bytes) {
    if (staging.bytes() < bytes) {
      hip_check(hipStreamSynchronize(stream), "synchronise before staging growth");
      staging.release();
      staging.allocate(bytes);
    }
    return staging.get();
  }

  void pack_from_staging(PackedWeight &w, int n, int row_bytes, bool gate_up, bool few_rows = false) {
    w.layout = gemm_weight_layout(n, row_bytes, gate_up, few_rows);
    w.data.allocate(static_cast<size_t>(n) * row_bytes);
    pack_weight(staging.get(), w.data.get(), w.layout, stream);
  }

  // e4m3 weight [n][k] (per-tensor scale), stored packed: seeded, or the checkpoint's bf16
  // segment quantised on the device (Fp8WeightArena::quantize, device_weights.cu:200-263).
  void fill_fp8(PackedWeight &w, int n, int k, bool gate_up, uint64_t tensor, float *scale,
                const std::string &segment) {
    const size_t count = static_cast<size_t>(n) * k;
    if (spec.fp8_scaling != 0) {
      fill_fp8_scaled(w, n, k, tensor, segment);
    } else if (copy_device_fp8(segment, staging_for(count), count, scale)) {
      // the source's own e4m3 bytes and scale (Fp8WeightArena::quantize already ran)
    } else if (has_source()) {
      if (load_staging.bytes() < count * sizeof(bf16_t)) {
        hip_check(hipStreamSynchronize(stream), "synchronise before staging growth");
        load_staging.release();
        load_staging.allocate(count * sizeof(bf16_t));
      }
      upload_segment(segment, load_staging.get(), count * sizeof(bf16_t));
      quantize_weight_bf16_to_fp8(load_staging.as<bf16_t>(), static_cast<fp8_t *>(staging_for(count)),
                                  count, scale, init_scratch.as<float>(), stream);
    } else {
      fill_fp8_weight(static_cast<fp8_t *>(staging_for(count)), count, seed_for(tensor),
                      spec.weight_std, scale, init_scratch.as<float>(), stream);
    }
    pack_from_staging(w, n, k, gate_up);
  }

  // The same under Fp8Scaling channel / block_128: the scales go to w.scale_table; the e4m3 bytes
  // into the staging buffer (the caller packs them).
  void fill_fp8_scaled(PackedWeight &w, int n, int k, uint64_t tensor, const std::string &segment) {
    const size_t count = static_cast<size_t>(n) * k;
    w.scaling = spec.fp8_scaling;
    const size_t floats = fp8_weight_scale_elements(w.scaling, n, k);
    w.scale_kblocks = w.scaling == 2 ? static_cast<int>(floats / ((static_cast<size_t>(n) + 127) / 128)) : 0;
    w.scale_table.allocate(sizeof(float) * floats);
    if (copy_device_fp8(segment, staging_for(count), count, w.scale_table.as<float>(), floats)) return;
    if (load_staging.bytes() < count * sizeof(bf16_t)) {
      hip_check(hipStreamSynchronize(stream), "synchronise before staging growth");
      load_staging.release();
      load_staging.allocate(count * sizeof(bf16_t));
    }
    if (has_source())
      upload_segment(segment, load_staging.get(), count * sizeof(bf16_t));
    else
      fill_normal_bf16(load_staging.as<bf16_t>(), count, seed_for(tensor), 0.0f, spec.weight_std,
                       stream);
    quantize_weight_bf16_to_fp8_scaled(load_staging.as<bf16_t>(), static_cast<fp8_t *>(staging_for(count)),
                                       n, k, w.scaling, w.scale_table.as<float>(),
                                       init_scratch.as<float>(), stream);
  }

  // bf16 weight [n][k], stored packed. With `fp8`, also its e4m3 copy with a per-tensor scale
  // into *fp8_scale: the device source's own (Fp8WeightArena, required when loading from device
  // segments), else the bf16 values quantised per tensor (amax/448) as Fp8WeightArena::quantize
  // does (device_weights.cu:200-263).
  void fill_bf16_weight(PackedWeight &w, int n, int k, bool gate_up, uint64_t tensor,
                        float stddev, const std::string &segment, PackedWeight *fp8 = nullptr,
                        float *fp8_scale = nullptr) {
    const size_t count = static_cast<size_t>(n) * k;
    void *dst = staging_for(count * sizeof(bf16_t));
    if (has_source())
      upload_segment(segment, dst, count * sizeof(bf16_t));
    else
      fill_normal_bf16(static_cast<bf16_t *>(dst), count, seed_for(tensor), 0.0f, stddev, stream);
    // the assistant's projections run a draft step's rows (<= the batch) per call
    const bool few_rows = batch_size <= 32;
    pack_from_staging(w, n, 2 * k, gate_up, few_rows);
    if (fp8 == nullptr) return;
    if (load_staging.bytes() < count) {
      hip_check(hipStreamSynchronize(stream), "synchronise before staging growth");
      load_staging.release();
      load_staging.allocate(count * sizeof(bf16_t));
    }
    fp8_t *e4m3 = load_staging.as<fp8_t>();
    if (!copy_device_fp8(segment, e4m3, count, fp8_scale)) {
      if (device_segment != nullptr)
        throw std::runtime_error("assistant FP8 mode requires quantized assistant weights");
      quantize_weight_bf16_to_fp8(static_cast<const bf16_t *>(dst), e4m3, count, fp8_scale,
                                  init_scratch.as<float>(), stream);
    }
    fp8->layout = gemm_weight_layout(n, k, gate_up, few_rows);
    fp8->data.allocate(count);
    pack_weight(e4m3, fp8->data.get(), fp8->layout, stream);
  }

  // AssistantFp8Mode of the assistant runner (assistant_runner.cu:31-44): the description's,
  // or CARAT_ASSISTANT_FP8_MODE. Quantized weights exist unless the runner loads device
  // segments whose source has no assistant e4m3 arena.
  int resolve_assistant_fp8_mode() {
    bool quantized = true;
    if (device_segment != nullptr) {
      const float *scale = nullptr;
      uint64_t bytes = static_cast<uint64_t>(spec.vocabulary) * spec.assistant.hidden;
      quantized = device_segment(device_segment_context, 1, 1, "token_embedding", &scale,
                                 &bytes) != nullptr;
    }
    int mode = spec.assistant.fp8_mode;
    if (mode < 0) {
      const char *configured = std::getenv("CARAT_ASSISTANT_FP8_MODE");
      const std::string text = configured == nullptr ? "off" : configured;
      if (text == "off") return 0;
      if (!quantized) throw std::runtime_error("assistant FP8 mode requires quantized assistant weights");
      if (text == "lm_head") return 1;
      if (text == "all") return 2;
      throw std::runtime_error("CARAT_ASSISTANT_FP8_MODE must be off, lm_head or all");
    }
    if (mode > 2) throw std::runtime_error("invalid assistant FP8 mode");
    if (mode != 0 && !quantized)
      throw std::runtime_error("assistant FP8 mode requires quantized assistant weights");
    return mode;
  }

  void fill_bf16(DeviceBuffer &buffer, size_t n, uint64_t tensor, float stddev,
                 const std::string &segment) {
    buffer.allocate(sizeof(bf16_t) * n);
    if (has_source())
      upload_segment(segment, buffer.get(), buffer.bytes());
    else
      fill_normal_bf16(buffer.as<bf16_t>(), n, seed_for(tensor), 0.0f, stddev, stream);
  }

  void allocate_target() {
    const size_t H = static_cast<size_t>(spec.hidden);
    layers.resize(spec.layers.size());
    uint64_t tensor = 100;
    for (size_t i = 0; i < spec.layers.size(); ++i) {
      TargetLayer &L = layers[i];
      L.spec = spec.layers[i];
      const int D = L.spec.head_dimension;
      if (L.spec.kv_heads <= 0 || L.spec.query_heads % L.spec.kv_heads != 0 ||
          (D != 128 && D != 256 && D != 512))
        throw std::runtime_error("unsupported layer attention shape");
      L.capacity = L.spec.sliding ? std::min(maximum_context, spec.sliding_window) : maximum_context;
      L.scales.allocate(4 * sizeof(float));
      float *scales = L.scales.as<float>();
      // unused under channel / block_128 scaling (the scale tables serve instead)
      if (spec.fp8_scaling != 0)
        hip_check(hipMemsetAsync(scales, 0, 4 * sizeof(float), stream), "clear tensor scales");
      const std::string p = "layer." + std::to_string(i) + ".";
      fill_norm(L.input_norm, spec.hidden, tensor++, p + "input_norm");
      fill_norm(L.q_norm, D, tensor++, p + "q_norm");
      fill_norm(L.k_norm, D, tensor++, p + "k_norm");
      fill_norm(L.post_attention_norm, spec.hidden, tensor++, p + "post_attention_norm");
      fill_norm(L.pre_mlp_norm, spec.hidden, tensor++, p + "pre_mlp_norm");
      fill_norm(L.post_mlp_norm, spec.hidden, tensor++, p + "post_mlp_norm");
      fill_norm(L.scalar, 1, tensor++, p + "scalar");
      fill_fp8(L.qkv, L.packed_width(), spec.hidden, false, tensor++, scales + 0, p + "qkv");
      fill_fp8(L.o, spec.hidden, L.query_width(), false, tensor++, scales + 1, p + "o");
      fill_fp8(L.gate_up, 2 * spec.intermediate, spec.hidden, true, tensor++, scales + 2,
               p + "gate_up");
      fill_fp8(L.down, spec.hidden, spec.intermediate, false, tensor++, scales + 3, p + "down");
      const size_t cache_elems =
          static_cast<size_t>(batch_size) * L.kv_width() * static_cast<size_t>(L.capacity);
      L.k_cache.allocate(sizeof(bf16_t) * cache_elems);
      L.v_cache.allocate(sizeof(bf16_t) * cache_elems);
      hip_check(hipMemsetAsync(L.k_cache.get(), 0, L.k_cache.bytes(), stream), "zero K cache");
      hip_check(hipMemsetAsync(L.v_cache.get(), 0, L.v_cache.bytes(), stream), "zero V cache");
      const size_t new_elems = static_cast<size_t>(step_rows) * L.kv_width();
      L.k_new.allocate(sizeof(bf16_t) * new_elems);
      L.v_new.allocate(sizeof(bf16_t) * new_elems);
      if (L.spec.sliding) {
        ++sliding_layer_count;
        last_sliding = static_cast<int>(i);
        rope_sliding_dim = D;
      } else {
        last_global = static_cast<int>(i);
        rope_global_dim = D;
      }
    }
    fill_bf16(embedding_bf16, static_cast<size_t>(spec.vocabulary) * H, 1, 1.0f, "token_embedding");
    embedding_scale.allocate(sizeof(float));
    const size_t embedding_count = static_cast<size_t>(spec.vocabulary) * H;
    if (spec.fp8_scaling != 0) {
      lm_head.scaling = spec.fp8_scaling;
      const size_t floats = fp8_weight_scale_elements(lm_head.scaling, spec.vocabulary, spec.hidden);
      lm_head.scale_kblocks = lm_head.scaling == 2
                                  ? static_cast<int>(floats / ((static_cast<size_t>(spec.vocabulary) + 127) / 128))
                                  : 0;
      lm_head.scale_table.allocate(sizeof(float) * floats);
      if (!copy_device_fp8("token_embedding", staging_for(embedding_count), embedding_count,
                           lm_head.scale_table.as<float>(), floats))
        quantize_weight_bf16_to_fp8_scaled(embedding_bf16.as<bf16_t>(),
                                           static_cast<fp8_t *>(staging_for(embedding_count)),
                                           spec.vocabulary, spec.hidden, lm_head.scaling,
                                           lm_head.scale_table.as<float>(), init_scratch.as<float>(),
                                           stream);
    } else if (!copy_device_fp8("token_embedding", staging_for(embedding_count), embedding_count,
                                embedding_scale.as<float>()))
      quantize_weight_bf16_to_fp8(embedding_bf16.as<bf16_t>(),
                                  static_cast<fp8_t *>(staging_for(embedding_count)),
                                  embedding_count, embedding_scale.as<float>(),
                                  init_scratch.as<float>(), stream);
    pack_from_staging(lm_head, spec.vocabulary, spec.hidden, false);
    fill_norm(final_norm, spec.hidden, 2, "final_norm");
    upload_rope();
  }

  void upload_rope() {
    auto upload = [&](int dimension, bool proportional, DeviceBuffer &cos_buffer,
                      DeviceBuffer &sin_buffer) {
      if (dimension == 0) return;
      std::vector<bf16_t> c, s;
      rope_table(dimension, proportional, maximum_context, c, s);
      cos_buffer.allocate(c.size() * sizeof(bf16_t));
      sin_buffer.allocate(s.size() * sizeof(bf16_t));
      hip_check(hipMemcpy(cos_buffer.get(), c.data(), c.size() * sizeof(bf16_t),
                          hipMemcpyHostToDevice),
                "upload RoPE cosine");
      hip_check(hipMemcpy(sin_buffer.get(), s.data(), s.size() * sizeof(bf16_t),
                          hipMemcpyHostToDevice),
                "upload RoPE sine");
    };
    upload(rope_sliding_dim, false, rope_sliding_cos, rope_sliding_sin);
    upload(rope_global_dim, true, rope_global_cos, rope_global_sin);
  }

  void allocate_assistant() {
    if (last_sliding < 0 || last_global < 0)
      throw std::runtime_error("target does not expose both assistant KV types");
    const AssistantSpec &as = spec.assistant;
    const size_t AH = static_cast<size_t>(as.hidden);
    const size_t AI = static_cast<size_t>(as.intermediate);
    const size_t H = static_cast<size_t>(spec.hidden);
    uint64_t tensor = 50000;
    assistant_fp8 = resolve_assistant_fp8_mode();
    const bool all8 = assistant_fp8 == 2;
    assistant_layers.resize(static_cast<size_t>(as.layers));
    for (int i = 0; i < as.layers; ++i) {
      AssistantLayer &L = assistant_layers[static_cast<size_t>(i)];
      L.global = i == as.layers - 1;
      const LayerSpec &target = spec.layers[static_cast<size_t>(L.global ? last_global : last_sliding)];
      L.kv_heads = target.kv_heads;
      L.head_dimension = target.head_dimension;
      if (as.query_heads % L.kv_heads != 0) throw std::runtime_error("assistant heads mismatch");
      const size_t qw = static_cast<size_t>(as.query_heads) * L.head_dimension;
      const std::string p = "assistant.layer." + std::to_string(i) + ".";
      const float sd = spec.weight_std;
      fill_norm(L.input_norm, as.hidden, tensor++, p + "input_norm");
      fill_norm(L.q_norm, L.head_dimension, tensor++, p + "q_norm");
      fill_norm(L.post_attention_norm, as.hidden, tensor++, p + "post_attention_norm");
      fill_norm(L.pre_mlp_norm, as.hidden, tensor++, p + "pre_mlp_norm");
      fill_norm(L.post_mlp_norm, as.hidden, tensor++, p + "post_mlp_norm");
      fill_norm(L.scalar, 1, tensor++, p + "scalar");
      float *scales8 = nullptr;
      if (all8) {
        L.scales8.allocate(4 * sizeof(float));
        scales8 = L.scales8.as<float>();
      }
      fill_bf16_weight(L.q, static_cast<int>(qw), as.hidden, false, tensor++, sd, p + "q",
                       all8 ? &L.q8 : nullptr, scales8);
      fill_bf16_weight(L.o, as.hidden, static_cast<int>(qw), false, tensor++, sd, p + "o",
                       all8 ? &L.o8 : nullptr, all8 ? scales8 + 1 : nullptr);
      fill_bf16_weight(L.gate_up, 2 * as.intermediate, as.hidden, true, tensor++, sd, p + "gate_up",
                       all8 ? &L.gate_up8 : nullptr, all8 ? scales8 + 2 : nullptr);
      fill_bf16_weight(L.down, as.hidden, as.intermediate, false, tensor++, sd, p + "down",
                       all8 ? &L.down8 : nullptr, all8 ? scales8 + 3 : nullptr);
    }
    float *scales8 = nullptr;
    if (assistant_fp8 != 0) {
      a_scales8.allocate(3 * sizeof(float));
      scales8 = a_scales8.as<float>();
    }
    fill_bf16_weight(a_embedding, spec.vocabulary, as.hidden, false, tensor++, spec.weight_std,
                     "assistant.token_embedding", assistant_fp8 != 0 ? &a_embedding8 : nullptr,
                     scales8);
    fill_bf16_weight(a_pre_projection, as.hidden, 2 * spec.hidden, false, tensor++,
                     spec.weight_std, "assistant.pre_projection", all8 ? &a_pre_projection8 : nullptr,
                     all8 ? scales8 + 1 : nullptr);
    fill_bf16_weight(a_post_projection, spec.hidden, as.hidden, false, tensor++, spec.weight_std,
                     "assistant.post_projection", all8 ? &a_post_projection8 : nullptr,
                     all8 ? scales8 + 2 : nullptr);
    if (assistant_fp8 != 0)
      a_amax.allocate(sizeof(float) * static_cast<size_t>(kMaximumDepth) *
                      assistant_amax_slots_per_step() * kAmaxSlotFloats);
    fill_norm(a_final_norm, as.hidden, tensor++, "assistant.final_norm");
    const size_t B = static_cast<size_t>(batch_size);
    size_t max_qw = 0;
    for (auto &L : assistant_layers)
      max_qw = std::max(max_qw, static_cast<size_t>(as.query_heads) * L.head_dimension);
    a_input.allocate(sizeof(bf16_t) * B * 2 * H);
    a_hidden_a.allocate(sizeof(bf16_t) * B * AH);
    a_hidden_b.allocate(sizeof(bf16_t) * B * AH);
    a_normalized.allocate(sizeof(bf16_t) * B * AH);
    a_first_residual.allocate(sizeof(bf16_t) * B * AH);
    a_pre_mlp.allocate(sizeof(bf16_t) * B * AH);
    a_activated.allocate(sizeof(bf16_t) * B * AI);
    a_queries.allocate(sizeof(bf16_t) * B * max_qw);
    a_attention_out.allocate(sizeof(bf16_t) * B * max_qw);
    a_final_hidden.allocate(sizeof(bf16_t) * B * AH);
    a_previous_hidden.allocate(sizeof(bf16_t) * B * H);
    a_io.allocate(sizeof(int32_t) * B * (5 + kMaximumDepth));
    hip_check(hipHostMalloc(reinterpret_cast<void **>(&a_host_io), sizeof(int32_t) * B * (5 + kMaximumDepth)),
              "allocate pinned assistant staging");
    a_tokens = a_io.as<int32_t>();
    a_outputs = a_tokens + B;
    a_forced = a_outputs + B;
    a_context = a_forced + B;
    a_slots = a_context + B;
    a_proposals = a_slots + B;
    has_assistant = true;
  }

  static int splits_for(const WeightLayout &l) {
    return gemm_choose_splits(gemm_blocks_n(l), l.row_bytes / 128);
  }
  static size_t gemm_partial_floats(const PackedWeight &w, int rows) {
    return static_cast<size_t>(splits_for(w.layout)) * rows * w.layout.n;
  }

  void allocate_workspaces() {
    const size_t M = static_cast<size_t>(step_rows);
    const size_t H = static_cast<size_t>(spec.hidden);
    const size_t I = static_cast<size_t>(spec.intermediate);
    size_t max_qw = 0;
    size_t partial = 0;
    for (auto &L : layers) {
      max_qw = std::max(max_qw, static_cast<size_t>(L.query_width()));
      partial = std::max(partial, gemm_partial_floats(L.qkv, step_rows));
      partial = std::max(partial, gemm_partial_floats(L.o, step_rows));
      partial = std::max(partial, gemm_partial_floats(L.down, step_rows));
    }
    if (has_assistant) {
      partial = std::max(partial, gemm_partial_floats(a_pre_projection, batch_size));
      partial = std::max(partial, gemm_partial_floats(a_post_projection, batch_size));
      for (auto &L : assistant_layers) {
        partial = std::max(partial, gemm_partial_floats(L.q, batch_size));
        partial = std::max(partial, gemm_partial_floats(L.o, batch_size));
        partial = std::max(partial, gemm_partial_floats(L.down, batch_size));
        if (assistant_fp8 == 2) {
          partial = std::max(partial, gemm_partial_floats(L.q8, batch_size));
          partial = std::max(partial, gemm_partial_floats(L.o8, batch_size));
          partial = std::max(partial, gemm_partial_floats(L.down8, batch_size));
        }
      }
      if (assistant_fp8 == 2) {
        partial = std::max(partial, gemm_partial_floats(a_pre_projection8, batch_size));
        partial = std::max(partial, gemm_partial_floats(a_post_projection8, batch_size));
      }
    }
    hidden_a.allocate(sizeof(bf16_t) * M * H);
    hidden_b.allocate(sizeof(bf16_t) * M * H);
    normalized.allocate(sizeof(bf16_t) * M * H);
    first_residual.allocate(sizeof(bf16_t) * M * H);
    pre_mlp.allocate(sizeof(bf16_t) * M * H);
    activated.allocate(sizeof(bf16_t) * M * I);
    queries.allocate(sizeof(bf16_t) * M * max_qw);
    attention_out.allocate(sizeof(bf16_t) * M * max_qw);
    final_hidden.allocate(sizeof(bf16_t) * M * H);
    partials.allocate(sizeof(float) * partial);
    // per-tensor amax slots (four per layer, eight more), then two fused-quantisation sync slots
    // per layer; step_init clears all of them
    amax.allocate(sizeof(float) * amax_slot_count() * kAmaxSlotFloats);
    {
      size_t xp = std::max(gemm_xprep_bytes(step_rows, spec.hidden),
                           gemm_xprep_bytes(step_rows, spec.intermediate));
      for (auto &L : layers) xp = std::max(xp, gemm_xprep_bytes(step_rows, L.query_width()));
      if (assistant_fp8 != 0) {
        const AssistantSpec &as = spec.assistant;
        for (const int k : {2 * spec.hidden, as.hidden, as.intermediate})
          xp = std::max(xp, gemm_xprep_bytes(batch_size, k));
        for (auto &L : assistant_layers)
          xp = std::max(xp, gemm_xprep_bytes(batch_size, as.query_heads * L.head_dimension));
      }
      xprep.allocate(xp);
      if (spec.fp8_scaling != 0) {
        size_t xs = std::max(gemm_x_scale_floats(step_rows, spec.hidden),
                             gemm_x_scale_floats(step_rows, spec.intermediate));
        for (auto &L : layers) xs = std::max(xs, gemm_x_scale_floats(step_rows, L.query_width()));
        x_scales.allocate(sizeof(float) * xs);
      }
      size_t keys = gemm_argmax_partials(step_rows, lm_head.layout);
      if (has_assistant) keys = std::max(keys, gemm_argmax_partials(batch_size, a_embedding.layout));
      if (assistant_fp8 != 0) keys = std::max(keys, gemm_argmax_partials(batch_size, a_embedding8.layout));
      argmax_partials.allocate(sizeof(uint64_t) * keys);
    }
    target_hidden.allocate(sizeof(bf16_t) * static_cast<size_t>(batch_size) * H);
    hip_check(hipMemsetAsync(target_hidden.get(), 0, target_hidden.bytes(), stream), "zero hidden");

    // attention: the chunk is chosen for the largest key count; the same chunk serves every call.
    int sliding_kv_heads = 1, global_kv_heads = 1;
    for (auto &L : layers) {
      int &kind = L.spec.sliding ? sliding_kv_heads : global_kv_heads;
      kind = std::max(kind, L.spec.kv_heads);
    }
    attention_chunk_sliding = attention_default_chunk(AttentionMode::sliding,
                                                      spec.sliding_window + kMaximumDepth,
                                                      batch_size, sliding_kv_heads);
    attention_chunk_global = attention_default_chunk(AttentionMode::global, maximum_context,
                                                     batch_size, global_kv_heads);
    // Partials of one call, per layer: requests x (its G x rows, rounded up to the kernel's query
    // tiles: at most 47 rows more per request) rows of kv heads x chunks x (D + 2) floats.
    attention_partial_floats = 0;
    for (auto &L : layers) {
      const int chunk = L.spec.sliding ? attention_chunk_sliding : attention_chunk_global;
      const int keys = L.spec.sliding ? std::min(spec.sliding_window, L.capacity) + step_rows
                                      : maximum_context;
      const int group = L.spec.query_heads / L.spec.kv_heads;
      attention_partial_floats = std::max(
          attention_partial_floats,
          attention_partials_floats(1, L.spec.kv_heads, keys, chunk,
                                    group * step_rows + 48 * batch_size, L.spec.head_dimension));
    }
    if (has_assistant)
      for (auto &L : assistant_layers) {
        const TargetLayer &target = layers[static_cast<size_t>(L.global ? last_global : last_sliding)];
        L.attention_chunk = attention_default_chunk(AttentionMode::decode, target.capacity, batch_size,
                                                    L.kv_heads, false, L.head_dimension);
        attention_partial_floats = std::max(
            attention_partial_floats,
            attention_partials_floats(batch_size, L.kv_heads, target.capacity, L.attention_chunk,
                                      spec.assistant.query_heads / L.kv_heads, L.head_dimension));
      }
    attention_partials.allocate(sizeof(float) * attention_partial_floats);

    // sliding-layer commit table
    std::vector<SlidingLayerKv> table;
    for (auto &L : layers) {
      if (!L.spec.sliding) continue;
      table.push_back(SlidingLayerKv{L.k_new.as<bf16_t>(), L.v_new.as<bf16_t>(),
                                     L.k_cache.as<bf16_t>(), L.v_cache.as<bf16_t>(),
                                     L.spec.kv_heads, L.spec.head_dimension, L.capacity, 0});
    }
    sliding_table.allocate(sizeof(SlidingLayerKv) * std::max<size_t>(1, table.size()));
    if (!table.empty())
      hip_check(hipMemcpy(sliding_table.get(), table.data(), table.size() * sizeof(SlidingLayerKv),
                          hipMemcpyHostToDevice),
                "upload sliding-layer table");

    // I/O block: tokens[M] positions[B] slots[B] first[B] caps[B] accepted[B] next[B] pred[M]
    // fault[1] (set by a fused quantisation whose wait exceeded its bound)
    io_ints = 2 * M + 6 * static_cast<size_t>(batch_size) + 1;
    device_io.allocate(sizeof(int32_t) * io_ints);
    hip_check(hipHostMalloc(reinterpret_cast<void **>(&host_io), sizeof(int32_t) * io_ints),
              "allocate pinned staging");
    int32_t *base = device_io.as<int32_t>();
    d_tokens = base;
    d_positions = d_tokens + M;
    d_slots = d_positions + batch_size;
    d_first = d_slots + batch_size;
    d_caps = d_first + batch_size;
    d_accepted = d_caps + batch_size;
    d_next = d_accepted + batch_size;
    d_predictions = d_next + batch_size;
    d_fault = d_predictions + M;
  }

  // Per-tensor amax slots, kAmaxStripes stripes each (four per layer, then the lm_head input).
  float *amax_slot(size_t layer, int which) {
    return amax.as<float>() + (layer * 4 + which) * kAmaxSlotFloats;
  }
  float *lm_head_amax() { return amax.as<float>() + layers.size() * 4 * kAmaxSlotFloats; }
  size_t amax_slot_count() const { return layers.size() * 6 + 8; }
  // The two sync slots of layer li's fused layer-end quantisations (0: after O, 1: after down).
  unsigned *sync_slot(size_t layer, int which) {
    return reinterpret_cast<unsigned *>(amax.as<float>() +
                                        (layers.size() * 4 + 8 + layer * 2 + which) * kAmaxSlotFloats);
  }

  void run_fp8_gemm(const bf16_t *x, int rows, int k, const float *x_amax, const PackedWeight &w,
                    const float *w_scale, GemmEpilogue epilogue, bf16_t *y, float *y_amax,
                    int *splits_out, int kind, bool xprep_ready = false) {
    GemmArgs g;
    g.xprep_ready = xprep_ready;
    std::tie(g.timing_start, g.timing_stop) = probe(kind);
    g.x = x;
    g.ldx = k;
    g.m = rows;
    g.k = k;
    g.x_amax = x_amax;
    g.w = w.get();
    g.n = w.layout.n;
    g.w_layout = w.layout;
    g.w_scale = w_scale;
    g.epilogue = epilogue;
    g.y = y;
    g.ldy = epilogue == GemmEpilogue::gelu_gate ? g.n / 2 : g.n;
    g.y_amax = y_amax;
    g.amax_stripes = kAmaxStripes;
    g.partial = partials.as<float>();
    g.argmax_partials = argmax_partials.as<uint64_t>();
    g.argmax_partial_capacity = argmax_partials.bytes() / sizeof(uint64_t);
    g.argmax_out = d_predictions;
    g.xprep = xprep.as<unsigned char>();
    g.xprep_capacity = xprep.bytes();
    if (w.scaling != 0) {
      g.scaling = w.scaling;
      g.w_scales = w.scale_table.as<float>();
      g.w_scale_kblocks = w.scale_kblocks;
      g.x_scales = x_scales.as<float>();
      g.x_scales_capacity = x_scales.bytes() / sizeof(float);
      g.xprep_ready = false;
    }
    if (epilogue == GemmEpilogue::partial_f32) g.k_splits = splits_for(w.layout);
    if (splits_out != nullptr) *splits_out = g.k_splits;
    launch_fp8_gemm(g, stream);
  }

  int run_bf16_gemm_partial(const bf16_t *x, int rows, int k, const PackedWeight &w) {
    GemmArgs g;
    g.x = x;
    g.ldx = k;
    g.m = rows;
    g.k = k;
    g.w = w.get();
    g.n = w.layout.n;
    g.w_layout = w.layout;
    g.epilogue = GemmEpilogue::partial_f32;
    g.partial = partials.as<float>();
    g.k_splits = splits_for(w.layout);
    launch_bf16_gemm(g, stream);
    return g.k_splits;
  }

  // Back-to-back launches of one per-layer fp8 GEMM kind over every layer (see the header).
  float stream_gemm_probe(int kind, int passes, int *launches) {
    if (last_rows <= 0) throw std::runtime_error("stream probe needs a verify call first");
    const bool attention = kind == probe_sliding_attention || kind == probe_global_attention;
    if (passes <= 0 || ((kind < probe_qkv_gemm || kind > probe_down_gemm) && !attention))
      throw std::runtime_error("invalid stream probe");
    const int rows = last_rows;
    auto launch = [&](size_t li, bool prepared) {
      TargetLayer &L = layers[li];
      const float *scales = L.scales.as<float>();
      switch (kind) {
      case probe_sliding_attention:
      case probe_global_attention:
        if (L.spec.sliding == (kind == probe_sliding_attention))
          launch_attention(layer_attention(li, last_requests, last_depth, d_positions, d_slots), stream);
        break;
      case probe_qkv_gemm:
        run_fp8_gemm(normalized.as<bf16_t>(), rows, spec.hidden, amax_slot(li, 0), L.qkv, scales + 0,
                     GemmEpilogue::partial_f32, nullptr, nullptr, nullptr, probe_none, prepared);
        break;
      case probe_o_gemm:
        run_fp8_gemm(attention_out.as<bf16_t>(), rows, L.query_width(), amax_slot(li, 1), L.o,
                     scales + 1, GemmEpilogue::partial_f32, nullptr, nullptr, nullptr, probe_none,
                     prepared);
        break;
      case probe_gate_up_gemm:
        run_fp8_gemm(pre_mlp.as<bf16_t>(), rows, spec.hidden, amax_slot(li, 2), L.gate_up, scales + 2,
                     GemmEpilogue::gelu_gate, activated.as<bf16_t>(), nullptr, nullptr, probe_none,
                     prepared);
        break;
      default:
        run_fp8_gemm(activated.as<bf16_t>(), rows, spec.intermediate, amax_slot(li, 3), L.down,
                     scales + 3, GemmEpilogue::partial_f32, nullptr, nullptr, nullptr, probe_none,
                     prepared);
        break;
      }
    };
    if (!attention) launch(0, false);  // prepares the activation operand once
    struct Events {  // destroyed on every exit, errors included
      hipEvent_t start = nullptr, stop = nullptr;
      ~Events() {
        if (start != nullptr) (void)hipEventDestroy(start);
        if (stop != nullptr) (void)hipEventDestroy(stop);
      }
    } ev;
    hip_check(hipEventCreate(&ev.start), "create probe event");
    hip_check(hipEventCreate(&ev.stop), "create probe event");
    hipEvent_t start = ev.start, stop = ev.stop;
    hip_check(hipEventRecord(start, stream), "record probe");
    for (int pass = 0; pass < passes; ++pass)
      for (size_t li = 0; li < layers.size(); ++li) launch(li, true);
    hip_check(hipEventRecord(stop, stream), "record probe");
    hip_check(hipEventSynchronize(stop), "probe sync");
    float ms = 0.0f;
    hip_check(hipEventElapsedTime(&ms, start, stop), "probe time");
    size_t per_pass = layers.size();
    if (attention) {
      per_pass = 0;
      for (auto &L : layers) per_pass += L.spec.sliding == (kind == probe_sliding_attention) ? 1 : 0;
      if (per_pass == 0) throw std::runtime_error("stream probe: the model has no layer of that kind");
    }
    *launches = passes * static_cast<int>(per_pass);
    return ms / static_cast<float>(*launches);
  }

  // ------------------------------------------------------------------------------- verify
  // Device operands of one step (a verify step, or one step of a forced prefill) through a
  // layer. `input` and `output` (the residual stream) may alias; `normalized` is the layer's
  // normalized input, with its amax in `in_amax`.
  struct StepIo {
    int requests = 0, depth = 0;
    const int32_t *positions = nullptr, *slots = nullptr;
    bf16_t *input = nullptr, *output = nullptr, *normalized = nullptr;
    float *in_amax = nullptr;
    // the layer-end rows quantise their output for the next GEMM themselves (verify steps of
    // <= kFusedQuantizeRows rows; sync slots and the fault flag cleared by this step's step_init)
    bool fused_quantize = false;
    bool input_prepared = false;  // the xprep workspace already holds `normalized`, quantised
  };

  // Verify attention of layer li over one step's rows (queries, this step's K/V rows and the
  // layer's cache; output and its amax into the step's buffers).
  AttentionArgs layer_attention(size_t li, int requests, int depth, const int32_t *positions,
                                const int32_t *slots) {
    TargetLayer &L = layers[li];
    AttentionArgs at;
    at.amax_stripes = kAmaxStripes;
    at.mode = L.spec.sliding ? AttentionMode::sliding : AttentionMode::global;
    at.q = queries.as<bf16_t>();
    at.k_cache = L.k_cache.get();
    at.v_cache = L.v_cache.get();
    at.k_new = L.k_new.get();
    at.v_new = L.v_new.get();
    at.slots = slots;
    at.slot_count = batch_size;
    at.positions = positions;
    at.requests = requests;
    at.tokens = depth;
    at.query_heads = L.spec.query_heads;
    at.kv_heads = L.spec.kv_heads;
    at.dimension = L.spec.head_dimension;
    at.capacity = L.capacity;
    at.window = std::min(spec.sliding_window, L.capacity);
    at.max_keys = L.spec.sliding ? at.window + depth - 1 : maximum_context;
    at.out = attention_out.as<bf16_t>();
    at.out_amax = amax_slot(li, 1);
    at.partials = attention_partials.as<float>();
    at.chunk_keys = L.spec.sliding ? attention_chunk_sliding : attention_chunk_global;
    return at;
  }

  // Layer li over one step's rows: QKV projection and post-processing (global rows go straight to
  // the cache, sliding rows to the layer's k_new/v_new for the commit), attention, O projection,
  // MLP and the residual; the next layer's normalized input (the final norm after the last layer)
  // goes to next_normalized with its amax in next_amax. The per-layer amax slots 1..3 are this
  // step's (amax_slot).
  // Returns whether next_normalized also went out quantised into the xprep workspace.
  bool enqueue_layer(size_t li, const StepIo &io, bf16_t *next_normalized, float *next_amax) {
    const int rows = io.requests * io.depth;
    // Each layer-end row quantises its output only where the row kernel has the fused shape
    // (otherwise the next GEMM prepares its operand itself, with the same bytes).
    auto fuse_quantize = [&](RowArgs &r, int which) {
      if (!io.fused_quantize || spec.fp8_scaling != 0 || !row_kernel_can_fuse_quantization(r))
        return false;
      r.xprep = xprep.as<unsigned char>();
      r.sync = sync_slot(li, which);
      r.fault = d_fault;
      r.quantize_spins = fused_quantize_mode == 2 ? 0 : kFusedQuantizeSpins;
      return true;
    };
    TargetLayer &L = layers[li];
    const float *scales = L.scales.as<float>();
    const int D = L.spec.head_dimension;
    // Channel / block-scaled GEMMs leave fully scaled partials: their consumers get no scale
    // operands (scale 1).
    const bool tensor_scaled = spec.fp8_scaling == 0;
    auto consumer_amax = [&](const float *x_amax) { return tensor_scaled ? x_amax : nullptr; };
    auto consumer_scale = [&](int i) { return tensor_scaled ? scales + i : nullptr; };
    // QKV projection
    int splits = 1;
    run_fp8_gemm(io.normalized, rows, spec.hidden, io.in_amax, L.qkv,
                 scales + 0, GemmEpilogue::partial_f32, nullptr, nullptr,
                 &splits, probe_qkv_gemm, io.input_prepared);
    QkvArgs q;
    q.amax_stripes = kAmaxStripes;
    q.partials = partials.as<float>();
    q.splits = splits;
    q.x_amax = consumer_amax(io.in_amax);
    q.w_scale = consumer_scale(0);
    q.rows = rows;
    q.tokens = io.depth;
    q.query_heads = L.spec.query_heads;
    q.kv_heads = L.spec.kv_heads;
    q.dimension = D;
    q.key_equals_value = L.spec.key_equals_value;
    q.eps = spec.eps;
    q.q_norm = L.q_norm.as<bf16_t>();
    q.k_norm = L.k_norm.as<bf16_t>();
    q.cosine = L.spec.sliding ? rope_sliding_cos.as<bf16_t>() : rope_global_cos.as<bf16_t>();
    q.sine = L.spec.sliding ? rope_sliding_sin.as<bf16_t>() : rope_global_sin.as<bf16_t>();
    q.positions = io.positions;
    q.slots = io.slots;
    q.q_out = queries.as<bf16_t>();
    q.k_new = L.k_new.as<bf16_t>();
    q.v_new = L.v_new.as<bf16_t>();
    if (!L.spec.sliding) {
      // Global rows go straight to the cache (stale tails past `accepted` stay unreachable,
      // batch_model_runner.h:52-54); sliding rows wait for the commit.
      q.k_cache = L.k_cache.as<bf16_t>();
      q.v_cache = L.v_cache.as<bf16_t>();
      q.capacity = L.capacity;
    }
    AttentionArgs at = layer_attention(li, io.requests, io.depth, io.positions, io.slots);
    // The attention kernel post-processes its own (request, kv head)'s QKV rows where it can
    // (same arithmetic, one launch fewer per layer); otherwise the separate kernel runs first.
    at.qkv = q;
    at.fuse_qkv = qkv_fusion && attention_can_fuse_qkv(at);
    if (!at.fuse_qkv) launch_qkv_post(q, stream);
    std::tie(at.timing_start, at.timing_stop) =
        probe(L.spec.sliding ? probe_sliding_attention : probe_global_attention);
    launch_attention(at, stream);
    // O projection + post-attention norm + residual + pre-MLP norm
    run_fp8_gemm(attention_out.as<bf16_t>(), rows, L.query_width(), amax_slot(li, 1),
                 L.o, scales + 1, GemmEpilogue::partial_f32, nullptr,
                 nullptr, &splits, probe_o_gemm);
    RowArgs ro;
    ro.amax_stripes = kAmaxStripes;
    ro.source = RowSource::partials;
    ro.rows = rows;
    ro.width = spec.hidden;
    ro.eps = spec.eps;
    ro.partials = partials.as<float>();
    ro.splits = splits;
    ro.x_amax = consumer_amax(amax_slot(li, 1));
    ro.w_scale = consumer_scale(1);
    ro.w1 = L.post_attention_norm.as<bf16_t>();
    ro.residual = io.input;
    ro.r1_out = first_residual.as<bf16_t>();
    ro.w2 = L.pre_mlp_norm.as<bf16_t>();
    ro.y_out = pre_mlp.as<bf16_t>();
    ro.y_amax = amax_slot(li, 2);
    const bool pre_mlp_prepared = fuse_quantize(ro, 0);
    launch_row_kernel(ro, stream);
    // gate/up with the GELU gate fused
    run_fp8_gemm(pre_mlp.as<bf16_t>(), rows, spec.hidden, amax_slot(li, 2), L.gate_up,
                 scales + 2, GemmEpilogue::gelu_gate,
                 activated.as<bf16_t>(), amax_slot(li, 3), nullptr, probe_gate_up_gemm,
                 pre_mlp_prepared);
    // down + post-MLP norm + residual + layer scalar + next input norm
    run_fp8_gemm(activated.as<bf16_t>(), rows, spec.intermediate, amax_slot(li, 3),
                 L.down, scales + 3, GemmEpilogue::partial_f32, nullptr,
                 nullptr, &splits, probe_down_gemm);
    RowArgs rd;
    rd.amax_stripes = kAmaxStripes;
    rd.source = RowSource::partials;
    rd.rows = rows;
    rd.width = spec.hidden;
    rd.eps = spec.eps;
    rd.partials = partials.as<float>();
    rd.splits = splits;
    rd.x_amax = consumer_amax(amax_slot(li, 3));
    rd.w_scale = consumer_scale(3);
    rd.w1 = L.post_mlp_norm.as<bf16_t>();
    rd.residual = first_residual.as<bf16_t>();
    rd.scalar = L.scalar.as<bf16_t>();
    rd.r1_out = io.output;
    rd.w2 = li + 1 == layers.size() ? final_norm.as<bf16_t>()
                                    : layers[li + 1].input_norm.as<bf16_t>();
    rd.y_out = next_normalized;
    rd.y_amax = next_amax;
    const bool next_prepared = fuse_quantize(rd, 1);
    launch_row_kernel(rd, stream);
    return next_prepared;
  }

  void enqueue_embedding(const int32_t *tokens, int rows, bf16_t *hidden, bf16_t *normalized_out,
                         float *normalized_amax) {
    RowArgs r;
    r.amax_stripes = kAmaxStripes;
    r.source = RowSource::embedding;
    r.rows = rows;
    r.width = spec.hidden;
    r.eps = spec.eps;
    r.embedding = embedding_bf16.as<bf16_t>();
    r.tokens = tokens;
    r.vocabulary = spec.vocabulary;
    r.embed_scale = std::sqrt(static_cast<float>(spec.hidden));
    r.v_out = hidden;
    r.w2 = layers[0].input_norm.as<bf16_t>();
    r.y_out = normalized_out;
    r.y_amax = normalized_amax;
    launch_row_kernel(r, stream);
  }

  // Greedy acceptance (or, forced, every row) and the commit of this step's rows of the sliding
  // layers [first_sliding, first_sliding + sliding_count); hands final_hidden's last accepted row
  // of each request to the slot when final_hidden is given.
  void enqueue_accept(int requests, int depth, bool has_caps, bool force_accept,
                      const int32_t *positions, const int32_t *slots, int first_sliding,
                      int sliding_count, const bf16_t *final_rows,
                      bool predictions_missing = false) {
    AcceptArgs ac;
    ac.predictions = d_predictions;
    ac.predictions_missing = predictions_missing;
    ac.proposals = d_tokens;
    ac.target_first = d_first;
    ac.caps = has_caps ? d_caps : nullptr;
    ac.requests = requests;
    ac.tokens = depth;
    ac.accepted = d_accepted;
    ac.next_tokens = d_next;
    ac.layers = sliding_table.as<SlidingLayerKv>() + first_sliding;
    ac.layer_count = sliding_count;
    ac.slots = slots;
    ac.positions = positions;
    ac.final_hidden = final_rows;
    ac.target_hidden = target_hidden.as<bf16_t>();
    ac.hidden = spec.hidden;
    ac.force_accept = force_accept;
    launch_accept_commit(ac, stream);
  }

  void enqueue_verify(int requests, int depth, bool has_caps, bool force_accept = false,
                      bool lm_head_pass = true) {
    const int rows = requests * depth;
    last_rows = rows;
    last_requests = requests;
    last_depth = depth;
    launch_step_init(amax.as<float>(), static_cast<int>(amax_slot_count() * kAmaxStripes), stream,
                     d_fault);
    enqueue_embedding(d_tokens, rows, hidden_a.as<bf16_t>(), normalized.as<bf16_t>(),
                      amax_slot(0, 0));
    StepIo io;
    io.requests = requests;
    io.depth = depth;
    io.positions = d_positions;
    io.slots = d_slots;
    io.input = hidden_a.as<bf16_t>();
    io.output = hidden_b.as<bf16_t>();
    io.normalized = normalized.as<bf16_t>();
    io.fused_quantize = fused_quantize_mode != 0;
    for (size_t li = 0; li < layers.size(); ++li) {
      io.in_amax = amax_slot(li, 0);
      const bool last = li + 1 == layers.size();
      const bool prepared = enqueue_layer(
          li, io, last ? final_hidden.as<bf16_t>() : normalized.as<bf16_t>(),
          last ? lm_head_amax() : amax_slot(li + 1, 0));
      io.input_prepared = prepared && !last;
      if (last) last_input_prepared = prepared;
      std::swap(io.input, io.output);
    }
    // lm_head + argmax (a forced prefill step whose predictions nobody reads skips it; the
    // acceptance then writes -1 predictions and next tokens)
    if (lm_head_pass)
      run_fp8_gemm(final_hidden.as<bf16_t>(), rows, spec.hidden, lm_head_amax(),
                   lm_head, embedding_scale.as<float>(),
                   GemmEpilogue::argmax, nullptr, nullptr, nullptr, probe_lm_head_gemm,
                   last_input_prepared);
    enqueue_accept(requests, depth, has_caps, force_accept, d_positions, d_slots, 0,
                   sliding_layer_count, final_hidden.as<bf16_t>(), !lm_head_pass);
  }

  // batch_model_runner.cu:1544-1615: one decode step per slot at its current position. It is a
  // verify step of depth 1 whose only row is the forced input token (accepted = 1): the same
  // kernels write the position's K/V rows, hand the hidden state off and return the argmax.
  std::vector<int> append_ragged(const std::vector<int> &tokens, const std::vector<int> &slots) {
    const int active = static_cast<int>(tokens.size());
    if (active <= 0 || active > batch_size || slots.size() != tokens.size())
      throw std::runtime_error("invalid ragged token batch");
    std::vector<bool> seen(static_cast<size_t>(batch_size), false);
    std::vector<std::vector<int>> rows(static_cast<size_t>(active));
    for (int r = 0; r < active; ++r) {
      const int slot = slots[static_cast<size_t>(r)];
      const int token = tokens[static_cast<size_t>(r)];
      if (slot < 0 || slot >= batch_size || seen[static_cast<size_t>(slot)] || token < 0 ||
          token >= spec.vocabulary)
        throw std::runtime_error("invalid or repeated ragged slot");
      seen[static_cast<size_t>(slot)] = true;
      const int position = slot_positions[static_cast<size_t>(slot)];
      if (position <= 0 || position >= maximum_context)
        throw std::runtime_error("ragged slot is empty or full");
      rows[static_cast<size_t>(r)] = {token};
    }
    return verify(rows, tokens, slots, {}).next_tokens;
  }

  // ------------------------------------------------------------------------------ prefill
  // Prompts run through the verify kernels as forced steps (force_accept: every row is
  // committed, next_tokens is the prediction after a request's last row; the slots may be empty).
  // A step holds every request that still has rows: up to step_rows / active rows each, never
  // more rows than the smallest sliding ring (the commit writes each ring entry once per step),
  // never more than any active request has left. The fp8 activation scales are per step.

  // Error texts of one prefill entry point (batch_model_runner.cu:1062-1091, 1127-1166,
  // 1219-1262, 1358-1405).
  struct PrefillMessages {
    const char *shape, *request, *extend, *token, *workspace;
  };
  static constexpr PrefillMessages kSlotChunkMessages{
      "invalid slot prefill chunk shape", "invalid slot prefill chunk shape",
      "slot prefill chunk does not extend resident context",
      "slot prompt contains an invalid token id", nullptr};
  static constexpr PrefillMessages kChunksMessages{
      "invalid batched chunk prefill shape", "invalid batched chunk prefill request",
      "batched chunk does not extend resident context", "batched chunk contains an invalid token id",
      "batched chunks exceed shared projection workspace"};
  static constexpr PrefillMessages kSuffixMessages{
      "invalid batched suffix prefill shape", "invalid batched suffix prefill request",
      "batched suffix does not extend resident context", "batched suffix contains an invalid token id",
      "batched suffix exceeds shared projection workspace"};
  static constexpr PrefillMessages kSliceMessages{
      "invalid layer-sliced suffix prefill shape", "invalid layer-sliced suffix request",
      "layer-sliced suffix does not extend resident context",
      "layer-sliced suffix contains an invalid token id",
      "layer-sliced suffix exceeds shared projection workspace"};

  struct PrefillStep {
    std::vector<size_t> requests;  // cohort indices
    std::vector<int> positions;    // their positions at the step
    int depth = 0;
  };

  // Validates a cohort (each prompt advancing from its slot's position by at most chunk_tokens)
  // and returns each request's [position, end).
  void prefill_cohort(const std::vector<int> &slots,
                      const std::vector<const std::vector<int> *> &prompts, int chunk_tokens,
                      const PrefillMessages &m, std::vector<int> &position, std::vector<int> &end) {
    const size_t n = slots.size();
    if (n == 0 || n > static_cast<size_t>(batch_size) || prompts.size() != n || chunk_tokens <= 0)
      throw std::runtime_error(m.shape);
    std::vector<bool> seen(static_cast<size_t>(batch_size), false);
    position.assign(n, 0);
    end.assign(n, 0);
    size_t packed = 0;
    for (size_t r = 0; r < n; ++r) {
      const int slot = slots[r];
      const std::vector<int> *prompt = prompts[r];
      if (slot < 0 || slot >= batch_size || seen[static_cast<size_t>(slot)] || prompt == nullptr ||
          prompt->empty() || prompt->size() > static_cast<size_t>(maximum_context))
        throw std::runtime_error(m.request);
      seen[static_cast<size_t>(slot)] = true;
      position[r] = slot_positions[static_cast<size_t>(slot)];
      if (position[r] < 0 || position[r] >= static_cast<int>(prompt->size()))
        throw std::runtime_error(m.extend);
      end[r] = static_cast<int>(std::min<int64_t>(static_cast<int64_t>(prompt->size()),
                                                  int64_t{position[r]} + chunk_tokens));
      for (int i = position[r]; i < end[r]; ++i) {
        const int token = (*prompt)[static_cast<size_t>(i)];
        if (token < 0 || token >= spec.vocabulary) throw std::runtime_error(m.token);
      }
      packed += static_cast<size_t>(end[r] - position[r]);
    }
    if (m.workspace != nullptr && packed > static_cast<size_t>(maximum_context))
      throw std::runtime_error(m.workspace);
  }

  std::vector<PrefillStep> prefill_plan(std::vector<int> position, const std::vector<int> &end) const {
    int ring = step_rows;
    for (const auto &L : layers)
      if (L.spec.sliding) ring = std::min(ring, L.capacity);
    std::vector<PrefillStep> steps;
    for (;;) {
      PrefillStep step;
      for (size_t r = 0; r < position.size(); ++r)
        if (position[r] < end[r]) step.requests.push_back(r);
      if (step.requests.empty()) break;
      step.depth = std::min(ring, step_rows / static_cast<int>(step.requests.size()));
      for (size_t r : step.requests) step.depth = std::min(step.depth, end[r] - position[r]);
      for (size_t r : step.requests) {
        step.positions.push_back(position[r]);
        position[r] += step.depth;
      }
      steps.push_back(std::move(step));
    }
    return steps;
  }

  // Step by step, every layer per step (batch_model_runner.cu prefill_slot_chunk /
  // prefill_slots_chunks / prefill_slots_suffix). An entry holds the greedy next token only
  // when that request's whole prompt is resident.
  std::vector<std::optional<int>> prefill_chunks(const std::vector<int> &slots,
                                                 const std::vector<const std::vector<int> *> &prompts,
                                                 int chunk_tokens, const PrefillMessages &m) {
    std::vector<int> position, end;
    prefill_cohort(slots, prompts, chunk_tokens, m, position, end);
    const size_t n = slots.size();
    std::vector<int> last(n, -1);
    for (const PrefillStep &step : prefill_plan(position, end)) {
      std::vector<std::vector<int>> rows;
      std::vector<int> first, step_slots;
      for (size_t i = 0; i < step.requests.size(); ++i) {
        const size_t r = step.requests[i];
        const auto begin = prompts[r]->begin() + step.positions[i];
        rows.emplace_back(begin, begin + step.depth);
        first.push_back(rows.back().front());
        step_slots.push_back(slots[r]);
      }
      // The lm_head runs only in a step where some request's whole prompt becomes resident.
      bool completes = false;
      for (size_t i = 0; i < step.requests.size(); ++i)
        completes |= step.positions[i] + step.depth == static_cast<int>(prompts[step.requests[i]]->size());
      const GreedyVerificationResult result = verify(rows, first, step_slots, {}, true, completes);
      for (size_t i = 0; i < step.requests.size(); ++i) last[step.requests[i]] = result.next_tokens[i];
    }
    std::vector<std::optional<int>> result(n);
    for (size_t r = 0; r < n; ++r)
      if (end[r] == static_cast<int>(prompts[r]->size())) result[r] = last[r];
    return result;
  }

  // Layer-sliced suffix prefill (batch_model_runner.cu:1356-1496): the cohort's steps are planned
  // once; each call runs the next maximum_layers layers over every step (step by step, the
  // sliding rows of those layers committed after each step) and keeps the residual stream, the
  // normalized next-layer input and its amax per step in buffers of its own, so verify or draft
  // calls on other slots may run between calls. Slot positions move when the last layer is done.
  struct SuffixSlices {
    std::vector<int> slots;
    std::vector<std::vector<int>> prompts;
    std::vector<PrefillStep> steps;
    std::vector<size_t> step_row0;  // first packed row of each step
    int next_layer = 0;
    int calls = 0;
    DeviceBuffer residual, normalized, amax, meta, tokens;  // meta: per step positions[B] slots[B]
  };
  std::unique_ptr<SuffixSlices> suffix_slices;  // null: no cohort in flight

  std::pair<bool, std::vector<int>> prefill_suffix_layer_slice(
      const std::vector<int> &slots, const std::vector<const std::vector<int> *> &prompts,
      int maximum_layers) {
    if (slots.empty() || slots.size() > static_cast<size_t>(batch_size) ||
        prompts.size() != slots.size() || maximum_layers <= 0)
      throw std::runtime_error(kSliceMessages.shape);
    const size_t n = slots.size();
    const size_t B = static_cast<size_t>(batch_size);
    if (!suffix_slices) {
      std::vector<int> position, end;
      prefill_cohort(slots, prompts, std::numeric_limits<int>::max(), kSliceMessages, position, end);
      suffix_slices.reset(new SuffixSlices);
      SuffixSlices &state = *suffix_slices;
      struct Reset {  // a failed set-up leaves no cohort in flight
        std::unique_ptr<SuffixSlices> &slices;
        bool armed = true;
        ~Reset() {
          if (armed) slices.reset();
        }
      } reset{suffix_slices};
      state.slots = slots;
      for (const auto *prompt : prompts) state.prompts.push_back(*prompt);
      state.steps = prefill_plan(position, end);
      const size_t steps = state.steps.size();
      std::vector<int32_t> meta(steps * 2 * B, 0), tokens;
      size_t rows = 0;
      for (size_t s = 0; s < steps; ++s) {
        const PrefillStep &step = state.steps[s];
        state.step_row0.push_back(rows);
        for (size_t i = 0; i < step.requests.size(); ++i) {
          const size_t r = step.requests[i];
          meta[s * 2 * B + i] = step.positions[i];
          meta[s * 2 * B + B + i] = slots[r];
          const auto begin = prompts[r]->begin() + step.positions[i];
          tokens.insert(tokens.end(), begin, begin + step.depth);
        }
        rows += step.requests.size() * static_cast<size_t>(step.depth);
      }
      const size_t H = static_cast<size_t>(spec.hidden);
      state.residual.allocate(sizeof(bf16_t) * rows * H);
      state.normalized.allocate(sizeof(bf16_t) * rows * H);
      state.amax.allocate(sizeof(float) * 2 * steps * kAmaxSlotFloats);  // [parity][step]
      state.meta.allocate(sizeof(int32_t) * meta.size());
      state.tokens.allocate(sizeof(int32_t) * tokens.size());
      hip_check(hipMemcpy(state.meta.get(), meta.data(), sizeof(int32_t) * meta.size(),
                          hipMemcpyHostToDevice),
                "copy layer-sliced suffix steps");
      hip_check(hipMemcpy(state.tokens.get(), tokens.data(), sizeof(int32_t) * tokens.size(),
                          hipMemcpyHostToDevice),
                "copy layer-sliced suffix tokens");
      launch_step_init(state.amax.as<float>(), static_cast<int>(2 * steps * kAmaxStripes), stream);
      for (size_t s = 0; s < steps; ++s) {
        const size_t row0 = state.step_row0[s];
        const int step_rows = static_cast<int>(state.steps[s].requests.size()) * state.steps[s].depth;
        enqueue_embedding(state.tokens.as<int32_t>() + row0, step_rows,
                          state.residual.as<bf16_t>() + row0 * H,
                          state.normalized.as<bf16_t>() + row0 * H,
                          state.amax.as<float>() + s * kAmaxSlotFloats);
      }
      reset.armed = false;
    } else {
      if (suffix_slices->slots != slots)
        throw std::runtime_error("layer-sliced suffix cohort changed while in flight");
      for (size_t r = 0; r < n; ++r)
        if (prompts[r] == nullptr || *prompts[r] != suffix_slices->prompts[r])
          throw std::runtime_error("layer-sliced suffix prompt changed while in flight");
    }
    SuffixSlices &state = *suffix_slices;
    const size_t steps = state.steps.size();
    const size_t H = static_cast<size_t>(spec.hidden);
    const int layer_count = static_cast<int>(layers.size());
    const int first = state.next_layer;
    const int last = std::min(layer_count, first + maximum_layers);
    const bool complete = last == layer_count;
    int first_sliding = 0, sliding_count = 0;
    for (int li = 0; li < last; ++li)
      if (layers[static_cast<size_t>(li)].spec.sliding) (li < first ? first_sliding : sliding_count) += 1;
    float *in_amax = state.amax.as<float>() + (state.calls % 2) * steps * kAmaxSlotFloats;
    float *out_amax = state.amax.as<float>() + ((state.calls + 1) % 2) * steps * kAmaxSlotFloats;
    if (!complete) launch_step_init(out_amax, static_cast<int>(steps * kAmaxStripes), stream);
    std::vector<int> predictions(n, -1);
    for (size_t s = 0; s < steps; ++s) {
      const PrefillStep &step = state.steps[s];
      const int requests = static_cast<int>(step.requests.size());
      const size_t row0 = state.step_row0[s];
      launch_step_init(amax.as<float>(), static_cast<int>(amax_slot_count() * kAmaxStripes),
                       stream);
      StepIo io;
      io.requests = requests;
      io.depth = step.depth;
      io.positions = state.meta.as<int32_t>() + s * 2 * B;
      io.slots = io.positions + B;
      io.input = io.output = state.residual.as<bf16_t>() + row0 * H;
      io.normalized = state.normalized.as<bf16_t>() + row0 * H;
      for (int li = first; li < last; ++li) {
        io.in_amax = li == first ? in_amax + s * kAmaxSlotFloats : amax_slot(static_cast<size_t>(li), 0);
        float *next_amax = li + 1 < last ? amax_slot(static_cast<size_t>(li) + 1, 0)
                           : complete    ? lm_head_amax()
                                         : out_amax + s * kAmaxSlotFloats;
        enqueue_layer(static_cast<size_t>(li), io, io.normalized, next_amax);
      }
      // the lm_head only where a request's last row is in this step
      bool completes = false;
      for (size_t i = 0; complete && i < step.requests.size(); ++i)
        completes |= step.positions[i] + step.depth ==
                     static_cast<int>(state.prompts[step.requests[i]].size());
      if (completes)
        run_fp8_gemm(io.normalized, requests * step.depth, spec.hidden, lm_head_amax(), lm_head,
                     embedding_scale.as<float>(), GemmEpilogue::argmax, nullptr, nullptr, nullptr,
                     probe_lm_head_gemm);
      enqueue_accept(requests, step.depth, false, true, io.positions, io.slots, first_sliding,
                     sliding_count, complete ? io.normalized : nullptr, !completes);
      if (completes) {
        std::vector<int32_t> next(static_cast<size_t>(requests));
        hip_check(hipMemcpyAsync(next.data(), d_next, sizeof(int32_t) * next.size(),
                                 hipMemcpyDeviceToHost, stream),
                  "copy layer-sliced suffix predictions");
        hip_check(hipStreamSynchronize(stream), "synchronize layer-sliced suffix step");
        for (size_t i = 0; i < step.requests.size(); ++i) predictions[step.requests[i]] = next[i];
      }
    }
    hip_check(hipStreamSynchronize(stream), "synchronize layer-sliced suffix prefill");
    state.next_layer = last;
    ++state.calls;
    if (!complete) return {false, {}};
    for (size_t r = 0; r < n; ++r)
      slot_positions[static_cast<size_t>(slots[r])] = static_cast<int>(state.prompts[r].size());
    suffix_slices.reset();
    return {true, predictions};
  }

  // batch_model_runner.cu:1507-1541: the source slot's resident KV rows (ring order, the first
  // min(position, capacity) rows of every kv head), its hidden hand-off row and its position.
  uint64_t clone_slot(int source, int destination) {
    if (source < 0 || source >= batch_size || destination < 0 || destination >= batch_size ||
        source == destination)
      throw std::runtime_error("invalid cache slot clone");
    const int position = slot_positions[static_cast<size_t>(source)];
    if (position <= 0 || position >= maximum_context)
      throw std::runtime_error("source cache slot is empty or full");
    uint64_t copied = 0;
    for (auto &L : layers) {
      const int resident = std::min(position, L.capacity);
      const size_t row_bytes = sizeof(bf16_t) * static_cast<size_t>(L.spec.head_dimension);
      const size_t head_pitch = row_bytes * static_cast<size_t>(L.capacity);
      const size_t slot_bytes = head_pitch * static_cast<size_t>(L.spec.kv_heads);
      for (DeviceBuffer *cache : {&L.k_cache, &L.v_cache})
        hip_check(hipMemcpy2DAsync(cache->as<unsigned char>() + destination * slot_bytes, head_pitch,
                                   cache->as<unsigned char>() + source * slot_bytes, head_pitch,
                                   row_bytes * static_cast<size_t>(resident),
                                   static_cast<size_t>(L.spec.kv_heads), hipMemcpyDeviceToDevice,
                                   stream),
                  "clone slot cache rows");
      copied += 2 * sizeof(bf16_t) * static_cast<uint64_t>(resident) *
                static_cast<uint64_t>(L.kv_width());
    }
    const size_t hidden_bytes = sizeof(bf16_t) * static_cast<size_t>(spec.hidden);
    hip_check(hipMemcpyAsync(target_hidden.as<unsigned char>() + destination * hidden_bytes,
                             target_hidden.as<unsigned char>() + source * hidden_bytes,
                             hidden_bytes, hipMemcpyDeviceToDevice, stream),
              "clone slot target hidden state");
    hip_check(hipStreamSynchronize(stream), "synchronize slot cache clone");
    slot_positions[static_cast<size_t>(destination)] = position;
    return copied;
  }

  // batch_model_runner.cu:1006-1040: one lock-step decode token for every slot at the shared
  // position; afterwards every slot is at the next position. A forced depth-1 step of all slots.
  std::vector<int> append(const std::vector<int> &tokens) {
    if (tokens.size() != static_cast<size_t>(batch_size))
      throw std::runtime_error("token batch has the wrong size");
    if (current_position >= maximum_context) throw std::runtime_error("batch context is full");
    std::vector<std::vector<int>> rows;
    std::vector<int> slots;
    for (int s = 0; s < batch_size; ++s) {
      const int token = tokens[static_cast<size_t>(s)];
      if (token < 0 || token >= spec.vocabulary)
        throw std::runtime_error("token batch contains an invalid token id");
      rows.push_back({token});
      slots.push_back(s);
    }
    const std::vector<int> before = slot_positions;
    std::fill(slot_positions.begin(), slot_positions.end(), current_position);
    GreedyVerificationResult result;
    try {
      result = verify(rows, tokens, slots, {}, true);
    } catch (...) {
      slot_positions = before;
      throw;
    }
    ++current_position;
    std::fill(slot_positions.begin(), slot_positions.end(), current_position);
    return result.next_tokens;
  }

  GreedyVerificationResult verify(const std::vector<std::vector<int>> &proposals,
                                  const std::vector<int> &target_first,
                                  const std::vector<int> &slots, const std::vector<int> &caps,
                                  bool force_accept = false, bool lm_head_pass = true) {
    const int requests = static_cast<int>(proposals.size());
    if (!lm_head_pass && !force_accept) throw std::runtime_error("only forced steps may skip the lm_head");
    const int depth = requests == 0 ? 0 : static_cast<int>(proposals.front().size());
    if (requests <= 0 || requests > batch_size || depth <= 0 ||
        (force_accept ? requests * depth > step_rows : depth > kMaximumDepth) ||
        target_first.size() != proposals.size() || slots.size() != proposals.size())
      throw std::runtime_error("invalid greedy verification batch");
    if (!caps.empty() && caps.size() != proposals.size())
      throw std::runtime_error("speculative acceptance caps do not match request count");
    std::vector<bool> seen(static_cast<size_t>(batch_size), false);
    const size_t M = static_cast<size_t>(step_rows);
    int32_t *h_tokens = host_io;
    int32_t *h_positions = h_tokens + M;
    int32_t *h_slots = h_positions + batch_size;
    int32_t *h_first = h_slots + batch_size;
    int32_t *h_caps = h_first + batch_size;
    for (int r = 0; r < requests; ++r) {
      const int slot = slots[static_cast<size_t>(r)];
      if (slot < 0 || slot >= batch_size || seen[static_cast<size_t>(slot)] ||
          static_cast<int>(proposals[static_cast<size_t>(r)].size()) != depth)
        throw std::runtime_error("invalid or repeated speculative slot");
      seen[static_cast<size_t>(slot)] = true;
      const int position = slot_positions[static_cast<size_t>(slot)];
      if (position < (force_accept ? 0 : 1) || position + depth > maximum_context)
        throw std::runtime_error("speculative slot is empty or lacks context capacity");
      for (int t = 0; t < depth; ++t) {
        const int token = proposals[static_cast<size_t>(r)][static_cast<size_t>(t)];
        if (token < 0 || token >= spec.vocabulary)
          throw std::runtime_error("speculative proposal contains an invalid token");
        h_tokens[r * depth + t] = token;
      }
      h_positions[r] = position;
      h_slots[r] = slot;
      h_first[r] = target_first[static_cast<size_t>(r)];
      h_caps[r] = caps.empty() ? depth : caps[static_cast<size_t>(r)];
    }
    // inputs: tokens .. caps (contiguous prefix of the I/O block)
    hip_check(hipMemcpyAsync(d_tokens, h_tokens, sizeof(int32_t) * (M + 4 * batch_size),
                             hipMemcpyHostToDevice, stream),
              "copy speculative inputs");
    hip_check(hipEventRecord(start_event, stream), "record verify start");
    const bool has_caps = !caps.empty();
    if (graphs_enabled && probe_kind == probe_none && !force_accept) {
      auto key = std::make_tuple(requests, depth, has_caps);
      auto found = verify_graphs.find(key);
      if (found == verify_graphs.end()) {
        hipGraph_t graph;
        hip_check(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal), "begin capture");
        enqueue_verify(requests, depth, has_caps);
        hip_check(hipStreamEndCapture(stream, &graph), "end capture");
        hipGraphExec_t exec;
        hip_check(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0), "instantiate graph");
        (void)hipGraphDestroy(graph);
        found = verify_graphs.emplace(key, exec).first;
      }
      hip_check(hipGraphLaunch(found->second, stream), "launch verify graph");
    } else {
      enqueue_verify(requests, depth, has_caps, force_accept, lm_head_pass);
    }
    hip_check(hipEventRecord(stop_event, stream), "record verify stop");
    int32_t *h_accepted = h_caps + batch_size;
    hip_check(hipMemcpyAsync(h_accepted, d_accepted,
                             sizeof(int32_t) * (2 * static_cast<size_t>(batch_size) + M + 1),
                             hipMemcpyDeviceToHost, stream),
              "copy speculative results");
    hip_check(hipStreamSynchronize(stream), "synchronize speculative verification");
    if (h_accepted[2 * static_cast<size_t>(batch_size) + M] != 0)
      throw std::runtime_error(
          "fused activation quantisation timed out waiting for the step's workgroups");
    hip_check(hipEventElapsedTime(&verify_ms, start_event, stop_event), "verify timing");
    collect_probes();
    int32_t *h_next = h_accepted + batch_size;
    int32_t *h_pred = h_next + batch_size;
    GreedyVerificationResult result;
    result.accepted_tokens.assign(h_accepted, h_accepted + requests);
    // a step without the lm_head reads -1 here: the acceptance kernel wrote it on the device
    result.next_tokens.assign(h_next, h_next + requests);
    predictions.assign(h_pred, h_pred + requests * depth);
    for (int r = 0; r < requests; ++r)
      slot_positions[static_cast<size_t>(slots[static_cast<size_t>(r)])] +=
          result.accepted_tokens[static_cast<size_t>(r)];
    return result;
  }

  // -------------------------------------------------------------------------------- draft
  // Striped amaxes of one draft step's projection inputs (fp8 modes): the pre-projection input,
  // then per layer its normalized input, attention output, pre-MLP row and GELU output, then the
  // final hidden row (the lm_head and post-projection input).
  size_t assistant_amax_slots_per_step() const { return 2 + 4 * spec.assistant.layers; }
  float *assistant_amax(int step, size_t which) {
    if (assistant_fp8 == 0) return nullptr;
    return a_amax.as<float>() +
           (static_cast<size_t>(step) * assistant_amax_slots_per_step() + which) * kAmaxSlotFloats;
  }
  // Layer li's amax slot k (0 normalized input, 1 attention output, 2 pre-MLP, 3 GELU output)
  // in `all` mode, else null (the bf16 projections need none).
  float *assistant_layer_amax(int step, size_t li, int k) {
    return assistant_fp8 == 2 ? assistant_amax(step, 1 + 4 * li + static_cast<size_t>(k)) : nullptr;
  }
  float *assistant_final_amax(int step) {
    return assistant_amax(step, assistant_amax_slots_per_step() - 1);
  }

  // One assistant projection into split-K partials: bf16 (Bf16Linear), or in `all` mode the e4m3
  // copy with the input quantised per tensor from its amax (run_linear's Fp8Linear path,
  // assistant_runner.cu:147-160). Returns the split count.
  int run_assistant_partial(const bf16_t *x, int rows, int k, const PackedWeight &w,
                            const PackedWeight &w8, const float *w8_scale, const float *x_amax) {
    if (assistant_fp8 != 2) return run_bf16_gemm_partial(x, rows, k, w);
    int splits = 1;
    run_fp8_gemm(x, rows, k, x_amax, w8, w8_scale, GemmEpilogue::partial_f32, nullptr, nullptr,
                 &splits, probe_none);
    return splits;
  }

  void run_assistant_layer(size_t li, const bf16_t *input, bf16_t *output, int active, int step,
                           bool last_layer) {
    const AssistantSpec &as = spec.assistant;
    AssistantLayer &L = assistant_layers[li];
    const TargetLayer &target = layers[static_cast<size_t>(L.global ? last_global : last_sliding)];
    const int qw = as.query_heads * L.head_dimension;
    const bool all8 = assistant_fp8 == 2;
    const float *scales8 = all8 ? L.scales8.as<float>() : nullptr;
    const int stripes = assistant_fp8 != 0 ? kAmaxStripes : 1;
    int splits = run_assistant_partial(a_normalized.as<bf16_t>(), active, as.hidden, L.q, L.q8,
                                       scales8, assistant_layer_amax(step, li, 0));
    QkvArgs q;
    q.amax_stripes = stripes;
    if (all8) {
      q.x_amax = assistant_layer_amax(step, li, 0);
      q.w_scale = scales8;
    }
    q.partials = partials.as<float>();
    q.splits = splits;
    q.rows = active;
    q.tokens = 1;
    q.query_heads = as.query_heads;
    q.kv_heads = 0;
    q.dimension = L.head_dimension;
    q.eps = spec.eps;
    q.q_norm = L.q_norm.as<bf16_t>();
    q.cosine = L.global ? rope_global_cos.as<bf16_t>() : rope_sliding_cos.as<bf16_t>();
    q.sine = L.global ? rope_global_sin.as<bf16_t>() : rope_sliding_sin.as<bf16_t>();
    q.positions = a_context;
    q.position_offset = step;
    q.q_out = a_queries.as<bf16_t>();
    AttentionArgs at;
    at.mode = AttentionMode::decode;
    at.q = a_queries.as<bf16_t>();
    at.k_cache = target.k_cache.get();
    at.v_cache = target.v_cache.get();
    at.slots = a_slots;
    at.slot_count = batch_size;
    at.positions = a_context;
    at.requests = active;
    at.tokens = 1;
    at.query_heads = as.query_heads;
    at.kv_heads = L.kv_heads;
    at.dimension = L.head_dimension;
    at.capacity = target.capacity;
    at.max_keys = target.capacity;
    at.out = a_attention_out.as<bf16_t>();
    at.out_amax = assistant_layer_amax(step, li, 1);
    at.amax_stripes = stripes;
    at.partials = attention_partials.as<float>();
    at.chunk_keys = L.attention_chunk;
    // the query post-processing inside the decode attention where it can run there
    at.qkv = q;
    at.fuse_qkv = qkv_fusion && attention_can_fuse_qkv(at);
    if (!at.fuse_qkv) launch_qkv_post(q, stream);
    launch_attention(at, stream);
    splits = run_assistant_partial(a_attention_out.as<bf16_t>(), active, qw, L.o, L.o8,
                                   all8 ? scales8 + 1 : nullptr, assistant_layer_amax(step, li, 1));
    RowArgs ro;
    ro.amax_stripes = stripes;
    if (all8) {
      ro.x_amax = assistant_layer_amax(step, li, 1);
      ro.w_scale = scales8 + 1;
    }
    ro.source = RowSource::partials;
    ro.rows = active;
    ro.width = as.hidden;
    ro.eps = spec.eps;
    ro.partials = partials.as<float>();
    ro.splits = splits;
    ro.w1 = L.post_attention_norm.as<bf16_t>();
    ro.residual = input;
    ro.r1_out = a_first_residual.as<bf16_t>();
    ro.w2 = L.pre_mlp_norm.as<bf16_t>();
    ro.y_out = a_pre_mlp.as<bf16_t>();
    ro.y_amax = assistant_layer_amax(step, li, 2);
    launch_row_kernel(ro, stream);
    if (all8) {
      run_fp8_gemm(a_pre_mlp.as<bf16_t>(), active, as.hidden, assistant_layer_amax(step, li, 2),
                   L.gate_up8, scales8 + 2, GemmEpilogue::gelu_gate, a_activated.as<bf16_t>(),
                   assistant_layer_amax(step, li, 3), nullptr, probe_none);
    } else {
      GemmArgs g;
      g.x = a_pre_mlp.as<bf16_t>();
      g.ldx = as.hidden;
      g.m = active;
      g.k = as.hidden;
      g.w = L.gate_up.get();
      g.n = 2 * as.intermediate;
      g.w_layout = L.gate_up.layout;
      g.epilogue = GemmEpilogue::gelu_gate;
      g.y = a_activated.as<bf16_t>();
      g.ldy = as.intermediate;
      launch_bf16_gemm(g, stream);
    }
    splits = run_assistant_partial(a_activated.as<bf16_t>(), active, as.intermediate, L.down,
                                   L.down8, all8 ? scales8 + 3 : nullptr,
                                   assistant_layer_amax(step, li, 3));
    RowArgs rd;
    rd.amax_stripes = stripes;
    if (all8) {
      rd.x_amax = assistant_layer_amax(step, li, 3);
      rd.w_scale = scales8 + 3;
    }
    rd.source = RowSource::partials;
    rd.rows = active;
    rd.width = as.hidden;
    rd.eps = spec.eps;
    rd.partials = partials.as<float>();
    rd.splits = splits;
    rd.w1 = L.post_mlp_norm.as<bf16_t>();
    rd.residual = a_first_residual.as<bf16_t>();
    rd.scalar = L.scalar.as<bf16_t>();
    rd.r1_out = output;
    rd.w2 = last_layer ? a_final_norm.as<bf16_t>() : assistant_layers[li + 1].input_norm.as<bf16_t>();
    rd.y_out = last_layer ? a_final_hidden.as<bf16_t>() : a_normalized.as<bf16_t>();
    rd.y_amax = last_layer ? assistant_final_amax(step) : assistant_layer_amax(step, li + 1, 0);
    launch_row_kernel(rd, stream);
  }

  std::vector<std::vector<int>> draft(const std::vector<int> &last_tokens,
                                      const std::vector<int> &slots,
                                      const std::vector<int> &forced, int depth) {
    if (!has_assistant || last_tokens.size() != slots.size() || last_tokens.empty())
      throw std::runtime_error("assistant is not configured or draft batch is invalid");
    std::vector<int> context_positions;
    for (const int slot : slots) {
      if (slot < 0 || slot >= batch_size || slot_positions[static_cast<size_t>(slot)] <= 0)
        throw std::runtime_error("assistant slot is empty or invalid");
      context_positions.push_back(slot_positions[static_cast<size_t>(slot)] - 1);
    }
    const int active = static_cast<int>(last_tokens.size());
    if (active > batch_size || depth <= 0 || depth > kMaximumDepth)
      throw std::runtime_error("invalid assistant draft batch");
    if (!forced.empty() && forced.size() != last_tokens.size())
      throw std::runtime_error("forced assistant first tokens do not match draft batch");
    const int global_capacity = layers[static_cast<size_t>(last_global)].capacity;
    for (int row = 0; row < active; ++row) {
      const int token = last_tokens[static_cast<size_t>(row)];
      const int ctx = context_positions[static_cast<size_t>(row)];
      if (token < 0 || token >= spec.vocabulary || ctx < 0 || ctx >= global_capacity)
        throw std::runtime_error("invalid assistant row metadata");
    }
    const size_t B = static_cast<size_t>(batch_size);
    // inputs: tokens[B] outputs[B] forced[B] context[B] slots[B] (the prefix of the I/O block), by
    // DMA from its pinned mirror
    int32_t *staging = a_host_io;
    std::fill(staging, staging + B * 5, 0);
    for (int row = 0; row < active; ++row) {
      staging[static_cast<size_t>(row)] = last_tokens[static_cast<size_t>(row)];
      if (!forced.empty()) staging[2 * B + static_cast<size_t>(row)] = forced[static_cast<size_t>(row)];
      staging[3 * B + static_cast<size_t>(row)] = context_positions[static_cast<size_t>(row)];
      staging[4 * B + static_cast<size_t>(row)] = slots[static_cast<size_t>(row)];
    }
    hip_check(hipMemcpyAsync(a_tokens, staging, sizeof(int32_t) * B * 5, hipMemcpyHostToDevice, stream),
              "copy assistant inputs");
    hip_check(hipEventRecord(start_event, stream), "record draft start");
    const AssistantSpec &as = spec.assistant;
    const int H = spec.hidden;
    const bool all8 = assistant_fp8 == 2;
    const int stripes = assistant_fp8 != 0 ? kAmaxStripes : 1;
    if (assistant_fp8 != 0)
      launch_step_init(a_amax.as<float>(),
                       static_cast<int>(depth * assistant_amax_slots_per_step() * kAmaxStripes),
                       stream);
    if (H % 8 != 0) throw std::runtime_error("assistant input rows need a hidden size divisible by 8");
    // Argmax keys per row of the assistant lm_head (its workgroup feature blocks).
    const int argmax_parts = gemm_blocks_n(assistant_fp8 != 0 ? a_embedding8.layout : a_embedding.layout);
    int post_splits = 0;  // split-K partials of the previous step's post-projection (0: none)
    bool previous_lm_head = false;  // the previous step ran the lm_head (else its token was forced)
    for (int d = 0; d < depth; ++d) {
      {
        // step 0: the given tokens and the target's hand-off rows (gather_rows_bf16 by slot);
        // later steps: the previous step's token (argmax keys, or the forced token) and the sum
        // of its post-projection partials
        AssistantInputArgs in;
        in.embedding = embedding_bf16.as<bf16_t>();
        in.vocabulary = spec.vocabulary;
        in.embed_scale = std::sqrt(static_cast<float>(H));
        if (d == 0) {
          in.tokens = a_tokens;
          in.gather_src = target_hidden.as<bf16_t>();
          in.gather_rows = a_slots;
        } else {
          if (previous_lm_head) {
            in.argmax_partials = argmax_partials.as<uint64_t>();
            in.argmax_parts = argmax_parts;
          } else {
            in.tokens = a_forced;  // assistant_runner.cu:306-312
          }
          in.table = a_proposals;
          in.table_stride = depth;
          in.table_column = d - 1;
          in.partials = partials.as<float>();
          in.splits = post_splits;
          if (all8) {
            in.x_amax = assistant_final_amax(d - 1);
            in.w_scale = a_scales8.as<float>() + 2;
          }
        }
        in.out = a_input.as<bf16_t>();
        in.rows = active;
        in.hidden = H;
        in.amax = all8 ? assistant_amax(d, 0) : nullptr;
        in.stripes = stripes;
        const dim3 grid(static_cast<unsigned>((2 * H / 8 + 255) / 256), static_cast<unsigned>(active));
        assistant_input_kernel<<<grid, 256, 0, stream>>>(in);
        hip_check(hipGetLastError(), "launch assistant input");
      }
      const int splits = run_assistant_partial(a_input.as<bf16_t>(), active, 2 * H, a_pre_projection,
                                         a_pre_projection8,
                                         all8 ? a_scales8.as<float>() + 1 : nullptr,
                                         all8 ? assistant_amax(d, 0) : nullptr);
      RowArgs rp;
      rp.amax_stripes = stripes;
      if (all8) {
        rp.x_amax = assistant_amax(d, 0);
        rp.w_scale = a_scales8.as<float>() + 1;
      }
      rp.source = RowSource::partials;
      rp.rows = active;
      rp.width = as.hidden;
      rp.eps = spec.eps;
      rp.partials = partials.as<float>();
      rp.splits = splits;
      rp.v_out = a_hidden_a.as<bf16_t>();
      rp.w2 = assistant_layers[0].input_norm.as<bf16_t>();
      rp.y_out = a_normalized.as<bf16_t>();
      rp.y_amax = assistant_layer_amax(d, 0, 0);
      launch_row_kernel(rp, stream);
      bf16_t *input = a_hidden_a.as<bf16_t>();
      bf16_t *output = a_hidden_b.as<bf16_t>();
      for (size_t li = 0; li < assistant_layers.size(); ++li) {
        run_assistant_layer(li, input, output, active, d, li + 1 == assistant_layers.size());
        std::swap(input, output);
      }
      const bool last = d + 1 == depth;
      previous_lm_head = !(d == 0 && !forced.empty());
      if (!previous_lm_head) {
        // assistant_runner.cu:306-312: the forced token replaces the dead first lm_head pass (the
        // next step's input kernel writes it to the table; a one-step draft does it here)
        if (last) {
          copy_tokens_kernel<<<(active + 255) / 256, 256, 0, stream>>>(a_forced, a_outputs,
                                                                       a_proposals, active, depth, d);
          hip_check(hipGetLastError(), "launch forced tokens");
        }
      } else {
        GemmArgs g;
        g.x = a_final_hidden.as<bf16_t>();
        g.ldx = as.hidden;
        g.m = active;
        g.k = as.hidden;
        g.w = a_embedding.get();
        g.n = spec.vocabulary;
        g.w_layout = a_embedding.layout;
        if (assistant_fp8 != 0) {
          // Fp8Linear over the e4m3 lm_head, the final hidden row quantised per tensor
          g.w = a_embedding8.get();
          g.w_layout = a_embedding8.layout;
          g.x_amax = assistant_final_amax(d);
          g.w_scale = a_scales8.as<float>();
          g.amax_stripes = kAmaxStripes;
          g.xprep = xprep.as<unsigned char>();
          g.xprep_capacity = xprep.bytes();
        }
        g.epilogue = GemmEpilogue::argmax;
        g.argmax_partials = argmax_partials.as<uint64_t>();
        g.argmax_partial_capacity = argmax_partials.bytes() / sizeof(uint64_t);
        // the next step's input kernel reduces the keys; the last step's go to the table here
        g.argmax_deferred = !last;
        g.argmax_out = a_outputs;
        g.argmax_table = a_proposals;
        g.argmax_table_stride = depth;
        g.argmax_table_column = d;
        if (assistant_fp8 != 0)
          launch_fp8_gemm(g, stream);
        else
          launch_bf16_gemm(g, stream);
      }
      post_splits = run_assistant_partial(a_final_hidden.as<bf16_t>(), active, as.hidden,
                                          a_post_projection, a_post_projection8,
                                          all8 ? a_scales8.as<float>() + 2 : nullptr,
                                          assistant_final_amax(d));
      if (last) {
        // the last step's hand-off row (assistant.previous_hidden); earlier ones are summed by the
        // next step's input kernel
        RowArgs rq;
        rq.amax_stripes = stripes;
        if (all8) {
          rq.x_amax = assistant_final_amax(d);
          rq.w_scale = a_scales8.as<float>() + 2;
        }
        rq.source = RowSource::partials;
        rq.rows = active;
        rq.width = H;
        rq.partials = partials.as<float>();
        rq.splits = post_splits;
        rq.v_out = a_previous_hidden.as<bf16_t>();
        launch_row_kernel(rq, stream);
      }
    }
    hip_check(hipEventRecord(stop_event, stream), "record draft stop");
    int32_t *table = a_host_io + 5 * B;  // the pinned mirror of a_proposals
    hip_check(hipMemcpyAsync(table, a_proposals, sizeof(int32_t) * static_cast<size_t>(active) * depth,
                             hipMemcpyDeviceToHost, stream),
              "copy assistant proposals");
    hip_check(hipStreamSynchronize(stream), "synchronize assistant draft");
    hip_check(hipEventElapsedTime(&draft_ms, start_event, stop_event), "draft timing");
    std::vector<std::vector<int>> proposals(static_cast<size_t>(active),
                                            std::vector<int>(static_cast<size_t>(depth)));
    for (int row = 0; row < active; ++row)
      for (int d = 0; d < depth; ++d)
        proposals[static_cast<size_t>(row)][static_cast<size_t>(d)] =
            table[static_cast<size_t>(row) * depth + d];
    return proposals;
  }

  // Named tensor; `layout` (optional) receives the packed layout of a weight (else n = 0).
  void *tensor(const std::string &name, size_t *bytes, WeightLayout *layout = nullptr) {
    if (layout != nullptr) *layout = WeightLayout{};
    auto give = [&](const DeviceBuffer &b) {
      if (b.get() == nullptr) throw std::runtime_error("runner tensor is not allocated: " + name);
      if (bytes != nullptr) *bytes = b.bytes();
      return b.get();
    };
    auto give_packed = [&](const PackedWeight &w) {
      if (layout != nullptr) *layout = w.layout;
      return give(w.data);
    };
    if (name == "token_embedding") return give(embedding_bf16);
    if (name == "token_embedding.fp8") return give_packed(lm_head);
    if (name == "token_embedding.scale") return give(embedding_scale);
    // channel / block_128 scales of the e4m3 lm_head and projections (Fp8WeightArena layout)
    if (name == "token_embedding.scale_table") return give(lm_head.scale_table);
    if (name == "final_norm") return give(final_norm);
    if (name == "target_hidden") return give(target_hidden);
    if (name == "final_hidden") return give(final_hidden);
    if (name == "rope.sliding.cos") return give(rope_sliding_cos);
    if (name == "rope.sliding.sin") return give(rope_sliding_sin);
    if (name == "rope.global.cos") return give(rope_global_cos);
    if (name == "rope.global.sin") return give(rope_global_sin);
    if (name == "assistant.token_embedding") return give_packed(a_embedding);
    if (name == "assistant.pre_projection") return give_packed(a_pre_projection);
    if (name == "assistant.post_projection") return give_packed(a_post_projection);
    if (name == "assistant.final_norm") return give(a_final_norm);
    // AssistantFp8Mode e4m3 copies (absent when the mode does not use them) and their scales
    // [lm_head, pre_projection, post_projection]
    if (name == "assistant.token_embedding.fp8") return give_packed(a_embedding8);
    if (name == "assistant.pre_projection.fp8") return give_packed(a_pre_projection8);
    if (name == "assistant.post_projection.fp8") return give_packed(a_post_projection8);
    if (name == "assistant.fp8_scales") return give(a_scales8);
    // the last draft step's post-projection output ([batch][hidden] bf16, rows < active valid)
    if (name == "assistant.previous_hidden") return give(a_previous_hidden);
    // the last draft step's intermediates, as the last assistant layer left them (rows < active)
    if (name == "assistant.input") return give(a_input);  // [embedding | previous hidden]
    if (name == "assistant.hidden_a") return give(a_hidden_a);
    if (name == "assistant.hidden_b") return give(a_hidden_b);
    if (name == "assistant.normalized") return give(a_normalized);
    if (name == "assistant.queries") return give(a_queries);
    if (name == "assistant.attention_out") return give(a_attention_out);
    if (name == "assistant.first_residual") return give(a_first_residual);
    if (name == "assistant.pre_mlp") return give(a_pre_mlp);
    if (name == "assistant.activated") return give(a_activated);
    if (name == "assistant.final_hidden") return give(a_final_hidden);
    const auto dot = name.find('.');
    const auto dot2 = name.find('.', dot + 1);
    if (dot != std::string::npos && dot2 != std::string::npos) {
      const std::string head = name.substr(0, dot);
      const std::string rest = name.substr(dot2 + 1);
      if (head == "assistant") {
        const auto dot3 = name.find('.', dot2 + 1);
        if (name.compare(dot + 1, dot2 - dot - 1, "layer") == 0 && dot3 != std::string::npos) {
          const size_t li = static_cast<size_t>(std::stoul(name.substr(dot2 + 1, dot3 - dot2 - 1)));
          const std::string field = name.substr(dot3 + 1);
          if (li < assistant_layers.size()) {
            AssistantLayer &L = assistant_layers[li];
            if (field == "input_norm") return give(L.input_norm);
            if (field == "q_norm") return give(L.q_norm);
            if (field == "q") return give_packed(L.q);
            if (field == "o") return give_packed(L.o);
            if (field == "post_attention_norm") return give(L.post_attention_norm);
            if (field == "pre_mlp_norm") return give(L.pre_mlp_norm);
            if (field == "gate_up") return give_packed(L.gate_up);
            if (field == "down") return give_packed(L.down);
            if (field == "post_mlp_norm") return give(L.post_mlp_norm);
            if (field == "scalar") return give(L.scalar);
            if (field == "q.fp8") return give_packed(L.q8);
            if (field == "o.fp8") return give_packed(L.o8);
            if (field == "gate_up.fp8") return give_packed(L.gate_up8);
            if (field == "down.fp8") return give_packed(L.down8);
            if (field == "fp8_scales") return give(L.scales8);  // [q, o, gate_up, down]
          }
        }
      } else {
        const size_t li = static_cast<size_t>(std::stoul(name.substr(dot + 1, dot2 - dot - 1)));
        if (li < layers.size()) {
          TargetLayer &L = layers[li];
          if (head == "layer") {
            if (rest == "input_norm") return give(L.input_norm);
            if (rest == "q_norm") return give(L.q_norm);
            if (rest == "k_norm") return give(L.k_norm);
            if (rest == "post_attention_norm") return give(L.post_attention_norm);
            if (rest == "pre_mlp_norm") return give(L.pre_mlp_norm);
            if (rest == "post_mlp_norm") return give(L.post_mlp_norm);
            if (rest == "scalar") return give(L.scalar);
            if (rest == "qkv") return give_packed(L.qkv);
            if (rest == "o") return give_packed(L.o);
            if (rest == "gate_up") return give_packed(L.gate_up);
            if (rest == "down") return give_packed(L.down);
            if (rest == "scales") return give(L.scales);
            if (rest == "qkv.scale_table") return give(L.qkv.scale_table);
            if (rest == "o.scale_table") return give(L.o.scale_table);
            if (rest == "gate_up.scale_table") return give(L.gate_up.scale_table);
            if (rest == "down.scale_table") return give(L.down.scale_table);
          } else if (head == "cache") {
            if (rest == "k") return give(L.k_cache);
            if (rest == "v") return give(L.v_cache);
          } else if (head == "new") {
            if (rest == "k") return give(L.k_new);
            if (rest == "v") return give(L.v_new);
          }
        }
      }
    }
    throw std::runtime_error("unknown runner tensor: " + name);
  }
};

namespace {
ModelSpec spec_of(const Checkpoint &checkpoint) {
  ModelSpec spec;
  checkpoint.describe(spec);
  return spec;
}
}  // namespace

BatchModelRunner::BatchModelRunner(const Checkpoint &checkpoint, int batch, int maximum_context)
    : implementation_(std::make_unique<Implementation>(spec_of(checkpoint), batch, maximum_context,
                                                       &checkpoint)) {}

BatchModelRunner::BatchModelRunner(const ModelSpec &spec, DeviceSegmentFn segment, void *context,
                                   int batch, int maximum_context)
    : implementation_(std::make_unique<Implementation>(
          spec, batch, maximum_context, nullptr,
          segment != nullptr ? segment : throw std::runtime_error("missing device weight lookup"),
          context)) {}

BatchModelRunner::BatchModelRunner(const ModelSpec &spec, int batch, int maximum_context)
    : implementation_(std::make_unique<Implementation>(spec, batch, maximum_context)) {}
BatchModelRunner::~BatchModelRunner() = default;

GreedyVerificationResult BatchModelRunner::verify_greedy_proposals(
    const std::vector<std::vector<int>> &proposals, const std::vector<int> &target_first_tokens,
    const std::vector<int> &slots, const std::vector<int> &maximum_accepted_tokens) {
  return implementation_->verify(proposals, target_first_tokens, slots, maximum_accepted_tokens);
}

int BatchModelRunner::prefill_slot(int slot, const std::vector<int> &token_ids, int chunk_tokens) {
  reset_slot(slot);
  return prefill_slot_from_prefix(slot, token_ids, 0, chunk_tokens);
}

int BatchModelRunner::prefill_slot_from_prefix(int slot, const std::vector<int> &token_ids,
                                               int cached_prefix_tokens, int chunk_tokens) {
  auto &s = *implementation_;
  if (slot < 0 || slot >= s.batch_size || token_ids.empty() ||
      token_ids.size() > static_cast<size_t>(s.maximum_context) || chunk_tokens <= 0 ||
      chunk_tokens > s.maximum_context || cached_prefix_tokens < 0 ||
      cached_prefix_tokens >= static_cast<int>(token_ids.size()) ||
      s.slot_positions[static_cast<size_t>(slot)] != cached_prefix_tokens)
    throw std::runtime_error("invalid slot prefill shape");
  std::optional<int> prediction;
  while (!prediction) prediction = prefill_slot_chunk(slot, token_ids, chunk_tokens);
  return *prediction;
}

std::optional<int> BatchModelRunner::prefill_slot_chunk(int slot, const std::vector<int> &token_ids,
                                                        int chunk_tokens) {
  auto &s = *implementation_;
  if (slot < 0 || slot >= s.batch_size || chunk_tokens > s.maximum_context)
    throw std::runtime_error(Implementation::kSlotChunkMessages.shape);
  return s.prefill_chunks({slot}, {&token_ids}, chunk_tokens, Implementation::kSlotChunkMessages)
      .front();
}

std::vector<std::optional<int>> BatchModelRunner::prefill_slots_chunks(
    const std::vector<int> &slots, const std::vector<const std::vector<int> *> &token_ids,
    int chunk_tokens) {
  return implementation_->prefill_chunks(slots, token_ids, chunk_tokens,
                                         Implementation::kChunksMessages);
}

std::vector<int> BatchModelRunner::prefill_slots_suffix(
    const std::vector<int> &slots, const std::vector<const std::vector<int> *> &token_ids) {
  const auto result = implementation_->prefill_chunks(slots, token_ids,
                                                      std::numeric_limits<int>::max(),
                                                      Implementation::kSuffixMessages);
  std::vector<int> predictions;
  for (const auto &p : result) predictions.push_back(*p);
  return predictions;
}

LayerSlicedSuffixPrefillResult BatchModelRunner::prefill_slots_suffix_layer_slice(
    const std::vector<int> &slots, const std::vector<const std::vector<int> *> &token_ids,
    int maximum_layers) {
  auto [complete, predictions] =
      implementation_->prefill_suffix_layer_slice(slots, token_ids, maximum_layers);
  return LayerSlicedSuffixPrefillResult{complete, std::move(predictions)};
}

void BatchModelRunner::abort_suffix_layer_slices() { implementation_->suffix_slices.reset(); }

bool BatchModelRunner::has_suffix_layer_slices() const {
  return implementation_->suffix_slices != nullptr;
}

uint64_t BatchModelRunner::clone_slot(int source_slot, int destination_slot) {
  return implementation_->clone_slot(source_slot, destination_slot);
}

std::vector<int> BatchModelRunner::append(const std::vector<int> &token_ids) {
  return implementation_->append(token_ids);
}

std::vector<int> BatchModelRunner::append_ragged(const std::vector<int> &token_ids,
                                                const std::vector<int> &slots) {
  return implementation_->append_ragged(token_ids, slots);
}

std::vector<std::vector<int>> BatchModelRunner::draft_four(const std::vector<int> &last_tokens,
                                                           const std::vector<int> &slots,
                                                           const std::vector<int> &forced,
                                                           int depth) {
  return implementation_->draft(last_tokens, slots, forced, depth);
}

bool BatchModelRunner::has_assistant() const { return implementation_->has_assistant; }

void BatchModelRunner::reset_slot(int slot) {
  if (slot < 0 || slot >= implementation_->batch_size) throw std::runtime_error("invalid cache slot");
  implementation_->slot_positions[static_cast<size_t>(slot)] = 0;
}

void BatchModelRunner::seed_empty_cache_for_benchmark(int position) {
  auto &s = *implementation_;
  if (position < 0 || position >= s.maximum_context)
    throw std::runtime_error("invalid benchmark cache position");
  for (auto &L : s.layers) {
    hip_check(hipMemsetAsync(L.k_cache.get(), 0, L.k_cache.bytes(), s.stream), "zero K cache");
    hip_check(hipMemsetAsync(L.v_cache.get(), 0, L.v_cache.bytes(), s.stream), "zero V cache");
  }
  hip_check(hipStreamSynchronize(s.stream), "zero benchmark KV cache");
  s.current_position = position;
  std::fill(s.slot_positions.begin(), s.slot_positions.end(), position);
}

void BatchModelRunner::seed_random_cache_for_benchmark(int position, uint64_t seed, float stddev) {
  auto &s = *implementation_;
  if (position < 0 || position >= s.maximum_context)
    throw std::runtime_error("invalid benchmark cache position");
  uint64_t tensor = 900000 + seed * 1000;
  for (auto &L : s.layers) {
    fill_normal_bf16(L.k_cache.as<bf16_t>(), L.k_cache.bytes() / 2, s.seed_for(tensor++), 0.0f,
                     stddev, s.stream);
    fill_normal_bf16(L.v_cache.as<bf16_t>(), L.v_cache.bytes() / 2, s.seed_for(tensor++), 0.0f,
                     stddev, s.stream);
  }
  fill_normal_bf16(s.target_hidden.as<bf16_t>(), s.target_hidden.bytes() / 2, s.seed_for(tensor++),
                   0.0f, 1.0f, s.stream);
  hip_check(hipStreamSynchronize(s.stream), "seed benchmark KV cache");
  s.current_position = position;
  std::fill(s.slot_positions.begin(), s.slot_positions.end(), position);
}

void BatchModelRunner::set_slot_position(int slot, int position) {
  auto &s = *implementation_;
  if (slot < 0 || slot >= s.batch_size || position < 0 || position > s.maximum_context)
    throw std::runtime_error("invalid cache slot");
  s.slot_positions[static_cast<size_t>(slot)] = position;
}

int BatchModelRunner::batch() const { return implementation_->batch_size; }
int BatchModelRunner::position() const { return implementation_->current_position; }
int BatchModelRunner::slot_position(int slot) const {
  if (slot < 0 || slot >= implementation_->batch_size) throw std::runtime_error("invalid cache slot");
  return implementation_->slot_positions[static_cast<size_t>(slot)];
}
const std::vector<int> &BatchModelRunner::last_predictions() const {
  return implementation_->predictions;
}
void *BatchModelRunner::tensor(const std::string &name, size_t *bytes,
                               WeightLayout *layout) const {
  return implementation_->tensor(name, bytes, layout);
}
hipStream_t BatchModelRunner::stream() const { return implementation_->stream; }
void BatchModelRunner::set_graphs_enabled(bool enabled) { implementation_->graphs_enabled = enabled; }
void BatchModelRunner::set_qkv_fusion(bool enabled) { implementation_->set_qkv_fusion(enabled); }
void BatchModelRunner::set_fused_quantization(int mode) {
  implementation_->set_fused_quantization(mode);
}
float BatchModelRunner::last_verify_ms() const { return implementation_->verify_ms; }
float BatchModelRunner::last_draft_ms() const { return implementation_->draft_ms; }
void BatchModelRunner::set_probe(int kind) {
  if (kind < probe_none || kind > probe_global_attention) throw std::runtime_error("invalid probe kind");
  implementation_->probe_kind = kind;
  implementation_->probe_total_ms = 0.0;
  implementation_->probe_launches = 0;
}
float BatchModelRunner::stream_gemm_probe(int kind, int passes, int *launches) {
  return implementation_->stream_gemm_probe(kind, passes, launches);
}
void BatchModelRunner::read_probe(float *total_ms, int *launches) {
  *total_ms = static_cast<float>(implementation_->probe_total_ms);
  *launches = implementation_->probe_launches;
  implementation_->probe_total_ms = 0.0;
  implementation_->probe_launches = 0;
}

}  // namespace carat_hip
