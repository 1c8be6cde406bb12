// Row-wise fused kernels of the verify step (see rowops.h). Rounding points follow the reference:
// every stage output is rounded to bf16 before it feeds the next stage (cuda/ops.cu:27-217,
// cuda/qkv.cu:387-530), and amax is taken over the rounded values.
#include "rowops.h"

#include <algorithm>
#include <type_traits>

namespace carat_hip {
namespace {

constexpr int kRowThreads = 1024;
constexpr int kQkvUnrolledSplits = 4;  // split-K partials the QKV post-processing loads at once
constexpr int kMaxAcceptRows = 1024;    // rows per request of a forced (prefill) commit
constexpr int kRowMaxQuadsPerThread = 4;  // widths up to 16384

__device__ __forceinline__ f32x4_t bf16x4_to_f32(uint2 v) {
  return f32x4_t{__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u),
                 __uint_as_float(v.y << 16), __uint_as_float(v.y & 0xffff0000u)};
}

__device__ __forceinline__ uint2 f32x4_to_bf16(f32x4_t v) {
  return uint2{static_cast<uint32_t>(f32_to_bf16(v[0])) | (static_cast<uint32_t>(f32_to_bf16(v[1])) << 16),
               static_cast<uint32_t>(f32_to_bf16(v[2])) | (static_cast<uint32_t>(f32_to_bf16(v[3])) << 16)};
}

// One workgroup per row (kThreads threads); thread t owns the 4-column quads t, t + kThreads,
// ... (Q of them, width % 4 == 0). Every global load of the row (source, residual, both norm
// weights) is issued before the first reduction, so the kernel pays one memory round trip plus
// its block reductions.
template <int Q, int kThreads = kRowThreads>
__global__ __launch_bounds__(kThreads) void row_kernel(const RowArgs a) {
  __shared__ float scratch[kThreads / kWave];
  const int row = blockIdx.x;
  const int quads = a.width / 4;
  const size_t row_offset = static_cast<size_t>(row) * a.width;

  // The scale operands are loaded alongside the row and reduced after it arrives, so their latency
  // is not paid first.
  float amax_part = 0.0f, w_scale = 1.0f;
  const bool scaled = a.source == RowSource::partials && a.x_amax != nullptr;
  if (scaled) amax_part = amax_lane(a.x_amax, a.amax_stripes);
  if (a.source == RowSource::partials && a.w_scale != nullptr) w_scale = *a.w_scale;
  const float embed_scale = round_bf16(a.embed_scale);
  int token = 0;
  if (a.source == RowSource::embedding) token = a.tokens[row];
  const bool token_ok = token >= 0 && token < a.vocabulary;

  // ---- loads
  f32x4_t v[Q], w1[Q], res[Q], w2[Q];
#pragma unroll
  for (int i = 0; i < Q; ++i) {
    const int q = threadIdx.x + i * kThreads;
    v[i] = w1[i] = res[i] = w2[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    if (q >= quads) continue;
    if (a.source == RowSource::embedding) {
      if (token_ok) {
        const f32x4_t e = bf16x4_to_f32(
            reinterpret_cast<const uint2 *>(a.embedding + static_cast<size_t>(token) * a.width)[q]);
#pragma unroll
        for (int c = 0; c < 4; ++c) v[i][c] = round_bf16(e[c] * embed_scale);
      }
    } else if (a.source == RowSource::partials) {
      f32x4_t sum = {0.f, 0.f, 0.f, 0.f};
      for (int k0 = 0; k0 < a.splits; k0 += 4) {
#pragma unroll
        for (int k = k0; k < k0 + 4; ++k)
          if (k < a.splits)
            sum += reinterpret_cast<const f32x4_t *>(
                a.partials + (static_cast<size_t>(k) * a.rows + row) * a.width)[q];
      }
      v[i] = sum;  // scaled and rounded below
    } else {
      v[i] = bf16x4_to_f32(reinterpret_cast<const uint2 *>(a.x + row_offset)[q]);
    }
    if (a.w1 != nullptr) {
      w1[i] = bf16x4_to_f32(reinterpret_cast<const uint2 *>(a.w1)[q]);
      if (a.residual != nullptr)
        res[i] = bf16x4_to_f32(reinterpret_cast<const uint2 *>(a.residual + row_offset)[q]);
    }
    if (a.w2 != nullptr) w2[i] = bf16x4_to_f32(reinterpret_cast<const uint2 *>(a.w2)[q]);
  }

  float scale = w_scale;
  if (scaled) scale *= fp8_scale_from_amax(wave_max(amax_part));

  // ---- source value (rounded to bf16), optional copy out
  float square_sum = 0.0f;
#pragma unroll
  for (int i = 0; i < Q; ++i) {
    const int q = threadIdx.x + i * kThreads;
    if (a.source == RowSource::partials)
#pragma unroll
      for (int c = 0; c < 4; ++c) v[i][c] = round_bf16(v[i][c] * scale);
    if (q < quads && a.v_out != nullptr)
      reinterpret_cast<uint2 *>(a.v_out + row_offset)[q] = f32x4_to_bf16(v[i]);
#pragma unroll
    for (int c = 0; c < 4; ++c) square_sum += v[i][c] * v[i][c];
  }

  // ---- stage 1: r1 = bf16(norm(v) * w1 + residual) [ * scalar ]
  if (a.w1 != nullptr) {
    const float inv = inverse_rms(block_sum(square_sum, scratch), a.width, a.eps);
    const float layer_scalar = a.scalar != nullptr ? bf16_to_f32(*a.scalar) : 1.0f;
    square_sum = 0.0f;
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const int q = threadIdx.x + i * kThreads;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        float r1 = round_bf16(v[i][c] * inv * w1[i][c] + res[i][c]);
        if (a.scalar != nullptr) r1 = round_bf16(r1 * layer_scalar);
        v[i][c] = q < quads ? r1 : 0.0f;
        square_sum += v[i][c] * v[i][c];
      }
      if (q < quads && a.r1_out != nullptr)
        reinterpret_cast<uint2 *>(a.r1_out + row_offset)[q] = f32x4_to_bf16(v[i]);
    }
  }

  // ---- stage 2: y = bf16(norm(.) * w2), amax
  if (a.w2 != nullptr) {
    const float inv = inverse_rms(block_sum(square_sum, scratch), a.width, a.eps);
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const int q = threadIdx.x + i * kThreads;
      if (q >= quads) continue;
      f32x4_t y;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        y[c] = round_bf16(v[i][c] * inv * w2[i][c]);
        amax = fmaxf(amax, fabsf(y[c]));
      }
      reinterpret_cast<uint2 *>(a.y_out + row_offset)[q] = f32x4_to_bf16(y);
    }
    if (a.y_amax != nullptr) {
      amax = block_max(amax, scratch);
      if (threadIdx.x == 0) amax_publish(a.y_amax, a.amax_stripes, amax);
    }
  }
}

// The verify step's layer-end rows, with every option fixed at compile time: split-K partials
// (kSplits of them, fp8 output scale), stage 1 with residual (layer scalar optional, a uniform
// load), stage 2 with amax. One workgroup per row, kThreads threads of Q quads each (width 5376:
// 448 threads x 3 quads, no idle lanes). Every global load of the row is issued in one straight
// run before the first reduction (no conditional load: the layer scalar's address is selected,
// not branched on); the runtime options of row_kernel put waits between them.
template <int Q, int kThreads, int kSplits, bool kScaled = true>
__global__ __launch_bounds__(kThreads) void layer_end_kernel(const RowArgs a) {
  constexpr int kWaves = kThreads / kWave;
  __shared__ float scratch[kWaves];
  const int row = blockIdx.x;
  const int quads = a.width / 4;
  const size_t row_offset = static_cast<size_t>(row) * a.width;
  const float w_scale = kScaled ? *a.w_scale : 1.0f;
  const float layer_scalar = bf16_to_f32(*(a.scalar != nullptr ? a.scalar : a.w2));
  f32x4_t v[Q], w1[Q], res[Q], w2[Q];
  f32x4_t part[Q][kSplits];
#pragma unroll
  for (int i = 0; i < Q; ++i) {
    const int q = min(threadIdx.x + i * kThreads, quads - 1);  // tail lanes re-read the last quad
#pragma unroll
    for (int k = 0; k < kSplits; ++k)
      part[i][k] = reinterpret_cast<const f32x4_t *>(a.partials + (static_cast<size_t>(k) * a.rows + row) * a.width)[q];
    w1[i] = bf16x4_to_f32(reinterpret_cast<const uint2 *>(a.w1)[q]);
    res[i] = bf16x4_to_f32(reinterpret_cast<const uint2 *>(a.residual + row_offset)[q]);
    w2[i] = bf16x4_to_f32(reinterpret_cast<const uint2 *>(a.w2)[q]);
  }
  float scale = 1.0f;
  if constexpr (kScaled) scale = w_scale * fp8_scale_from_amax(wave_max(amax_lane(a.x_amax, a.amax_stripes)));

  float square_sum = 0.0f;
#pragma unroll
  for (int i = 0; i < Q; ++i) {
    const bool live = threadIdx.x + i * kThreads < quads;
    f32x4_t sum = part[i][0];
#pragma unroll
    for (int k = 1; k < kSplits; ++k) sum += part[i][k];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      v[i][c] = live ? round_bf16(sum[c] * scale) : 0.0f;
      square_sum += v[i][c] * v[i][c];
    }
  }

  // stage 1: r1 = bf16(norm(v) * w1 + residual) [* scalar]
  // With the fused quantisation every store waits until the workgroups have agreed on the amax, so
  // that the agreement's release finds no store of this kernel to write back.
  const bool fused = a.xprep != nullptr && a.y_amax != nullptr;
  const bool has_scalar = a.scalar != nullptr;
  float inv = inverse_rms(block_sum(square_sum, scratch), a.width, a.eps);
  square_sum = 0.0f;
  f32x4_t r1v[Q];
#pragma unroll
  for (int i = 0; i < Q; ++i) {
    const int q = threadIdx.x + i * kThreads;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float r1 = round_bf16(v[i][c] * inv * w1[i][c] + res[i][c]);
      if (has_scalar) r1 = round_bf16(r1 * layer_scalar);
      v[i][c] = q < quads ? r1 : 0.0f;
      square_sum += v[i][c] * v[i][c];
    }
    r1v[i] = v[i];
    if (!fused && q < quads) reinterpret_cast<uint2 *>(a.r1_out + row_offset)[q] = f32x4_to_bf16(v[i]);
  }

  // stage 2: y = bf16(norm(r1) * w2), amax
  inv = inverse_rms(block_sum(square_sum, scratch), a.width, a.eps);
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < Q; ++i) {
    const int q = threadIdx.x + i * kThreads;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      v[i][c] = round_bf16(v[i][c] * inv * w2[i][c]);  // y, kept for the fused quantisation
      amax = fmaxf(amax, fabsf(v[i][c]));
    }
    if (!fused && q < quads) reinterpret_cast<uint2 *>(a.y_out + row_offset)[q] = f32x4_to_bf16(v[i]);
  }
  if (a.y_amax == nullptr) return;  // bf16 consumers (the assistant's GEMMs) need no amax
  amax = block_max(amax, scratch);
  if (!fused) {
    if (threadIdx.x == 0) amax_publish(a.y_amax, a.amax_stripes, amax);
    return;
  }

  // ---- fused e4m3 quantisation of y: the workgroups agree on the tensor's amax, then each
  // stores r1, y and its row of the quantised operand.
  __shared__ float tensor_amax;
  if (threadIdx.x < kWave) {
    const float total = fused_amax_release(a.y_amax, a.amax_stripes, a.sync, a.fault, gridDim.x, amax,
                                           a.quantize_spins);
    if (threadIdx.x == 0) tensor_amax = total;
  }
  __syncthreads();
  const float q_inv = 1.0f / fp8_scale_from_amax(tensor_amax);
  // operand layout (prepare_x_kernel's): row-major [row][width] e4m3, so the row's bytes are
  // whole cache lines of this workgroup's own
  unsigned char *operand = a.xprep + static_cast<size_t>(row) * a.width;
#pragma unroll
  for (int i = 0; i < Q; ++i) {
    const int q = threadIdx.x + i * kThreads;
    if (q >= quads) continue;
    reinterpret_cast<uint2 *>(a.r1_out + row_offset)[q] = f32x4_to_bf16(r1v[i]);
    reinterpret_cast<uint2 *>(a.y_out + row_offset)[q] = f32x4_to_bf16(v[i]);
    reinterpret_cast<uint32_t *>(operand)[q] =
        f32x4_to_e4m3x4(v[i][0] * q_inv, v[i][1] * q_inv, v[i][2] * q_inv, v[i][3] * q_inv);
  }
}

// One wave per (row, head). Lane l owns elements [l*E, l*E+E) with E = D/64; the rotate-half
// partner of element i (i +- D/2) lives in lane l ^ 32. kSplits > 0: the source is that many
// split-K partials (a compile-time count, so that every load of the wave -- partials, scale
// operands, norm weight, position -- goes out in one straight run, and only the RoPE table rows,
// which need the position, wait for it); kSplits = 0: the packed bf16 rows or any other split
// count.
template <int D, int kSplits>
__global__ __launch_bounds__(64) void qkv_post_kernel(const QkvArgs a) {
  constexpr int E = D / 64;
  const int row = blockIdx.x;
  const int head = blockIdx.y;
  const int lane = threadIdx.x;
  const int hq = a.query_heads;
  const int hkv = a.kv_heads;
  const int query_width = hq * D;
  const int kv_width = hkv * D;
  const int packed_width = query_width + (hkv == 0 ? 0 : kv_width * (a.key_equals_value ? 1 : 2));

  int kind;  // 0 = query, 1 = key (+ value when K == V), 2 = value
  int h;
  int column0;
  if (head < hq) {
    kind = 0;
    h = head;
    column0 = head * D;
  } else if (head < hq + hkv) {
    kind = 1;
    h = head - hq;
    column0 = query_width + h * D;
  } else {
    kind = 2;
    h = head - hq - hkv;
    column0 = query_width + kv_width + h * D;
  }

  const int request = row / a.tokens;
  const int t = row % a.tokens;
  const int position_base = a.positions[request];
  // the norm weight of this head's kind (the V rows have none; they load q_norm unused)
  const bf16_t *norm_w = kind == 1 ? a.k_norm : a.q_norm;
  const int c0 = column0 + lane * E;
  float raw[E];
  float amax_part = 0.0f, w_scale = 1.0f;
  float part[kSplits > 0 ? kSplits : 1][E];
  if constexpr (kSplits > 0) {
#pragma unroll
    for (int k = 0; k < kSplits; ++k)
#pragma unroll
      for (int e = 0; e < E; ++e)
        part[k][e] = a.partials[(static_cast<size_t>(k) * a.rows + row) * packed_width + c0 + e];
    amax_part = amax_lane(a.x_amax, a.amax_stripes);
    w_scale = *a.w_scale;
  } else {
    if (a.x_amax != nullptr) amax_part = amax_lane(a.x_amax, a.amax_stripes);
    if (a.w_scale != nullptr) w_scale = *a.w_scale;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int c = c0 + e;
      if (a.partials != nullptr) {
        float part[kQkvUnrolledSplits];
#pragma unroll
        for (int k = 0; k < kQkvUnrolledSplits; ++k)
          part[k] = a.partials[(static_cast<size_t>(min(k, a.splits - 1)) * a.rows + row) * packed_width + c];
        float sum = part[0];
#pragma unroll
        for (int k = 1; k < kQkvUnrolledSplits; ++k) sum += k < a.splits ? part[k] : 0.0f;
        for (int k = kQkvUnrolledSplits; k < a.splits; ++k)
          sum += a.partials[(static_cast<size_t>(k) * a.rows + row) * packed_width + c];
        raw[e] = sum;
      } else {
        raw[e] = bf16_to_f32(a.packed[static_cast<size_t>(row) * packed_width + c]);
      }
    }
  }
  float wv[E];
#pragma unroll
  for (int e = 0; e < E; ++e) wv[e] = bf16_to_f32(norm_w[lane * E + e]);
  // every independent load above is issued before the RoPE rows wait for the position
  __asm__ volatile("" ::: "memory");
  if constexpr (kSplits > 0) {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      float sum = part[0][e];
#pragma unroll
      for (int k = 1; k < kSplits; ++k) sum += part[k][e];
      raw[e] = sum;
    }
  }
  const int position = position_base + t + a.position_offset;
  // the RoPE rows of this position: the only loads that wait for another (the position)
  float cs[E], sn[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    cs[e] = bf16_to_f32(a.cosine[static_cast<size_t>(position) * D + lane * E + e]);
    sn[e] = bf16_to_f32(a.sine[static_cast<size_t>(position) * D + lane * E + e]);
  }
  const bool scaled = kSplits > 0 || a.partials != nullptr;
  float scale = w_scale;
  if (kSplits > 0 || a.x_amax != nullptr) scale *= fp8_scale_from_amax(wave_max(amax_part));

  float x[E];
  float square_sum = 0.0f;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const float v = scaled ? round_bf16(raw[e] * scale) : raw[e];
    x[e] = v;
    square_sum += v * v;
  }
  const float inv = inverse_rms(wave_sum(square_sum), D, a.eps);

  auto write_kv = [&](bf16_t *new_rows, bf16_t *cache, const bf16_t (&vals)[E]) {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int i = lane * E + e;
      new_rows[(static_cast<size_t>(row) * hkv + h) * D + i] = vals[e];
      if (cache != nullptr) {
        const size_t cache_row =
            (static_cast<size_t>(a.slots[request]) * hkv + h) * a.capacity + position % a.capacity;
        cache[cache_row * D + i] = vals[e];
      }
    }
  };

  if (kind == 0 || kind == 1) {
    float normalized[E];
#pragma unroll
    for (int e = 0; e < E; ++e) normalized[e] = round_bf16(x[e] * inv * wv[e]);
    bf16_t out[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int i = lane * E + e;
      const float partner = __shfl_xor(normalized[e], 32, kWave);
      const float rotated = i < D / 2 ? -partner : partner;
      out[e] = f32_to_bf16(normalized[e] * cs[e] + rotated * sn[e]);
    }
    if (kind == 0) {
#pragma unroll
      for (int e = 0; e < E; ++e)
        a.q_out[(static_cast<size_t>(row) * hq + h) * D + lane * E + e] = out[e];
    } else {
      write_kv(a.k_new, a.k_cache, out);
    }
  }
  if (kind == 2 || (kind == 1 && a.key_equals_value)) {
    bf16_t out[E];
#pragma unroll
    for (int e = 0; e < E; ++e) out[e] = f32_to_bf16(x[e] * inv);
    write_kv(a.v_new, a.v_cache, out);
  }
}

// Clears every stripe of `amax_count` striped amaxes (stripe i at i * kAmaxStripeFloats).
__global__ void step_init_kernel(float *amax, int amax_count, int32_t *flag) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < amax_count) amax[static_cast<size_t>(i) * kAmaxStripeFloats] = 0.0f;
  if (flag != nullptr && i == 0) *flag = 0;
}

// Greedy longest-prefix acceptance (cuda/batch_model_runner.cu:1738-1759).
__device__ __forceinline__ int accept_one(const int32_t *proposals, const int32_t *predictions,
                                          int first, int cap, int tokens) {
  int accepted = 0;
  while (accepted < cap) {
    const int expected = accepted == 0 ? first : predictions[accepted - 1];
    if (proposals[accepted] != expected) break;
    ++accepted;
  }
  return accepted;
}

__device__ __forceinline__ int clamp_cap(const int32_t *caps, int r, int tokens) {
  if (caps == nullptr) return tokens;
  return min(max(caps[r], 0), tokens);
}

__global__ __launch_bounds__(256) void accept_commit_kernel(const AcceptArgs a) {
  const int r = blockIdx.x;
  const int part = blockIdx.y;  // 0: bookkeeping + hidden; 1..: one sliding layer each
  const int T = a.tokens;
  __shared__ int32_t pred[kMaxAcceptRows];
  __shared__ int accepted_s;
  for (int t = threadIdx.x; t < T; t += blockDim.x) {
    if (a.predictions_missing) {
      pred[t] = -1;
      if (part == 0) a.predictions[r * T + t] = -1;
    } else {
      pred[t] = a.predictions[r * T + t];
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const int accepted = a.force_accept ? T
                                        : accept_one(a.proposals + r * T, pred, a.target_first[r],
                                                     clamp_cap(a.caps, r, T), T);
    accepted_s = accepted;
    if (part == 0) {
      a.accepted[r] = accepted;
      a.next_tokens[r] = accepted == 0 ? a.target_first[r] : pred[accepted - 1];
    }
  }
  __syncthreads();
  const int accepted = accepted_s;
  if (part == 0) {
    if (a.final_hidden != nullptr && accepted > 0) {
      const bf16_t *src = a.final_hidden + static_cast<size_t>(r * T + accepted - 1) * a.hidden;
      bf16_t *dst = a.target_hidden + static_cast<size_t>(a.slots[r]) * a.hidden;
      for (int c = threadIdx.x; c < a.hidden; c += blockDim.x) dst[c] = src[c];
    }
    return;
  }
  const SlidingLayerKv layer = a.layers[part - 1];
  const int D = layer.dimension;
  const int per_row = layer.kv_heads * D;  // elements of one token's K (or V) row
  const int total = accepted * per_row;
  const int p = a.positions[r];
  const int slot = a.slots[r];
  for (int idx = threadIdx.x * 8; idx < total; idx += blockDim.x * 8) {
    const int t = idx / per_row;
    const int within = idx % per_row;
    const int h = within / D;
    const int d = within % D;
    const size_t src = (static_cast<size_t>(r * T + t) * layer.kv_heads + h) * D + d;
    const size_t dst =
        ((static_cast<size_t>(slot) * layer.kv_heads + h) * layer.capacity + (p + t) % layer.capacity) * D + d;
    *reinterpret_cast<uint4 *>(layer.k_cache + dst) = *reinterpret_cast<const uint4 *>(layer.k_new + src);
    *reinterpret_cast<uint4 *>(layer.v_cache + dst) = *reinterpret_cast<const uint4 *>(layer.v_new + src);
  }
}

constexpr int kArgmaxChunkBytes = 32768;  // logits bytes per streaming workgroup

template <bool kF32>
__global__ __launch_bounds__(256) void argmax_partial_kernel(const ArgmaxAcceptArgs a, int chunk,
                                                             int chunks) {
  const int row = blockIdx.y;
  const int begin = blockIdx.x * chunk;
  const int end = min(begin + chunk, a.vocabulary);
  uint64_t best = kArgmaxInitialKey;
  constexpr int kLoads = kArgmaxChunkBytes / (256 * 16);  // 16-byte loads per thread per chunk
  if constexpr (kF32) {
    const float *values = a.logits_f32 + static_cast<size_t>(row) * a.vocabulary;
    if (end - begin == chunk) {
      // Full chunk: every load in flight before the first compare.
      f32x4_t v[kLoads];
#pragma unroll
      for (int l = 0; l < kLoads; ++l)
        v[l] = __builtin_nontemporal_load(
            reinterpret_cast<const f32x4_t *>(values + begin + (l * 256 + threadIdx.x) * 4));
#pragma unroll
      for (int l = 0; l < kLoads; ++l)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint64_t key = argmax_key(
              round_bf16(v[l][q]), static_cast<uint32_t>(begin + (l * 256 + threadIdx.x) * 4 + q));
          best = key > best ? key : best;
        }
    } else
    for (int i = begin + threadIdx.x * 4; i < end; i += blockDim.x * 4) {
      const f32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t *>(values + i));
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint64_t key = argmax_key(round_bf16(v[q]), static_cast<uint32_t>(i + q));
        best = key > best ? key : best;
      }
    }
  } else {
    const bf16_t *values = a.logits_bf16 + static_cast<size_t>(row) * a.vocabulary;
    if (end - begin == chunk) {
      u32x4_t v[kLoads];
#pragma unroll
      for (int l = 0; l < kLoads; ++l)
        v[l] = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4_t *>(values + begin + (l * 256 + threadIdx.x) * 8));
#pragma unroll
      for (int l = 0; l < kLoads; ++l)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t base = begin + (l * 256 + threadIdx.x) * 8 + 2 * q;
          const uint64_t k0 = argmax_key(bf16_to_f32(static_cast<bf16_t>(v[l][q] & 0xffffu)), base);
          const uint64_t k1 = argmax_key(bf16_to_f32(static_cast<bf16_t>(v[l][q] >> 16)), base + 1);
          best = k0 > best ? k0 : best;
          best = k1 > best ? k1 : best;
        }
    } else
    for (int i = begin + threadIdx.x * 8; i < end; i += blockDim.x * 8) {
      const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(values + i));
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint64_t k0 = argmax_key(bf16_to_f32(static_cast<bf16_t>(v[q] & 0xffffu)),
                                       static_cast<uint32_t>(i + 2 * q));
        const uint64_t k1 = argmax_key(bf16_to_f32(static_cast<bf16_t>(v[q] >> 16)),
                                       static_cast<uint32_t>(i + 2 * q + 1));
        best = k0 > best ? k0 : best;
        best = k1 > best ? k1 : best;
      }
    }
  }
  best = wave_max_u64(best);
  __shared__ uint64_t wave_best[4];
  if ((threadIdx.x & 63) == 0) wave_best[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t b = wave_best[0];
    for (int w = 1; w < 4; ++w) b = wave_best[w] > b ? wave_best[w] : b;
    a.partials[static_cast<size_t>(row) * chunks + blockIdx.x] = b;
  }
}

// One workgroup per request: wave w reduces rows w, w + 4 of the request's T rows (all their
// key loads in flight together), then greedy acceptance.
__global__ __launch_bounds__(256) void argmax_accept_final_kernel(const ArgmaxAcceptArgs a,
                                                                  int chunks) {
  const int r = blockIdx.x;
  const int T = a.tokens;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __shared__ int32_t pred[8];
  __shared__ int32_t proposals[8];
  __shared__ int32_t first_cap[2];
  // The acceptance operands load alongside the keys (the last wave has the fewest rows).
  if (a.proposals != nullptr && threadIdx.x >= 192) {
    const int i = threadIdx.x - 192;
    if (i < T) proposals[i] = a.proposals[r * T + i];
    if (i == 8) first_cap[0] = a.target_first[r];
    if (i == 9) first_cap[1] = clamp_cap(a.caps, r, T);
  }
  for (int t = wave; t < T; t += 4) {
    const uint64_t *row = a.partials + static_cast<size_t>(r * T + t) * chunks;
    uint64_t best = kArgmaxInitialKey;
    for (int i = lane; i < chunks; i += 64) best = row[i] > best ? row[i] : best;
    best = wave_max_u64(best);
    if (lane == 0) {
      pred[t] = static_cast<int32_t>(argmax_key_index(best));
      if (a.predictions != nullptr) a.predictions[r * T + t] = pred[t];
    }
  }
  __syncthreads();
  if (threadIdx.x == 0 && a.proposals != nullptr) {
    const int accepted = accept_one(proposals, pred, first_cap[0], first_cap[1], T);
    a.accepted[r] = accepted;
    a.next_tokens[r] = accepted == 0 ? first_cap[0] : pred[accepted - 1];
  }
}

}  // namespace

namespace {
// The layer-end kernel's shape test (see layer_end_kernel): whether it serves `a`, whether the
// partials carry fp8 scale operands, and its quads per thread (0: no instance for the width).
struct LayerEndShape {
  bool fixed = false;
  bool scaled = false;
  int q = 0;
};

LayerEndShape layer_end_shape(const RowArgs &a) {
  LayerEndShape s;
  // fp8 projections' partials carry their scale operands; bf16 ones (the assistant) none
  s.scaled = a.x_amax != nullptr && a.w_scale != nullptr;
  s.fixed = a.source == RowSource::partials && (s.scaled || (a.x_amax == nullptr && a.w_scale == nullptr)) &&
            a.w1 != nullptr && a.residual != nullptr && a.r1_out != nullptr &&
            a.w2 != nullptr && a.y_out != nullptr && (a.y_amax != nullptr || !s.scaled) &&
            a.v_out == nullptr && a.rows < 512 &&
            ((a.splits >= 1 && a.splits <= 4) || a.splits == 8);
  const int quads = a.width / 4;
  // (quads per thread, threads): 5376 wide rows take 448 x 3 with no idle lane
  s.q = a.width == 5376 ? 3 : quads <= 256 ? 5 : quads <= 1024 ? 1 : quads <= 2048 ? 2 : quads <= 4096 ? 4 : 0;
  return s;
}

bool fused_quantization_fits(const RowArgs &a, const LayerEndShape &s) {
  return s.fixed && s.scaled && s.q != 0 && a.rows <= kFusedQuantizeRows && a.y_amax != nullptr &&
         a.width % 128 == 0;
}

// The layer-end shape of the verify step (see layer_end_kernel); false when it does not apply.
bool launch_layer_end(const RowArgs &a, hipStream_t stream) {
  const LayerEndShape shape = layer_end_shape(a);
  const bool scaled = shape.scaled;
  const int q = shape.q;
  if (a.xprep != nullptr &&
      (!fused_quantization_fits(a, shape) || a.sync == nullptr || a.fault == nullptr))
    throw std::runtime_error("fused row quantisation needs the layer-end shape, <= 192 rows and its sync words");
  if (!shape.fixed || q == 0) return false;
  auto go = [&](auto quads_per_thread, auto threads) {
    constexpr int Q = decltype(quads_per_thread)::value;
    constexpr int T = decltype(threads)::value;
    auto pick = [&](auto scaled_constant) {
      constexpr bool S = decltype(scaled_constant)::value;
      switch (a.splits) {
      case 1: layer_end_kernel<Q, T, 1, S><<<a.rows, T, 0, stream>>>(a); break;
      case 2: layer_end_kernel<Q, T, 2, S><<<a.rows, T, 0, stream>>>(a); break;
      case 3: layer_end_kernel<Q, T, 3, S><<<a.rows, T, 0, stream>>>(a); break;
      case 4: layer_end_kernel<Q, T, 4, S><<<a.rows, T, 0, stream>>>(a); break;
      default: layer_end_kernel<Q, T, 8, S><<<a.rows, T, 0, stream>>>(a); break;  // the assistant's down
      }
    };
    if (scaled) pick(std::true_type{}); else pick(std::false_type{});
  };
  using I = std::integral_constant<int, 1>;
  switch (q) {
  case 3: go(std::integral_constant<int, 3>{}, std::integral_constant<int, 448>{}); break;
  case 5: go(I{}, std::integral_constant<int, 256>{}); break;  // rows up to 1024 wide
  case 1: go(I{}, std::integral_constant<int, 1024>{}); break;
  case 2: go(std::integral_constant<int, 2>{}, std::integral_constant<int, 1024>{}); break;
  default: go(std::integral_constant<int, 4>{}, std::integral_constant<int, 1024>{}); break;
  }
  return true;
}
}  // namespace

bool row_kernel_can_fuse_quantization(const RowArgs &a) {
  return fused_quantization_fits(a, layer_end_shape(a));
}

void launch_row_kernel(const RowArgs &a, hipStream_t stream) {
  if (a.rows <= 0 || a.width <= 0) throw std::runtime_error("invalid row kernel shape");
  check_amax_stripes(a.amax_stripes);
  if (a.w2 != nullptr && a.y_out == nullptr) throw std::runtime_error("row kernel: y_out missing");
  if (a.width % 4 != 0) throw std::runtime_error("row kernel: width must be a multiple of 4");
  if (launch_layer_end(a, stream)) {
    hip_check(hipGetLastError(), "launch row kernel");
    return;
  }
  const int per_thread = (a.width / 4 + kRowThreads - 1) / kRowThreads;
  if (per_thread > kRowMaxQuadsPerThread) throw std::runtime_error("row kernel: row too wide");
  // Many rows (prefill steps): 512-thread workgroups, four per CU, so that about a thousand rows
  // run in one round instead of two (measured on MI355X at 1008 x 5376).
  const int per_thread_512 = (a.width / 4 + 511) / 512;
  if (a.rows >= 512 && per_thread_512 <= 4) {
    if (per_thread_512 == 1)
      row_kernel<1, 512><<<a.rows, 512, 0, stream>>>(a);
    else if (per_thread_512 == 2)
      row_kernel<2, 512><<<a.rows, 512, 0, stream>>>(a);
    else if (per_thread_512 == 3)
      row_kernel<3, 512><<<a.rows, 512, 0, stream>>>(a);
    else
      row_kernel<4, 512><<<a.rows, 512, 0, stream>>>(a);
  } else if (per_thread == 1) {
    row_kernel<1><<<a.rows, kRowThreads, 0, stream>>>(a);
  } else if (per_thread == 2) {
    row_kernel<2><<<a.rows, kRowThreads, 0, stream>>>(a);
  } else {
    row_kernel<kRowMaxQuadsPerThread><<<a.rows, kRowThreads, 0, stream>>>(a);
  }
  hip_check(hipGetLastError(), "launch row kernel");
}

void launch_qkv_post(const QkvArgs &a, hipStream_t stream) {
  if (a.rows <= 0 || a.tokens <= 0 || a.rows % a.tokens != 0 || a.query_heads <= 0 ||
      (a.partials == nullptr && a.packed == nullptr) || a.q_out == nullptr ||
      a.positions == nullptr || a.cosine == nullptr || a.sine == nullptr)
    throw std::runtime_error("invalid QKV post-processing shape");
  check_amax_stripes(a.amax_stripes);
  if (a.kv_heads > 0 && (a.k_new == nullptr || a.v_new == nullptr))
    throw std::runtime_error("QKV post-processing needs K/V outputs");
  if (a.q_norm == nullptr || (a.kv_heads > 0 && a.k_norm == nullptr))
    throw std::runtime_error("QKV post-processing needs the query and key norm weights");
  if ((a.k_cache != nullptr || a.v_cache != nullptr) && (a.slots == nullptr || a.capacity <= 0))
    throw std::runtime_error("QKV cache writes need slots and capacity");
  const int heads = a.query_heads + (a.kv_heads == 0 ? 0 : a.kv_heads * (a.key_equals_value ? 1 : 2));
  const dim3 grid(a.rows, heads);
  // compile-time split counts for the projections' partials (1..4), else the generic path
  const int ks = a.partials != nullptr && a.x_amax != nullptr && a.w_scale != nullptr &&
                         a.splits >= 1 && a.splits <= 4
                     ? a.splits
                     : 0;
  auto launch = [&](auto dim) {
    constexpr int D = decltype(dim)::value;
    switch (ks) {
    case 1: qkv_post_kernel<D, 1><<<grid, 64, 0, stream>>>(a); break;
    case 2: qkv_post_kernel<D, 2><<<grid, 64, 0, stream>>>(a); break;
    case 3: qkv_post_kernel<D, 3><<<grid, 64, 0, stream>>>(a); break;
    case 4: qkv_post_kernel<D, 4><<<grid, 64, 0, stream>>>(a); break;
    default: qkv_post_kernel<D, 0><<<grid, 64, 0, stream>>>(a); break;
    }
  };
  switch (a.dimension) {
  case 128: launch(std::integral_constant<int, 128>{}); break;
  case 256: launch(std::integral_constant<int, 256>{}); break;
  case 512: launch(std::integral_constant<int, 512>{}); break;
  default: throw std::runtime_error("QKV post-processing: unsupported head dimension");
  }
  hip_check(hipGetLastError(), "launch QKV post-processing");
}

__global__ __launch_bounds__(64) void amax_fold_kernel(const float *striped, int stripes, float *out) {
  const float value = amax_read(striped, stripes);
  if (threadIdx.x == 0) atomic_max_nonneg(out, value);
}

void launch_amax_fold(const float *striped, int stripes, float *out, hipStream_t stream) {
  check_amax_stripes(stripes);
  amax_fold_kernel<<<1, 64, 0, stream>>>(striped, stripes, out);
  hip_check(hipGetLastError(), "launch amax fold");
}

void launch_step_init(float *amax, int amax_count, hipStream_t stream, int32_t *flag) {
  if (amax_count <= 0) return;
  step_init_kernel<<<(amax_count + 255) / 256, 256, 0, stream>>>(amax, amax_count, flag);
  hip_check(hipGetLastError(), "launch step init");
}

void launch_accept_commit(const AcceptArgs &a, hipStream_t stream) {
  if (a.predictions_missing && !a.force_accept)
    throw std::runtime_error("only forced steps may run without predictions");
  if (a.predictions == nullptr || a.proposals == nullptr || a.target_first == nullptr ||
      a.requests <= 0 || a.tokens <= 0 || a.tokens > kMaxAcceptRows ||
      (!a.force_accept && a.tokens > 8) || a.accepted == nullptr ||
      a.next_tokens == nullptr)
    throw std::runtime_error("invalid acceptance arguments");
  if (a.layer_count > 0 && (a.layers == nullptr || a.slots == nullptr || a.positions == nullptr))
    throw std::runtime_error("KV commit needs layers, slots and positions");
  if (a.final_hidden != nullptr && (a.target_hidden == nullptr || a.slots == nullptr))
    throw std::runtime_error("hidden hand-off needs target rows and slots");
  const dim3 grid(a.requests, 1 + a.layer_count);
  accept_commit_kernel<<<grid, 256, 0, stream>>>(a);
  hip_check(hipGetLastError(), "launch acceptance");
}

int argmax_accept_chunks(int vocabulary, bool f32) {
  const int elems = kArgmaxChunkBytes / (f32 ? 4 : 2);
  return (vocabulary + elems - 1) / elems;
}

void launch_argmax_accept(const ArgmaxAcceptArgs &a, hipStream_t stream) {
  if ((a.logits_f32 == nullptr) == (a.logits_bf16 == nullptr) || a.requests <= 0 ||
      a.tokens <= 0 || a.tokens > 8 || a.vocabulary <= 0 || a.partials == nullptr)
    throw std::runtime_error("invalid argmax arguments");
  if (a.vocabulary % 8 != 0) throw std::runtime_error("argmax vocabulary must be a multiple of 8");
  if (a.proposals != nullptr && (a.target_first == nullptr || a.accepted == nullptr ||
                                 a.next_tokens == nullptr))
    throw std::runtime_error("fused acceptance needs target tokens and outputs");
  const bool f32 = a.logits_f32 != nullptr;
  const int chunks = argmax_accept_chunks(a.vocabulary, f32);
  if (static_cast<size_t>(chunks) * a.requests * a.tokens > a.partial_capacity)
    throw std::runtime_error("argmax partial workspace too small");
  const int chunk = kArgmaxChunkBytes / (f32 ? 4 : 2);
  const dim3 grid(chunks, a.requests * a.tokens);
  if (f32)
    argmax_partial_kernel<true><<<grid, 256, 0, stream>>>(a, chunk, chunks);
  else
    argmax_partial_kernel<false><<<grid, 256, 0, stream>>>(a, chunk, chunks);
  argmax_accept_final_kernel<<<a.requests, 256, 0, stream>>>(a, chunks);
  hip_check(hipGetLastError(), "launch argmax/acceptance");
}

}  // namespace carat_hip
