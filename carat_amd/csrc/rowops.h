// Row-wise fused kernels of the verify step: split-K reduction of the projection GEMMs fused with
// the RMSNorm / residual / layer-scalar epilogues, QKV post-processing (per-head RMSNorm, RoPE,
// KV rows), the step prologue, and acceptance with KV commit.
#pragma once

#include "common.h"

namespace carat_hip {

// ---------------------------------------------------------------------------------------------
// Row kernel. Produces v[row][c] from one of three sources, then applies the epilogue chain:
//   source: embedding  v = bf16(E[token][c] * bf16(embed_scale))          (cuda/ops.cu:321-335)
//           partials   v = bf16(sum_s partial[s][row][c] * scale)         (GEMM split-K reduce)
//           input      v = x[row][c]
//   stage1 (optional): r1 = bf16(norm(v) * w1 + residual) [* scalar -> bf16]  (ops.cu:87-217)
//   stage2 (optional): y  = bf16(norm(r1 or v) * w2), amax(|y|)              (ops.cu:27-85)
// ---------------------------------------------------------------------------------------------
enum class RowSource : int { embedding = 0, partials = 1, input = 2 };

struct RowArgs {
  RowSource source = RowSource::input;
  int rows = 0;
  int width = 0;
  float eps = 1e-6f;
  // embedding
  const bf16_t *embedding = nullptr;
  const int32_t *tokens = nullptr;
  int vocabulary = 0;
  float embed_scale = 1.0f;
  // partials
  const float *partials = nullptr;
  int splits = 1;
  const float *x_amax = nullptr;   // fp8 GEMM: activation amax (nullptr -> scale 1)
  const float *w_scale = nullptr;  // fp8 GEMM: weight scale (nullptr -> 1)
  // input
  const bf16_t *x = nullptr;
  bf16_t *v_out = nullptr;         // optional store of v
  // stage 1
  const bf16_t *w1 = nullptr;      // nullptr: stage 1 skipped
  const bf16_t *residual = nullptr;
  const bf16_t *scalar = nullptr;  // optional layer scalar (device, 1 element)
  bf16_t *r1_out = nullptr;
  // stage 2
  const bf16_t *w2 = nullptr;      // nullptr: stage 2 skipped
  bf16_t *y_out = nullptr;
  float *y_amax = nullptr;
  int amax_stripes = 1;            // floats per amax (x_amax and y_amax), see amax_publish
  // Optional (the verify step's layer-end rows, <= kFusedQuantizeRows rows): y also goes out
  // quantised to e4m3 with its per-tensor scale (amax / 448), in the fp8 GEMM's activation
  // operand layout (gemm.hip prepare_x_kernel's: row-major e4m3),
  // so no separate quantisation kernel runs. The workgroups agree on the amax through `sync`
  // (kFusedSyncWords zeroed words, kAmaxStripeFloats floats apart: arrival counters and the
  // released amax); a wait that exceeds its bound sets *fault and the output is not to be used.
  unsigned char *xprep = nullptr;
  unsigned *sync = nullptr;
  int32_t *fault = nullptr;
  int quantize_spins = kFusedQuantizeSpins;  // bound of a wait for the agreed amax (0: no wait)
};
constexpr int kFusedQuantizeRows = 192;  // every row's workgroup is resident at once (256 CUs)
void launch_row_kernel(const RowArgs &args, hipStream_t stream);
// Whether launch_row_kernel can quantise `args`'s output into the operand workspace (the
// layer-end shape: split-K partials of an fp8 GEMM with 1-4 or 8 splits, both norms, a width
// with a layer-end instance that is a multiple of 128, <= kFusedQuantizeRows rows, the output
// amax). The xprep, sync and fault fields are not looked at.
bool row_kernel_can_fuse_quantization(const RowArgs &args);

// ---------------------------------------------------------------------------------------------
// QKV post-processing (cuda/qkv.cu:387-530): reduces the QKV GEMM partials into the packed row,
// then per head: Q/K RMSNorm with weight + rotate-half RoPE (bf16 cos/sin tables), V weightless
// RMSNorm. Q -> q_out [M][Hq][D]; K/V -> k_new/v_new [M][Hkv][D] and, when given, straight into
// the cache row position % capacity of the request's slot.
// ---------------------------------------------------------------------------------------------
struct QkvArgs {
  const float *partials = nullptr;  // [splits][M][packed_width] (or nullptr with `packed`)
  int splits = 1;
  const float *x_amax = nullptr;
  int amax_stripes = 1;            // floats per x_amax, see amax_publish
  const float *w_scale = nullptr;
  const bf16_t *packed = nullptr;   // alternative source: bf16 packed rows [M][packed_width]
  int rows = 0;                     // M = requests * tokens
  int tokens = 1;                   // T
  int query_heads = 0;
  int kv_heads = 0;                 // 0: queries only (assistant)
  int dimension = 0;
  bool key_equals_value = false;
  float eps = 1e-6f;
  const bf16_t *q_norm = nullptr;
  const bf16_t *k_norm = nullptr;
  const bf16_t *cosine = nullptr;   // [positions][D]
  const bf16_t *sine = nullptr;
  const int32_t *positions = nullptr;  // [R]: row r*T+t sits at positions[r] + t
  const int32_t *slots = nullptr;      // [R] (cache writes only)
  int position_offset = 0;             // added to every position (assistant draft index)
  bf16_t *q_out = nullptr;
  bf16_t *k_new = nullptr;
  bf16_t *v_new = nullptr;
  bf16_t *k_cache = nullptr;  // optional [slots][Hkv][C][D]
  bf16_t *v_cache = nullptr;
  int capacity = 0;
};
void launch_qkv_post(const QkvArgs &args, hipStream_t stream);

// Zeroes the stripes of `amax_count` per-step striped amaxes (stripe i at i * kAmaxStripeFloats).
void launch_step_init(float *amax, int amax_count, hipStream_t stream, int32_t *flag = nullptr);
// Folds a striped amax (`stripes` floats kAmaxStripeFloats apart) into one float with an atomic
// max (the single-float form that op-level callers pass).
void launch_amax_fold(const float *striped, int stripes, float *out, hipStream_t stream);

// ---------------------------------------------------------------------------------------------
// Acceptance + commit (cuda/batch_model_runner.cu:1735-1808, net effect of ops.cu:827-871).
// ---------------------------------------------------------------------------------------------
struct SlidingLayerKv {
  const bf16_t *k_new;  // [M][Hkv][D]
  const bf16_t *v_new;
  bf16_t *k_cache;      // [slots][Hkv][C][D]
  bf16_t *v_cache;
  int kv_heads;
  int dimension;
  int capacity;
  int pad;
};

struct AcceptArgs {
  int32_t *predictions = nullptr;        // [R*T] target argmax of every verified row
  const int32_t *proposals = nullptr;    // [R][T]
  const int32_t *target_first = nullptr; // [R]
  const int32_t *caps = nullptr;         // [R] or nullptr
  int requests = 0;
  int tokens = 0;
  int32_t *accepted = nullptr;           // [R]
  int32_t *next_tokens = nullptr;        // [R]
  // commit (optional)
  const SlidingLayerKv *layers = nullptr;  // device array
  int layer_count = 0;
  const int32_t *slots = nullptr;
  const int32_t *positions = nullptr;
  // hidden hand-off (optional): target_hidden[slot] = final_hidden[r*T + accepted-1]
  const bf16_t *final_hidden = nullptr;
  bf16_t *target_hidden = nullptr;
  int hidden = 0;
  // prefill: every row is accepted (no comparison); next = the prediction after the last row
  bool force_accept = false;
  // forced steps that ran no lm_head: there are no predictions; the kernel sets every row's
  // prediction and every next token to -1 instead of reading stale ones
  bool predictions_missing = false;
};
void launch_accept_commit(const AcceptArgs &args, hipStream_t stream);

// Row argmax (bf16-rounded comparison) over logits held as fp32 (`logits_f32`) or bf16
// (`logits_bf16`): a streaming kernel writes one partial key per (row, chunk) to `partials`
// (argmax_accept_chunks keys per row), then one workgroup per request reduces its T
// rows and runs the greedy acceptance.
struct ArgmaxAcceptArgs {
  const float *logits_f32 = nullptr;
  const bf16_t *logits_bf16 = nullptr;
  int requests = 0;
  int tokens = 0;
  int vocabulary = 0;
  const int32_t *proposals = nullptr;  // nullptr: argmax only
  const int32_t *target_first = nullptr;
  const int32_t *caps = nullptr;
  int32_t *predictions = nullptr;
  int32_t *accepted = nullptr;
  int32_t *next_tokens = nullptr;
  uint64_t *partials = nullptr;
  size_t partial_capacity = 0;  // keys
};
int argmax_accept_chunks(int vocabulary, bool f32);
void launch_argmax_accept(const ArgmaxAcceptArgs &args, hipStream_t stream);

}  // namespace carat_hip
