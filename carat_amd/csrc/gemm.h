// Weight-streaming GEMMs for the verify step: Y[M][N] = X[M][K] . W[N][K]^T for M up to
// kGemmMaxRows tokens (verify steps have M <= 192; prefill steps take more). fp8 (OCP e4m3,
// per-tensor scales, activation quantised on the fly from a producer amax) and bf16 variants,
// fused epilogues. Host-side launch API.
#pragma once

#include "common.h"

namespace carat_hip {

// Token rows per GEMM call. Above 192 the token blocks (128 rows each) of one weight block run
// on the same XCD and share its L2 copy of the weights.
constexpr int kGemmMaxRows = 2048;

enum class GemmEpilogue : int {
  store_bf16 = 0,   // Y = bf16(acc * s) (+ optional amax of the rounded output)
  partial_f32 = 1,  // raw fp32 partial sums per K split: partial[split][M][N]
  argmax = 2,       // per-row argmax keys over bf16(acc * s) (fused lm_head + argmax)
  gelu_gate = 3,    // packed [gate | up] weights: Y[M][N/2] = bf16(gelu(bf16(g s)) * bf16(u s))
};

// Weight storage. Weights stream HBM -> VGPRs exactly once per launch, so they are stored in the
// order the kernel reads them: feature rows are grouped into workgroup blocks of W * F tiles of 16
// rows (F = tiles per wave, W waves), and the block's W * F tiles of one 128-byte K step form one
// contiguous W * F * 2 KiB run: packed[step][block][tile][half][lane][16 B] (step-major, so that
// the runs of one K step of all blocks are contiguous; packed[block][step][...] with step_major
// false), lane = g * 16 + c holding row (tile row c) bytes [step * 128 + half * 64 + g * 16, +16). A gate/up weight
// ([gate rows | up rows], cuda/ops.cu:264-270) puts F/2 gate tiles and the matching F/2 up tiles
// in each wave. The logical matrix stays [N][row_bytes] (pack_weight / unpack_weight convert).
struct WeightLayout {
  int n = 0;               // feature rows
  int row_bytes = 0;       // bytes per row (K for e4m3, 2K for bf16); multiple of 128
  int tiles_per_wave = 1;  // F: 1, 2 or 4 (even for gate/up)
  int waves = 4;           // W: waves per workgroup, 3 or 4 (1 or 2 for few-row weights)
  bool gate_up = false;
  // Step-major order: packed[step][block][...] instead of packed[block][step][...], so that the
  // workgroups of one K step read one contiguous run of the weight.
  bool step_major = false;
};

// Storage layout for an [n][row_bytes] weight: the widest F that still leaves >= 64 workgroups.
// few_rows: the weight serves GEMMs of a few rows per call (the assistant's), which are latency-
// bound; a small grid then takes narrower workgroups (1 or 2 waves).
WeightLayout gemm_weight_layout(int n, int row_bytes, bool gate_up, bool few_rows = false);
int gemm_blocks_n(const WeightLayout &layout);
void pack_weight(const void *row_major, void *packed, const WeightLayout &layout,
                 hipStream_t stream);
void unpack_weight(const void *packed, void *row_major, const WeightLayout &layout,
                   hipStream_t stream);

struct GemmArgs {
  const bf16_t *x = nullptr;   // [M][ldx] bf16 activations
  int ldx = 0;
  int m = 0;
  int k = 0;
  const float *x_amax = nullptr;  // fp8 only: producer amax of x (device); scale = amax/448
  const void *w = nullptr;        // packed e4m3 or bf16 weights (WeightLayout)
  int n = 0;
  WeightLayout w_layout;           // must describe w (n, row bytes, F, gate/up)
  const float *w_scale = nullptr;  // fp8 only: per-tensor weight scale (device)
  // Fp8Scaling (include/carat/linear.h:27): 0 tensor (x_amax, w_scale); 1 channel and
  // 2 block_128 quantise the activations per token row / per token and 128-element K block
  // themselves and scale inside the GEMM, every epilogue's output carrying the full scale:
  // w_scales [n] (channel) or [ceil(n/128)][w_scale_kblocks] (block_128, Fp8WeightArena layout);
  // x_scales a workspace of x_scales_capacity floats (gemm_x_scale_floats).
  int scaling = 0;
  const float *w_scales = nullptr;
  int w_scale_kblocks = 0;
  float *x_scales = nullptr;
  size_t x_scales_capacity = 0;
  int k_splits = 1;
  GemmEpilogue epilogue = GemmEpilogue::store_bf16;
  bf16_t *y = nullptr;             // store_bf16 / gelu_gate output
  int ldy = 0;
  float *y_amax = nullptr;         // optional: atomic max of |rounded output|
  int amax_stripes = 1;            // floats per amax (x_amax and y_amax), see amax_publish
  float *partial = nullptr;        // partial_f32 output, [k_splits][m][n]
  // argmax: per-(token, workgroup) partial keys reduced by a second kernel into argmax_out[m]
  // and, optionally, column `argmax_table_column` of a [m][argmax_table_stride] table.
  uint64_t *argmax_partials = nullptr;
  size_t argmax_partial_capacity = 0;  // in keys
  int32_t *argmax_out = nullptr;
  int32_t *argmax_table = nullptr;
  int argmax_table_stride = 0;
  int argmax_table_column = 0;
  // argmax: leave the partial keys for the caller to reduce (no reduction kernel; argmax_out and
  // the table are not written)
  bool argmax_deferred = false;
  // e4m3 GEMMs only: activation operand workspace (gemm_xprep_bytes); bf16 GEMMs read x directly
  unsigned char *xprep = nullptr;
  size_t xprep_capacity = 0;
  bool xprep_ready = false;  // e4m3: xprep already holds this call's prepared activations
  // optional: events recorded around the main GEMM kernel (timing probes)
  hipEvent_t timing_start = nullptr;
  hipEvent_t timing_stop = nullptr;
};

// Bytes of the e4m3 activation operand workspace for m rows of k elements.
size_t gemm_xprep_bytes(int m, int k);
// Floats of the activation scale workspace of a scaled (channel / block_128) e4m3 GEMM.
size_t gemm_x_scale_floats(int m, int k);
// 16-token tiles per token block of the e4m3 activation operand for m rows (2 or 8).
inline int gemm_token_tiles(int m) { return m <= 32 ? 2 : 8; }
// Keys of the argmax partial workspace for an m-row lm_head of this layout.
size_t gemm_argmax_partials(int m, const WeightLayout &layout);
// Split-K factor: a divisor of k_steps (128-byte steps) that fills the GPU.
int gemm_choose_splits(int n_blocks, int k_steps);

// fp8 weights (e4m3) with bf16 activations quantised in the prologue.
void launch_fp8_gemm(const GemmArgs &args, hipStream_t stream);
// bf16 weights and activations.
void launch_bf16_gemm(const GemmArgs &args, hipStream_t stream);

}  // namespace carat_hip
