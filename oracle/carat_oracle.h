/*
 * carat CPU oracle -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain C (C11 + OpenMP) restatement of the reference algorithms on the speculative-decoding
 * verify path of Gradiated/carat. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it, and only as the checker or as the timed CPU baseline. The HIP
 * library never links or calls it.
 *
 * Each function names the reference file:line it restates. bf16 values are carried as uint16_t
 * bit patterns and e4m3 values as uint8_t bit patterns (OCP E4M3FN, max 448, 0x7F = NaN).
 *
 * Pinning status (what checks each function beyond retyping its formula):
 *   orc_acceptance_cap / orc_commit_speculation  -- golden vectors from the reference's own
 *        speculation.cpp compiled into oracle/_ref, and speculation_tests.cpp known answers.
 *   orc_greedy_accept      -- speculative-parity patterns (ragged_batch_parity.cu:212-229),
 *        brute force over every proposal pattern on tiny vocabularies, invariants.
 *   orc_argmax_*           -- test_batched_argmax known answers (cuda_ops_tests.cu:1137-1164),
 *        numpy first-maximum on bf16-rounded rows, NaN/-inf/-0 special cases.
 *   orc_f32_to_e4m3 / orc_quantize_e4m3 -- exhaustive table against an independent
 *        nearest-value search over all 255 codes, plus ml_dtypes-free closed forms.
 *   orc_fp8_linear         -- float64 numpy matmul over the same e4m3 bytes. Parity with the
 *        reference's cuBLASLt kernel is tolerance-only (closed library).
 *   norms / gelu / embedding / qkv / rope -- numpy float64 closed forms.
 *   orc_bf16_linear        -- float64 numpy matmul over the same bf16 operands.
 *   orc_qkv_post           -- float64 closed form of the rotate-half rotation in its stated sense
 *        at nonzero positions, partial rotary (global D/8 pairs) and K=V mode.
 *   orc_verify_attention   -- the reference's own ring+backup formulation restated separately
 *        (orc_ring_backup_attention, cuda_ops_tests.cu:1630-1779) and numpy brute force.
 *   orc_verify_attention_fp8 -- bit-equal to orc_verify_attention on dequantised K/V under
 *        power-of-two scales (exact in bf16), and numpy brute force under any scales.
 *   orc_decode_attention   -- numpy brute force softmax attention.
 */
#ifndef CARAT_ORACLE_H
#define CARAT_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar conversions ---- */
float orc_bf16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float f);
float orc_e4m3_to_f32(uint8_t q);
uint8_t orc_f32_to_e4m3(float f);
void orc_f32_to_bf16_array(const float *x, uint16_t *y, int64_t n);
void orc_f32_to_e4m3_array(const float *x, uint8_t *y, int64_t n);
void orc_bf16_to_f32_array(const uint16_t *x, float *y, int64_t n);

/* ---- speculation helpers (src/runtime/speculation.cpp) ---- */
int orc_acceptance_cap(int depth, int remaining, const int32_t *proposals, int proposal_count,
                       const int32_t *stop_ids, int stop_count);
/* resident/emitted must hold accepted_count + 1 entries; returns stopped flag. */
int orc_commit_speculation(int forced_token, const int32_t *accepted_drafts, int accepted_count,
                           int next_token, const int32_t *stop_ids, int stop_count,
                           int32_t *resident, int *resident_count, int32_t *emitted,
                           int *emitted_count, int32_t *next_out);

/* ---- greedy acceptance (cuda/batch_model_runner.cu:1735-1759) ---- */
void orc_greedy_accept(int requests, int depth, const int32_t *proposals,
                       const int32_t *target_first, const int32_t *predictions,
                       const int32_t *caps, int32_t *accepted, int32_t *next_tokens);

/* ---- argmax (cuda/ops.cu:890-981) ---- */
void orc_argmax_bf16_rows(const uint16_t *logits, int rows, int64_t vocabulary, int32_t *out);
/* fp32 logits, compared after RNE rounding to bf16 (the reference's logits dtype). */
void orc_argmax_f32_rows_as_bf16(const float *logits, int rows, int64_t vocabulary, int32_t *out);

/* ---- FP8 (cuda/linear.cu:76-153, 645-803) ---- */
float orc_quantize_e4m3(const uint16_t *x, int64_t n, float scale_multiplier, uint8_t *q);
void orc_quantize_e4m3_with_amax(const uint16_t *x, int64_t n, float amax, float scale_multiplier,
                                 uint8_t *q, float *scale_out);
void orc_fp8_linear(const uint8_t *qx, float sx, const uint8_t *qw, float sw, int m, int k, int n,
                    uint16_t *out);
void orc_fp8_linear_f32(const uint8_t *qx, float sx, const uint8_t *qw, float sw, int m, int k,
                        int n, float *out);
/* Bf16Linear::run (linear.cu:534-643): bf16 output of an fp32-accumulated GEMM. */
void orc_bf16_linear(const uint16_t *x, const uint16_t *w, int m, int k, int n, uint16_t *out);
/* lm_head restatement: quantize x, fp8 GEMM, bf16 logits, argmax. */
/* Fp8Scaling::channel / ::block_128 (linear.cu:300-420, 706-717): scale = max(amax/448, 2^-24),
 * q = e4m3(x / scale). Row scales [rows]; weight block scales [ceil(n/128)][kbp] (kbp = ceil(k/128)
 * rounded up to 4, padding 0); activation block scales [ceil(k/128)][rows]. scaling 1 channel,
 * 2 block_128. */
void orc_quantize_e4m3_rows(const uint16_t *x, int rows, int width, uint8_t *q, float *scales);
int64_t orc_fp8_weight_block_scale_elements(int n, int k);
void orc_quantize_e4m3_weight_block128(const uint16_t *w, int n, int k, uint8_t *q, float *scales);
void orc_quantize_e4m3_activation_block128(const uint16_t *x, int rows, int k, uint8_t *q,
                                           float *scales);
void orc_fp8_linear_scaled_f32(const uint8_t *qx, const float *sx, const uint8_t *qw,
                               const float *sw, int m, int k, int n, int scaling, float *out);
void orc_fp8_linear_scaled(const uint8_t *qx, const float *sx, const uint8_t *qw, const float *sw,
                           int m, int k, int n, int scaling, uint16_t *out);
void orc_fp8_lm_head_argmax(const uint16_t *x, int m, int k, const uint8_t *qw, float sw, int n,
                            int32_t *argmax_out, uint16_t *logits_out /* nullable */);

/* ---- elementwise / row ops (cuda/ops.cu) ---- */
void orc_rms_norm(const uint16_t *x, const uint16_t *w, const uint16_t *residual, uint16_t *out,
                  float *row_amax, int rows, int width, float eps);
void orc_rms_norm_add_and_norm(const uint16_t *x, const uint16_t *w, const uint16_t *residual,
                               const uint16_t *next_w, uint16_t *residual_out,
                               uint16_t *normalized_out, float *row_amax, int rows, int width,
                               float eps);
void orc_rms_norm_add_scale(const uint16_t *x, const uint16_t *w, const uint16_t *residual,
                            uint16_t scalar, uint16_t *out, int rows, int width, float eps);
void orc_gelu_tanh_gate_rows(const uint16_t *packed, uint16_t *out, float *row_amax, int rows,
                             int width);
void orc_embedding(const uint16_t *weight, const int32_t *tokens, uint16_t *out, int rows,
                   int vocabulary, int hidden, float scale);

/* ---- QKV post-processing (cuda/qkv.cu) ---- */
void orc_rope_table(int dimension, int proportional, int positions, uint16_t *cosine,
                    uint16_t *sine);
/* packed [rows][query_width + kv_width*(k_eq_v?1:2)] -> q [rows][Hq][D], k,v [rows][Hkv][D] */
void orc_qkv_post(const uint16_t *packed, const uint16_t *q_norm, const uint16_t *k_norm,
                  const uint16_t *cosine, const uint16_t *sine, const int32_t *positions,
                  int rows, int query_heads, int kv_heads, int dimension, int key_equals_value,
                  float eps, uint16_t *q_out, uint16_t *k_out, uint16_t *v_out);

/* ---- verify attention (cuda/prefill_gemm_attention.cu) ----
 * q        [R][T][Hq][D] bf16 (token-major)
 * k_cache  [slots][Hkv][C][D] bf16, contents BEFORE this step's proposals were written
 * k_new    [R][T][Hkv][D] bf16 (this step's proposal keys/values)
 * slots[R], positions[R] = tokens already resident (logical position of proposal 0)
 * window = 0 for global causal attention, else the sliding window (ring capacity C == window)
 * round_like_reference: round scores and probabilities to bf16 at the reference's points.
 * out      [R][T][Hq][D] bf16
 */
void orc_verify_attention(const uint16_t *q, const uint16_t *k_cache, const uint16_t *v_cache,
                          const uint16_t *k_new, const uint16_t *v_new, const int32_t *slots,
                          const int32_t *positions, int requests, int tokens, int query_heads,
                          int kv_heads, int dimension, int capacity, int window,
                          int round_like_reference, uint16_t *out);
/* Same but K/V cache held as e4m3 with per-tensor scales (new K/V also e4m3). */
void orc_verify_attention_fp8(const uint16_t *q, const uint8_t *k_cache, const uint8_t *v_cache,
                              const uint8_t *k_new, const uint8_t *v_new, float k_scale,
                              float v_scale, const int32_t *slots, const int32_t *positions,
                              int requests, int tokens, int query_heads, int kv_heads,
                              int dimension, int capacity, uint16_t *out);
/* The reference's ring formulation, restated separately (prefill_gemm_attention.cu:126-298 and
 * its test cuda_ops_tests.cu:1630-1779): the ring already holds the proposals at
 * (p+u)%C, backup[R][Hkv][T][D] holds the overwritten rows, every one of the C physical rows is
 * in the softmax, rows of proposals u > t are replaced by backup u. q head-major [R][Hq][T][D],
 * out head-major, fp32 math. */
void orc_ring_backup_attention(const uint16_t *q_head_major, const uint16_t *k_ring,
                               const uint16_t *v_ring, const uint16_t *k_backup,
                               const uint16_t *v_backup, const int32_t *positions, int requests,
                               int tokens, int query_heads, int kv_heads, int dimension,
                               int capacity, float *out_head_major);

/* ---- assistant decode attention (cuda/gemm_attention.cu:88-132, 618-676) ----
 * q [B][Hq][D]; caches [slots][Hkv][C][D]; valid rows = min(position+1, C). */
void orc_decode_attention(const uint16_t *q, const uint16_t *k_cache, const uint16_t *v_cache,
                          const int32_t *slots, const int32_t *positions, int batch,
                          int query_heads, int kv_heads, int dimension, int capacity,
                          int round_like_reference, uint16_t *out);

/* ---- KV commit (cuda/ops.cu:827-871 backup/restore, restated as its net effect) ----
 * Writes proposal rows t < accepted[r] into ring/contiguous caches at (p+t)%C. */
void orc_commit_kv(uint16_t *k_cache, uint16_t *v_cache, const uint16_t *k_new,
                   const uint16_t *v_new, const int32_t *slots, const int32_t *positions,
                   const int32_t *accepted, int requests, int tokens, int kv_heads, int dimension,
                   int capacity);

#ifdef __cplusplus
}
#endif
#endif
