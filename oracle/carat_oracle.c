/*
 * carat CPU oracle -- TEST INFRASTRUCTURE ONLY (see carat_oracle.h for the pinning status of
 * every function). Plain C11 + OpenMP; no part of the HIP product links this file.
 */
#include "carat_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------------------------ */
/* scalar conversions                                                                          */
/* ------------------------------------------------------------------------------------------ */

static inline uint32_t f2u(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static inline float u2f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

float orc_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* Round-to-nearest-even float -> bf16, the behaviour of __float2bfloat16_rn. */
uint16_t orc_f32_to_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static inline float bf(float f) { return orc_bf16_to_f32(orc_f32_to_bf16(f)); }

float orc_e4m3_to_f32(uint8_t q) {
  const int sign = q >> 7;
  const int exponent = (q >> 3) & 0xf;
  const int mantissa = q & 7;
  float v;
  if (exponent == 0xf && mantissa == 7) return NAN;
  if (exponent == 0)
    v = ldexpf((float)mantissa, -9);
  else
    v = ldexpf(1.0f + (float)mantissa / 8.0f, exponent - 7);
  return sign ? -v : v;
}

/* float -> OCP e4m3, round to nearest even with saturation to +-448 (the documented behaviour of
 * the __nv_fp8_e4m3(float) constructor used at cuda/linear.cu:110,128,186). */
uint8_t orc_f32_to_e4m3(float f) {
  const uint32_t u = f2u(f);
  const uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
  const uint32_t a_bits = u & 0x7fffffffu;
  if (a_bits > 0x7f800000u) return (uint8_t)(sign | 0x7f);
  const int e = (int)(a_bits >> 23) - 127;
  uint32_t code;
  if (e >= -6) {
    uint32_t keep = (a_bits & 0x7fffffu) >> 20;
    const uint32_t rem = a_bits & 0xfffffu;
    int ee = e;
    if (rem > 0x80000u || (rem == 0x80000u && (keep & 1u))) keep++;
    if (keep == 8) {
      keep = 0;
      ee++;
    }
    if (ee > 8) return (uint8_t)(sign | 0x7e);
    code = ((uint32_t)(ee + 7) << 3) | keep;
    if (code > 0x7e) code = 0x7e;
  } else {
    const float s = u2f(a_bits) * 512.0f; /* exact: power-of-two scaling */
    float r = floorf(s);
    const float diff = s - r;
    if (diff > 0.5f || (diff == 0.5f && fmodf(r, 2.0f) != 0.0f)) r += 1.0f;
    code = (uint32_t)r; /* 0..8; 8 encodes 2^-6, the smallest normal */
  }
  return (uint8_t)(sign | code);
}

void orc_f32_to_bf16_array(const float *x, uint16_t *y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = orc_f32_to_bf16(x[i]);
}
void orc_f32_to_e4m3_array(const float *x, uint8_t *y, int64_t n) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) y[i] = orc_f32_to_e4m3(x[i]);
}
void orc_bf16_to_f32_array(const uint16_t *x, float *y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = orc_bf16_to_f32(x[i]);
}

/* ------------------------------------------------------------------------------------------ */
/* speculation helpers: src/runtime/speculation.cpp:7-36                                        */
/* ------------------------------------------------------------------------------------------ */

static int is_stop(int token, const int32_t *stop_ids, int stop_count) {
  for (int i = 0; i < stop_count; ++i)
    if (stop_ids[i] == token) return 1;
  return 0;
}

/* speculation.cpp:7-18 -- min(depth, remaining), ended after the first stop at index >= 1. */
int orc_acceptance_cap(int depth, int remaining, const int32_t *proposals, int proposal_count,
                       const int32_t *stop_ids, int stop_count) {
  const int cap = depth < remaining ? depth : remaining;
  const int inspected = cap < proposal_count ? cap : proposal_count;
  for (int index = 1; index < inspected; ++index)
    if (is_stop(proposals[index], stop_ids, stop_count)) return index + 1;
  return cap;
}

/* speculation.cpp:20-36 */
int orc_commit_speculation(int forced_token, const int32_t *accepted_drafts, int accepted_count,
                           int next_token, const int32_t *stop_ids, int stop_count,
                           int32_t *resident, int *resident_count, int32_t *emitted,
                           int *emitted_count, int32_t *next_out) {
  int nr = 0, ne = 0;
  resident[nr++] = forced_token;
  *next_out = next_token;
  for (int i = 0; i < accepted_count; ++i) {
    const int token = accepted_drafts[i];
    resident[nr++] = token;
    emitted[ne++] = token;
    if (is_stop(token, stop_ids, stop_count)) {
      *resident_count = nr;
      *emitted_count = ne;
      return 1;
    }
  }
  emitted[ne++] = next_token;
  *resident_count = nr;
  *emitted_count = ne;
  return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* greedy acceptance: cuda/batch_model_runner.cu:1735-1759                                     */
/* ------------------------------------------------------------------------------------------ */

void orc_greedy_accept(int requests, int depth, const int32_t *proposals,
                       const int32_t *target_first, const int32_t *predictions,
                       const int32_t *caps, int32_t *accepted, int32_t *next_tokens) {
  for (int r = 0; r < requests; ++r) {
    int cap = depth;
    if (caps) {
      cap = caps[r];
      if (cap < 0) cap = 0;
      if (cap > depth) cap = depth;
    }
    int a = 0;
    while (a < cap) {
      const int expected = a == 0 ? target_first[r] : predictions[r * depth + a - 1];
      if (proposals[r * depth + a] != expected) break;
      ++a;
    }
    accepted[r] = a;
    next_tokens[r] = a == 0 ? target_first[r] : predictions[r * depth + a - 1];
  }
}

/* ------------------------------------------------------------------------------------------ */
/* argmax: cuda/ops.cu:890-981 -- a strictly greater value wins, equal values keep the lower    */
/* index, NaN never wins (comparisons are false), the running best starts at (-inf, 0).        */
/* ------------------------------------------------------------------------------------------ */

static int32_t argmax_row_values(const float *v, int64_t n) {
  float best = -INFINITY;
  int64_t best_index = 0;
  for (int64_t i = 0; i < n; ++i) {
    if (v[i] > best) {
      best = v[i];
      best_index = i;
    }
  }
  return (int32_t)best_index;
}

void orc_argmax_bf16_rows(const uint16_t *logits, int rows, int64_t vocabulary, int32_t *out) {
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; ++r) {
    const uint16_t *row = logits + (int64_t)r * vocabulary;
    float best = -INFINITY;
    int64_t best_index = 0;
    for (int64_t i = 0; i < vocabulary; ++i) {
      const float v = orc_bf16_to_f32(row[i]);
      if (v > best) {
        best = v;
        best_index = i;
      }
    }
    out[r] = (int32_t)best_index;
  }
}

void orc_argmax_f32_rows_as_bf16(const float *logits, int rows, int64_t vocabulary, int32_t *out) {
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; ++r) {
    const float *row = logits + (int64_t)r * vocabulary;
    float best = -INFINITY;
    int64_t best_index = 0;
    for (int64_t i = 0; i < vocabulary; ++i) {
      const float v = bf(row[i]);
      if (v > best) {
        best = v;
        best_index = i;
      }
    }
    out[r] = (int32_t)best_index;
  }
  (void)argmax_row_values;
}

/* ------------------------------------------------------------------------------------------ */
/* FP8: cuda/linear.cu:76-153 (per-tensor scale = amax * multiplier / 448, 1 when amax == 0;    */
/* q = e4m3(x * (1 / scale))) and Fp8Linear::run (linear.cu:780-803):                           */
/* Y = bf16(scale_x * scale_w * sum_k qx[m,k] * qw[n,k]), fp32 accumulation.                     */
/* ------------------------------------------------------------------------------------------ */

void orc_quantize_e4m3_with_amax(const uint16_t *x, int64_t n, float amax, float scale_multiplier,
                                 uint8_t *q, float *scale_out) {
  const float scale = amax > 0.0f ? amax * scale_multiplier / 448.0f : 1.0f;
  const float inverse = 1.0f / scale;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) q[i] = orc_f32_to_e4m3(orc_bf16_to_f32(x[i]) * inverse);
  *scale_out = scale;
}

float orc_quantize_e4m3(const uint16_t *x, int64_t n, float scale_multiplier, uint8_t *q) {
  float amax = 0.0f;
  for (int64_t i = 0; i < n; ++i) amax = fmaxf(amax, fabsf(orc_bf16_to_f32(x[i])));
  float scale;
  orc_quantize_e4m3_with_amax(x, n, amax, scale_multiplier, q, &scale);
  return scale;
}

/* Shared by the fp8 and bf16 GEMMs: out[row][col] = s * sum_k x[row][k] * w[col][k] over
 * float operands, accumulated in double per output (so the summation order does not matter at
 * the tolerance the tests use). Four token rows share each weight row pass. */
static void linear_f32_rows(const float *xf, int m, int k,
                            int n, float s, float *out, const uint8_t *qw, const float *table,
                            const uint16_t *bw) {
#pragma omp parallel
  {
    float *wrow = (float *)malloc(sizeof(float) * (size_t)(k > 0 ? k : 1));
#pragma omp for schedule(static)
    for (int col = 0; col < n; ++col) {
      if (qw)
        for (int kk = 0; kk < k; ++kk) wrow[kk] = table[qw[(int64_t)col * k + kk]];
      else
        for (int kk = 0; kk < k; ++kk) wrow[kk] = orc_bf16_to_f32(bw[(int64_t)col * k + kk]);
      int row = 0;
      for (; row + 4 <= m; row += 4) {
        const float *x0 = xf + (int64_t)row * k, *x1 = x0 + k, *x2 = x1 + k, *x3 = x2 + k;
        double a0 = 0.0, a1 = 0.0, a2 = 0.0, a3 = 0.0;
        for (int kk = 0; kk < k; ++kk) {
          const double w = wrow[kk];
          a0 += (double)x0[kk] * w;
          a1 += (double)x1[kk] * w;
          a2 += (double)x2[kk] * w;
          a3 += (double)x3[kk] * w;
        }
        out[(int64_t)row * n + col] = (float)a0 * s;
        out[(int64_t)(row + 1) * n + col] = (float)a1 * s;
        out[(int64_t)(row + 2) * n + col] = (float)a2 * s;
        out[(int64_t)(row + 3) * n + col] = (float)a3 * s;
      }
      for (; row < m; ++row) {
        const float *xr = xf + (int64_t)row * k;
        double acc = 0.0;
        for (int kk = 0; kk < k; ++kk) acc += (double)xr[kk] * wrow[kk];
        out[(int64_t)row * n + col] = (float)acc * s;
      }
    }
    free(wrow);
  }
}

void orc_fp8_linear_f32(const uint8_t *qx, float sx, const uint8_t *qw, float sw, int m, int k,
                        int n, float *out) {
  float table[256];
  for (int i = 0; i < 256; ++i) table[i] = orc_e4m3_to_f32((uint8_t)i);
  float *xf = (float *)malloc(sizeof(float) * (size_t)m * k);
  for (int64_t i = 0; i < (int64_t)m * k; ++i) xf[i] = table[qx[i]];
  linear_f32_rows(xf, m, k, n, sx * sw, out, qw, table, NULL);
  free(xf);
}

/* Bf16Linear::run (linear.cu:534-643; cuBLASLt bf16 GEMM, fp32 accumulation, bf16 output):
 * Y[m][n] = bf16(sum_k x[m][k] * w[n][k]). The assistant's projections and lm_head
 * (assistant_runner.cu:147-160, AssistantFp8Mode::off). */
void orc_bf16_linear(const uint16_t *x, const uint16_t *w, int m, int k, int n, uint16_t *out) {
  float *xf = (float *)malloc(sizeof(float) * (size_t)m * k);
  float *tmp = (float *)malloc(sizeof(float) * (size_t)m * n);
  for (int64_t i = 0; i < (int64_t)m * k; ++i) xf[i] = orc_bf16_to_f32(x[i]);
  linear_f32_rows(xf, m, k, n, 1.0f, tmp, NULL, NULL, w);
  for (int64_t i = 0; i < (int64_t)m * n; ++i) out[i] = orc_f32_to_bf16(tmp[i]);
  free(tmp);
  free(xf);
}

void orc_fp8_linear(const uint8_t *qx, float sx, const uint8_t *qw, float sw, int m, int k, int n,
                    uint16_t *out) {
  float *tmp = (float *)malloc(sizeof(float) * (size_t)m * n);
  orc_fp8_linear_f32(qx, sx, qw, sw, m, k, n, tmp);
  for (int64_t i = 0; i < (int64_t)m * n; ++i) out[i] = orc_f32_to_bf16(tmp[i]);
  free(tmp);
}

/* cuda/batch_model_runner.cu:840-853 (quantize final hidden, FP8 lm_head) and :1727-1729
 * (argmax over the bf16 logits). */
void orc_fp8_lm_head_argmax(const uint16_t *x, int m, int k, const uint8_t *qw, float sw, int n,
                            int32_t *argmax_out, uint16_t *logits_out) {
  uint8_t *qx = (uint8_t *)malloc((size_t)m * k);
  const float sx = orc_quantize_e4m3(x, (int64_t)m * k, 1.0f, qx);
  uint16_t *logits = logits_out ? logits_out : (uint16_t *)malloc(sizeof(uint16_t) * (size_t)m * n);
  orc_fp8_linear(qx, sx, qw, sw, m, k, n, logits);
  orc_argmax_bf16_rows(logits, m, n, argmax_out);
  if (!logits_out) free(logits);
  free(qx);
}

/* ------------------------------------------------------------------------------------------ */
/* Fp8Scaling::channel and ::block_128 (include/carat/linear.h:27, cuda/linear.cu:300-420,      */
/* 706-717; Fp8WeightArena::quantize device_weights.cu:222-256; run_decode_linear                */
/* layer_runner.cu:220-238). Every scale is max(amax / 448, 2^-24) and q = e4m3(x / scale):     */
/*  - channel: one scale per weight row [n] and per activation row [m] (quantize_bf16_rows);   */
/*  - block_128: one scale per 128 x 128 weight block, [ceil(n/128)][kbp] with kbp =           */
/*    ceil(k/128) rounded up to a multiple of 4 (padding zeroed), and one per 1 x 128           */
/*    activation block, [ceil(k/128)][m];                                                      */
/* Y[m][n] = bf16(sum over K blocks b of (sx(m, b) * sw(n, b)) * sum_{k in b} qx * qw), with   */
/* channel as the one-block case (sx(m), sw(n)).                                               */
/* ------------------------------------------------------------------------------------------ */

static float scaled_block_scale(float amax) { return fmaxf(amax / 448.0f, 0x1p-24f); }

/* quantize_bf16_rows_kernel (linear.cu:300-316): rows x width, scales[rows] */
void orc_quantize_e4m3_rows(const uint16_t *x, int rows, int width, uint8_t *q, float *scales) {
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; ++r) {
    const uint16_t *xr = x + (int64_t)r * width;
    float amax = 0.0f;
    for (int c = 0; c < width; ++c) amax = fmaxf(amax, fabsf(orc_bf16_to_f32(xr[c])));
    const float scale = scaled_block_scale(amax);
    scales[r] = scale;
    for (int c = 0; c < width; ++c) q[(int64_t)r * width + c] = orc_f32_to_e4m3(orc_bf16_to_f32(xr[c]) / scale);
  }
}

int64_t orc_fp8_weight_block_scale_elements(int n, int k) {
  const int64_t kb = (k + 127) / 128;
  return ((kb + 3) & ~(int64_t)3) * ((n + 127) / 128);
}

/* quantize_weight_block_128_kernel (linear.cu:352-380): w [n][k] */
void orc_quantize_e4m3_weight_block128(const uint16_t *w, int n, int k, uint8_t *q, float *scales) {
  const int kb_count = (k + 127) / 128, kbp = (kb_count + 3) & ~3, nb_count = (n + 127) / 128;
  memset(scales, 0, sizeof(float) * (size_t)kbp * nb_count);
#pragma omp parallel for collapse(2) schedule(static)
  for (int nb = 0; nb < nb_count; ++nb)
    for (int kb = 0; kb < kb_count; ++kb) {
      float amax = 0.0f;
      for (int r = nb * 128; r < n && r < nb * 128 + 128; ++r)
        for (int c = kb * 128; c < k && c < kb * 128 + 128; ++c)
          amax = fmaxf(amax, fabsf(orc_bf16_to_f32(w[(int64_t)r * k + c])));
      const float scale = scaled_block_scale(amax);
      scales[(int64_t)nb * kbp + kb] = scale;
      for (int r = nb * 128; r < n && r < nb * 128 + 128; ++r)
        for (int c = kb * 128; c < k && c < kb * 128 + 128; ++c)
          q[(int64_t)r * k + c] = orc_f32_to_e4m3(orc_bf16_to_f32(w[(int64_t)r * k + c]) / scale);
    }
}

/* quantize_activation_block_128_kernel (linear.cu:382-401): x [rows][k], scales[kb][rows] */
void orc_quantize_e4m3_activation_block128(const uint16_t *x, int rows, int k, uint8_t *q,
                                           float *scales) {
  const int kb_count = (k + 127) / 128;
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; ++r)
    for (int kb = 0; kb < kb_count; ++kb) {
      const uint16_t *xr = x + (int64_t)r * k;
      float amax = 0.0f;
      for (int c = kb * 128; c < k && c < kb * 128 + 128; ++c) amax = fmaxf(amax, fabsf(orc_bf16_to_f32(xr[c])));
      const float scale = scaled_block_scale(amax);
      scales[(int64_t)kb * rows + r] = scale;
      for (int c = kb * 128; c < k && c < kb * 128 + 128; ++c)
        q[(int64_t)r * k + c] = orc_f32_to_e4m3(orc_bf16_to_f32(xr[c]) / scale);
    }
}

/* Fp8Linear::run with OUTER_VEC (channel) or VEC128 x BLK128x128 (block_128) scales
 * (linear.cu:706-717): fp32 out[m][n]; each block's dot product is exact in double, scaled by
 * the fp32 product sx * sw and summed in double. scaling: 1 channel, 2 block_128. */
void orc_fp8_linear_scaled_f32(const uint8_t *qx, const float *sx, const uint8_t *qw,
                               const float *sw, int m, int k, int n, int scaling, float *out) {
  float table[256];
  for (int i = 0; i < 256; ++i) table[i] = orc_e4m3_to_f32((uint8_t)i);
  const int kb_count = (k + 127) / 128, kbp = (kb_count + 3) & ~3;
#pragma omp parallel for schedule(static)
  for (int col = 0; col < n; ++col) {
    const uint8_t *wr = qw + (int64_t)col * k;
    for (int row = 0; row < m; ++row) {
      const uint8_t *xr = qx + (int64_t)row * k;
      double total = 0.0;
      if (scaling == 1) {
        double acc = 0.0;
        for (int c = 0; c < k; ++c) acc += (double)table[xr[c]] * table[wr[c]];
        total = (double)((float)acc * (sx[row] * sw[col]));
      } else {
        for (int kb = 0; kb < kb_count; ++kb) {
          double acc = 0.0;
          for (int c = kb * 128; c < k && c < kb * 128 + 128; ++c) acc += (double)table[xr[c]] * table[wr[c]];
          total += acc * (double)(sx[(int64_t)kb * m + row] * sw[(int64_t)(col / 128) * kbp + kb]);
        }
      }
      out[(int64_t)row * n + col] = (float)total;
    }
  }
}

void orc_fp8_linear_scaled(const uint8_t *qx, const float *sx, const uint8_t *qw, const float *sw,
                           int m, int k, int n, int scaling, uint16_t *out) {
  float *tmp = (float *)malloc(sizeof(float) * (size_t)m * n);
  orc_fp8_linear_scaled_f32(qx, sx, qw, sw, m, k, n, scaling, tmp);
  for (int64_t i = 0; i < (int64_t)m * n; ++i) out[i] = orc_f32_to_bf16(tmp[i]);
  free(tmp);
}

/* ------------------------------------------------------------------------------------------ */
/* row ops: cuda/ops.cu:27-217 (RMSNorm variants), 228-284 (GELU gate), 321-335 (embedding)     */
/* ------------------------------------------------------------------------------------------ */

static float inverse_rms_bf16(const uint16_t *x, int width, float eps) {
  float sum = 0.0f;
  for (int c = 0; c < width; ++c) {
    const float v = orc_bf16_to_f32(x[c]);
    sum += v * v;
  }
  return 1.0f / sqrtf(sum / (float)width + eps);
}

/* ops.cu:27-85: out = bf16(x * inv_rms * w [+ residual]); row amax of the rounded output. */
void orc_rms_norm(const uint16_t *x, const uint16_t *w, const uint16_t *residual, uint16_t *out,
                  float *row_amax, int rows, int width, float eps) {
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; ++r) {
    const uint16_t *xr = x + (int64_t)r * width;
    const float inv = inverse_rms_bf16(xr, width, eps);
    float m = 0.0f;
    for (int c = 0; c < width; ++c) {
      float v = orc_bf16_to_f32(xr[c]) * inv * orc_bf16_to_f32(w[c]);
      if (residual) v += orc_bf16_to_f32(residual[(int64_t)r * width + c]);
      const uint16_t h = orc_f32_to_bf16(v);
      out[(int64_t)r * width + c] = h;
      m = fmaxf(m, fabsf(orc_bf16_to_f32(h)));
    }
    if (row_amax) row_amax[r] = m;
  }
}

/* ops.cu:87-179: r1 = bf16(norm(x)*w + residual); y = bf16(norm(r1)*next_w); amax(y). */
void orc_rms_norm_add_and_norm(const uint16_t *x, const uint16_t *w, const uint16_t *residual,
                               const uint16_t *next_w, uint16_t *residual_out,
                               uint16_t *normalized_out, float *row_amax, int rows, int width,
                               float eps) {
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; ++r) {
    const uint16_t *xr = x + (int64_t)r * width;
    uint16_t *r1 = residual_out + (int64_t)r * width;
    const float inv = inverse_rms_bf16(xr, width, eps);
    for (int c = 0; c < width; ++c)
      r1[c] = orc_f32_to_bf16(orc_bf16_to_f32(xr[c]) * inv * orc_bf16_to_f32(w[c]) +
                              orc_bf16_to_f32(residual[(int64_t)r * width + c]));
    const float inv2 = inverse_rms_bf16(r1, width, eps);
    float m = 0.0f;
    for (int c = 0; c < width; ++c) {
      const uint16_t h = orc_f32_to_bf16(orc_bf16_to_f32(r1[c]) * inv2 * orc_bf16_to_f32(next_w[c]));
      normalized_out[(int64_t)r * width + c] = h;
      m = fmaxf(m, fabsf(orc_bf16_to_f32(h)));
    }
    if (row_amax) row_amax[r] = m;
  }
}

/* ops.cu:181-217: out = bf16(bf16(norm(x)*w + residual) * scalar). */
void orc_rms_norm_add_scale(const uint16_t *x, const uint16_t *w, const uint16_t *residual,
                            uint16_t scalar, uint16_t *out, int rows, int width, float eps) {
  const float s = orc_bf16_to_f32(scalar);
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; ++r) {
    const uint16_t *xr = x + (int64_t)r * width;
    const float inv = inverse_rms_bf16(xr, width, eps);
    for (int c = 0; c < width; ++c) {
      const float rv = bf(orc_bf16_to_f32(xr[c]) * inv * orc_bf16_to_f32(w[c]) +
                          orc_bf16_to_f32(residual[(int64_t)r * width + c]));
      out[(int64_t)r * width + c] = orc_f32_to_bf16(rv * s);
    }
  }
}

static float gelu_tanh(float v) {
  const float coefficient = 0.7978845608028654f;
  return 0.5f * v * (1.0f + tanhf(coefficient * (v + 0.044715f * v * v * v)));
}

/* ops.cu:228-284: out = bf16(gelu_tanh(g) * u) from packed rows [g | u]; row amax. */
void orc_gelu_tanh_gate_rows(const uint16_t *packed, uint16_t *out, float *row_amax, int rows,
                             int width) {
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; ++r) {
    const uint16_t *base = packed + (int64_t)r * 2 * width;
    float m = 0.0f;
    for (int c = 0; c < width; ++c) {
      const uint16_t h =
          orc_f32_to_bf16(gelu_tanh(orc_bf16_to_f32(base[c])) * orc_bf16_to_f32(base[width + c]));
      out[(int64_t)r * width + c] = h;
      m = fmaxf(m, fabsf(orc_bf16_to_f32(h)));
    }
    if (row_amax) row_amax[r] = m;
  }
}

/* ops.cu:321-335 with the wrapper's bf16(scale) (:1140-1153). */
void orc_embedding(const uint16_t *weight, const int32_t *tokens, uint16_t *out, int rows,
                   int vocabulary, int hidden, float scale) {
  const float s = bf(scale);
  for (int r = 0; r < rows; ++r) {
    const int t = tokens[r];
    if (t < 0 || t >= vocabulary) continue;
    for (int c = 0; c < hidden; ++c)
      out[(int64_t)r * hidden + c] =
          orc_f32_to_bf16(orc_bf16_to_f32(weight[(int64_t)t * hidden + c]) * s);
  }
}

/* ------------------------------------------------------------------------------------------ */
/* QKV post-processing: cuda/qkv.cu:44-64 (RoPE tables), 387-422 (queries), 477-530 (K/V)      */
/* ------------------------------------------------------------------------------------------ */

/* qkv.cu:44-64. Sliding: theta 1e4 over all D/2 frequencies. Global ("proportional"):
 * theta 1e6, only the first D/8 half-indices rotate (partial rotary of D/4). Evaluated in
 * double precision then rounded to bf16. */
void orc_rope_table(int dimension, int proportional, int positions, uint16_t *cosine,
                    uint16_t *sine) {
  for (int p = 0; p < positions; ++p) {
    for (int i = 0; i < dimension; ++i) {
      const int half_index = i % (dimension / 2);
      double frequency = 0.0;
      if (proportional) {
        if (half_index < dimension / 8)
          frequency = pow(1000000.0, -2.0 * half_index / dimension);
      } else {
        frequency = pow(10000.0, -2.0 * half_index / dimension);
      }
      const float f32_frequency = (float)frequency;
      const double angle = (double)((float)p * f32_frequency);
      cosine[(int64_t)p * dimension + i] = orc_f32_to_bf16((float)cos(angle));
      sine[(int64_t)p * dimension + i] = orc_f32_to_bf16((float)sin(angle));
    }
  }
}

static void norm_rope_head(const uint16_t *in, const uint16_t *w, const uint16_t *cosine,
                           const uint16_t *sine, int position, int dimension, float eps,
                           uint16_t *out) {
  const float inv = inverse_rms_bf16(in, dimension, eps);
  const int half = dimension / 2;
  for (int i = 0; i < dimension; ++i) {
    const int partner = i < half ? i + half : i - half;
    const float normalized = bf(orc_bf16_to_f32(in[i]) * inv * orc_bf16_to_f32(w[i]));
    const float partner_normalized =
        bf(orc_bf16_to_f32(in[partner]) * inv * orc_bf16_to_f32(w[partner]));
    const float rotated = i < half ? -partner_normalized : partner_normalized;
    const float c = orc_bf16_to_f32(cosine[(int64_t)position * dimension + i]);
    const float s = orc_bf16_to_f32(sine[(int64_t)position * dimension + i]);
    out[i] = orc_f32_to_bf16(normalized * c + rotated * s);
  }
}

void orc_qkv_post(const uint16_t *packed, const uint16_t *q_norm, const uint16_t *k_norm,
                  const uint16_t *cosine, const uint16_t *sine, const int32_t *positions,
                  int rows, int query_heads, int kv_heads, int dimension, int key_equals_value,
                  float eps, uint16_t *q_out, uint16_t *k_out, uint16_t *v_out) {
  const int query_width = query_heads * dimension;
  const int kv_width = kv_heads * dimension;
  const int packed_width = query_width + kv_width * (key_equals_value ? 1 : 2);
#pragma omp parallel for schedule(static)
  for (int row = 0; row < rows; ++row) {
    const uint16_t *base = packed + (int64_t)row * packed_width;
    const int position = positions[row];
    for (int h = 0; h < query_heads; ++h)
      norm_rope_head(base + h * dimension, q_norm, cosine, sine, position, dimension, eps,
                     q_out + ((int64_t)row * query_heads + h) * dimension);
    for (int h = 0; h < kv_heads; ++h) {
      const uint16_t *k_in = base + query_width + h * dimension;
      const uint16_t *v_in = key_equals_value ? k_in : base + query_width + kv_width + h * dimension;
      norm_rope_head(k_in, k_norm, cosine, sine, position, dimension, eps,
                     k_out + ((int64_t)row * kv_heads + h) * dimension);
      const float inv_v = inverse_rms_bf16(v_in, dimension, eps);
      for (int i = 0; i < dimension; ++i)
        v_out[((int64_t)row * kv_heads + h) * dimension + i] =
            orc_f32_to_bf16(orc_bf16_to_f32(v_in[i]) * inv_v);
    }
  }
}

/* ------------------------------------------------------------------------------------------ */
/* verify attention                                                                              */
/* ------------------------------------------------------------------------------------------ */

/* Logical restatement of the reference's two verify attention paths:
 *  - sliding (run_uniform_ring_batch, prefill_gemm_attention.cu:657-730, and the unwrapped
 *    direct path layer_runner.cu:851-880): query at position q sees keys j with
 *    q - window + 1 <= j <= q, j >= 0;
 *  - global (run_uniform_batch, :552-610, causal softmax :300-349): keys 0 <= j <= q.
 * Keys j < p come from the cache at physical row j % C; keys p + u come from this step's new
 * rows. No 1/sqrt(D) scaling (Gemma 4 normalises q and k). With round_like_reference the scores
 * and probabilities are rounded to bf16 (the reference's QK GEMM writes bf16 scores and its
 * softmax writes bf16 probabilities). */
void orc_verify_attention(const uint16_t *q, const uint16_t *k_cache, const uint16_t *v_cache,
                          const uint16_t *k_new, const uint16_t *v_new, const int32_t *slots,
                          const int32_t *positions, int requests, int tokens, int query_heads,
                          int kv_heads, int dimension, int capacity, int window,
                          int round_like_reference, uint16_t *out) {
  const int group = query_heads / kv_heads;
#pragma omp parallel for collapse(3) schedule(dynamic)
  for (int r = 0; r < requests; ++r) {
    for (int t = 0; t < tokens; ++t) {
      for (int h = 0; h < query_heads; ++h) {
        const int kvh = h / group;
        const int p = positions[r];
        const int qpos = p + t;
        int lo = window > 0 ? qpos - window + 1 : 0;
        if (lo < 0) lo = 0;
        const int count = qpos - lo + 1;
        const uint16_t *qv = q + (((int64_t)r * tokens + t) * query_heads + h) * dimension;
        float *scores = (float *)malloc(sizeof(float) * (size_t)count);
        const uint16_t **vrows = (const uint16_t **)malloc(sizeof(void *) * (size_t)count);
        float maximum = -INFINITY;
        for (int i = 0; i < count; ++i) {
          const int j = lo + i;
          const uint16_t *krow, *vrow;
          if (j >= p) {
            const int u = j - p;
            krow = k_new + (((int64_t)r * tokens + u) * kv_heads + kvh) * dimension;
            vrow = v_new + (((int64_t)r * tokens + u) * kv_heads + kvh) * dimension;
          } else {
            const int64_t base =
                (((int64_t)slots[r] * kv_heads + kvh) * capacity + (j % capacity)) * dimension;
            krow = k_cache + base;
            vrow = v_cache + base;
          }
          float s = 0.0f;
          for (int d = 0; d < dimension; ++d) s += orc_bf16_to_f32(qv[d]) * orc_bf16_to_f32(krow[d]);
          if (round_like_reference) s = bf(s);
          scores[i] = s;
          vrows[i] = vrow;
          if (s > maximum) maximum = s;
        }
        float sum = 0.0f;
        for (int i = 0; i < count; ++i) sum += expf(scores[i] - maximum);
        const float inverse_sum = 1.0f / sum;
        for (int i = 0; i < count; ++i) {
          float prob = expf(scores[i] - maximum) * inverse_sum;
          if (round_like_reference) prob = bf(prob);
          scores[i] = prob;
        }
        uint16_t *o = out + (((int64_t)r * tokens + t) * query_heads + h) * dimension;
        for (int d = 0; d < dimension; ++d) {
          float acc = 0.0f;
          for (int i = 0; i < count; ++i) acc += scores[i] * orc_bf16_to_f32(vrows[i][d]);
          o[d] = orc_f32_to_bf16(acc);
        }
        free(scores);
        free(vrows);
      }
    }
  }
}

/* Global attention over an e4m3 K/V cache with per-tensor scales: the dequantised values are
 * e4m3(k) * k_scale. There is no reference verify counterpart (the reference's fp8 global KV is
 * decode-only, gemm_attention.h:40-55); semantics otherwise equal orc_verify_attention with
 * window 0, fp32 math. */
void orc_verify_attention_fp8(const uint16_t *q, const uint8_t *k_cache, const uint8_t *v_cache,
                              const uint8_t *k_new, const uint8_t *v_new, float k_scale,
                              float v_scale, const int32_t *slots, const int32_t *positions,
                              int requests, int tokens, int query_heads, int kv_heads,
                              int dimension, int capacity, uint16_t *out) {
  const int group = query_heads / kv_heads;
  float table[256];
  for (int i = 0; i < 256; ++i) table[i] = orc_e4m3_to_f32((uint8_t)i);
#pragma omp parallel for collapse(3) schedule(dynamic)
  for (int r = 0; r < requests; ++r) {
    for (int t = 0; t < tokens; ++t) {
      for (int h = 0; h < query_heads; ++h) {
        const int kvh = h / group;
        const int p = positions[r];
        const int count = p + t + 1;
        const uint16_t *qv = q + (((int64_t)r * tokens + t) * query_heads + h) * dimension;
        float *scores = (float *)malloc(sizeof(float) * (size_t)count);
        float maximum = -INFINITY;
        for (int j = 0; j < count; ++j) {
          const uint8_t *krow =
              j >= p ? k_new + (((int64_t)r * tokens + (j - p)) * kv_heads + kvh) * dimension
                     : k_cache + (((int64_t)slots[r] * kv_heads + kvh) * capacity + j) * dimension;
          float s = 0.0f;
          for (int d = 0; d < dimension; ++d) s += orc_bf16_to_f32(qv[d]) * table[krow[d]];
          s *= k_scale;
          scores[j] = s;
          if (s > maximum) maximum = s;
        }
        float sum = 0.0f;
        for (int j = 0; j < count; ++j) sum += expf(scores[j] - maximum);
        for (int j = 0; j < count; ++j) scores[j] = expf(scores[j] - maximum) / sum;
        uint16_t *o = out + (((int64_t)r * tokens + t) * query_heads + h) * dimension;
        for (int d = 0; d < dimension; ++d) {
          float acc = 0.0f;
          for (int j = 0; j < count; ++j) {
            const uint8_t *vrow =
                j >= p ? v_new + (((int64_t)r * tokens + (j - p)) * kv_heads + kvh) * dimension
                       : v_cache + (((int64_t)slots[r] * kv_heads + kvh) * capacity + j) * dimension;
            acc += scores[j] * table[vrow[d]];
          }
          o[d] = orc_f32_to_bf16(acc * v_scale);
        }
        free(scores);
      }
    }
  }
}

/* The reference's ring formulation (prefill_gemm_attention.cu:126-298, checked by
 * cuda_ops_tests.cu:1630-1779): all C physical rows of the ring are in the softmax; the ring
 * holds proposal u at (p+u)%C; for query t the rows of proposals u > t are replaced by the
 * backup rows. fp32 math, head-major q/out. Kept as an independent formulation to pin
 * orc_verify_attention's window arithmetic. */
void orc_ring_backup_attention(const uint16_t *q_head_major, const uint16_t *k_ring,
                               const uint16_t *v_ring, const uint16_t *k_backup,
                               const uint16_t *v_backup, const int32_t *positions, int requests,
                               int tokens, int query_heads, int kv_heads, int dimension,
                               int capacity, float *out_head_major) {
  const int group = query_heads / kv_heads;
  for (int r = 0; r < requests; ++r) {
    for (int h = 0; h < query_heads; ++h) {
      const int kvh = h / group;
      for (int t = 0; t < tokens; ++t) {
        float *scores = (float *)malloc(sizeof(float) * (size_t)capacity);
        float maximum = -INFINITY;
        const uint16_t *qv = q_head_major + (((int64_t)r * query_heads + h) * tokens + t) * dimension;
        for (int phys = 0; phys < capacity; ++phys) {
          int backup = -1;
          for (int u = t + 1; u < tokens; ++u)
            if ((positions[r] + u) % capacity == phys) backup = u;
          const uint16_t *krow =
              backup >= 0 ? k_backup + (((int64_t)r * kv_heads + kvh) * tokens + backup) * dimension
                          : k_ring + (((int64_t)r * kv_heads + kvh) * capacity + phys) * dimension;
          float s = 0.0f;
          for (int d = 0; d < dimension; ++d) s += orc_bf16_to_f32(qv[d]) * orc_bf16_to_f32(krow[d]);
          scores[phys] = s;
          if (s > maximum) maximum = s;
        }
        float denominator = 0.0f;
        for (int phys = 0; phys < capacity; ++phys) {
          scores[phys] = expf(scores[phys] - maximum);
          denominator += scores[phys];
        }
        for (int d = 0; d < dimension; ++d) {
          float acc = 0.0f;
          for (int phys = 0; phys < capacity; ++phys) {
            int backup = -1;
            for (int u = t + 1; u < tokens; ++u)
              if ((positions[r] + u) % capacity == phys) backup = u;
            const uint16_t *vrow =
                backup >= 0
                    ? v_backup + (((int64_t)r * kv_heads + kvh) * tokens + backup) * dimension
                    : v_ring + (((int64_t)r * kv_heads + kvh) * capacity + phys) * dimension;
            acc += scores[phys] / denominator * orc_bf16_to_f32(vrow[d]);
          }
          out_head_major[(((int64_t)r * query_heads + h) * tokens + t) * dimension + d] = acc;
        }
        free(scores);
      }
    }
  }
}

/* gemm_attention.cu:88-132 (softmax over valid = min(position + 1, C) physical rows, ring order
 * irrelevant) and :618-676 (per-slot K/V, no scaling). q [B][Hq][D], out [B][Hq][D]. */
void orc_decode_attention(const uint16_t *q, const uint16_t *k_cache, const uint16_t *v_cache,
                          const int32_t *slots, const int32_t *positions, int batch,
                          int query_heads, int kv_heads, int dimension, int capacity,
                          int round_like_reference, uint16_t *out) {
  const int group = query_heads / kv_heads;
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (int b = 0; b < batch; ++b) {
    for (int h = 0; h < query_heads; ++h) {
      const int kvh = h / group;
      int valid = positions[b] + 1;
      if (valid > capacity) valid = capacity;
      const uint16_t *qv = q + ((int64_t)b * query_heads + h) * dimension;
      const int64_t head_base = ((int64_t)slots[b] * kv_heads + kvh) * capacity;
      float *scores = (float *)malloc(sizeof(float) * (size_t)valid);
      float maximum = -INFINITY;
      for (int j = 0; j < valid; ++j) {
        const uint16_t *krow = k_cache + (head_base + j) * dimension;
        float s = 0.0f;
        for (int d = 0; d < dimension; ++d) s += orc_bf16_to_f32(qv[d]) * orc_bf16_to_f32(krow[d]);
        if (round_like_reference) s = bf(s);
        scores[j] = s;
        if (s > maximum) maximum = s;
      }
      float sum = 0.0f;
      for (int j = 0; j < valid; ++j) sum += expf(scores[j] - maximum);
      const float inverse_sum = 1.0f / sum;
      for (int j = 0; j < valid; ++j) {
        float prob = expf(scores[j] - maximum) * inverse_sum;
        if (round_like_reference) prob = bf(prob);
        scores[j] = prob;
      }
      for (int d = 0; d < dimension; ++d) {
        float acc = 0.0f;
        for (int j = 0; j < valid; ++j)
          acc += scores[j] * orc_bf16_to_f32(v_cache[(head_base + j) * dimension + d]);
        out[((int64_t)b * query_heads + h) * dimension + d] = orc_f32_to_bf16(acc);
      }
      free(scores);
    }
  }
}

/* Net effect of backup_kv_ring_spans + proposal write + restore_kv_ring_suffixes
 * (ops.cu:827-871, batch_model_runner.cu:1785-1803): after verification the ring holds the
 * proposals t < accepted[r] at (p+t)%C and its previous contents elsewhere. */
void orc_commit_kv(uint16_t *k_cache, uint16_t *v_cache, const uint16_t *k_new,
                   const uint16_t *v_new, const int32_t *slots, const int32_t *positions,
                   const int32_t *accepted, int requests, int tokens, int kv_heads, int dimension,
                   int capacity) {
  for (int r = 0; r < requests; ++r)
    for (int t = 0; t < accepted[r] && t < tokens; ++t)
      for (int h = 0; h < kv_heads; ++h) {
        const int64_t dst =
            (((int64_t)slots[r] * kv_heads + h) * capacity + (positions[r] + t) % capacity) *
            dimension;
        const int64_t src = (((int64_t)r * tokens + t) * kv_heads + h) * dimension;
        memcpy(k_cache + dst, k_new + src, sizeof(uint16_t) * (size_t)dimension);
        memcpy(v_cache + dst, v_new + src, sizeof(uint16_t) * (size_t)dimension);
      }
}
