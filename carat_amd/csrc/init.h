// Seeded synthetic weights / caches and RoPE tables.
#pragma once

#include "common.h"

#include <cstring>
#include <vector>

namespace carat_hip {

void fill_normal_bf16(bf16_t *out, size_t n, uint64_t seed, float mean, float stddev,
                      hipStream_t stream);
// bf16 N(0, stddev) weight quantised per tensor to e4m3; writes the weight scale to *scale_out.
void fill_fp8_weight(fp8_t *out, size_t n, uint64_t seed, float stddev, float *scale_out,
                     float *amax_scratch, hipStream_t stream);
void quantize_weight_bf16_to_fp8(const bf16_t *in, fp8_t *out, size_t n, float *scale_out,
                                 float *amax_scratch, hipStream_t stream);
// Fp8Scaling (include/carat/linear.h:27): 0 tensor, 1 channel, 2 block_128. Scale floats of an
// [n][k] weight: 1, n, or ceil(n/128) x kbp (kbp = ceil(k/128) rounded up to 4; padding 0) as
// Fp8WeightArena lays them out (device_weights.cu:222-229, linear.cu:403-409).
size_t fp8_weight_scale_elements(int scaling, int n, int k);
// Fp8WeightArena::quantize of one [n][k] bf16 segment (device_weights.cu:240-256) into row-major
// e4m3 and its scales (layout above).
void quantize_weight_bf16_to_fp8_scaled(const bf16_t *in, fp8_t *out, int n, int k, int scaling,
                                        float *scales, float *amax_scratch, hipStream_t stream);
void rope_table(int dimension, bool proportional, int positions, std::vector<bf16_t> &cosine,
                std::vector<bf16_t> &sine);

}  // namespace carat_hip
