// Seeded synthetic weights / caches generated on the device (no host staging of ~30 GB), and the
// RoPE tables.
//
// Values: splitmix64(seed, index) -> two uniforms -> Box-Muller normal. fp8 weights follow the
// reference's per-tensor weight quantisation (Fp8WeightArena::quantize, cuda/device_weights.cu:
// 200-263): the bf16 weight w is generated, s = amax(|w|) / 448, q = e4m3(w * (1 / s)).
#include "init.h"

#include <cmath>
#include <vector>

namespace carat_hip {
namespace {

__host__ __device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
  x += 0x9e3779b97f4a7c15ull;
  x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
  x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
  return x ^ (x >> 31);
}

__device__ __forceinline__ float normal_at(uint64_t seed, uint64_t index) {
  const uint64_t bits = splitmix64(seed * 0x632be59bd9b4e019ull + index);
  const float u1 = (static_cast<float>(bits >> 40) + 1.0f) * (1.0f / 16777217.0f);  // (0, 1]
  const float u2 = static_cast<float>((bits >> 16) & 0xffffffull) * (1.0f / 16777216.0f);
  return sqrtf(-2.0f * logf(u1)) * cospif(2.0f * u2);
}

__global__ void fill_normal_bf16_kernel(bf16_t *out, size_t n, uint64_t seed, float mean,
                                        float stddev) {
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * blockDim.x)
    out[i] = f32_to_bf16(mean + stddev * normal_at(seed, i));
}

__global__ void weight_amax_kernel(size_t n, uint64_t seed, float stddev, float *amax) {
  float m = 0.0f;
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * blockDim.x)
    m = fmaxf(m, fabsf(round_bf16(stddev * normal_at(seed, i))));
  m = wave_max(m);
  if ((threadIdx.x & 63) == 0) atomic_max_nonneg(amax, m);
}

__global__ void weight_quantize_kernel(fp8_t *out, size_t n, uint64_t seed, float stddev,
                                       const float *amax, float *scale_out) {
  const float scale = *amax > 0.0f ? *amax / 448.0f : 1.0f;
  const float inverse = 1.0f / scale;
  if (blockIdx.x == 0 && threadIdx.x == 0) *scale_out = scale;
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const float w = round_bf16(stddev * normal_at(seed, i));
    out[i] = static_cast<fp8_t>(f32x2_to_e4m3x2(w * inverse, 0.0f) & 0xffu);
  }
}

__global__ void bf16_to_fp8_weight_kernel(const bf16_t *in, fp8_t *out, size_t n,
                                          const float *amax, float *scale_out) {
  const float scale = *amax > 0.0f ? *amax / 448.0f : 1.0f;
  const float inverse = 1.0f / scale;
  if (blockIdx.x == 0 && threadIdx.x == 0) *scale_out = scale;
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * blockDim.x)
    out[i] = static_cast<fp8_t>(f32x2_to_e4m3x2(bf16_to_f32(in[i]) * inverse, 0.0f) & 0xffu);
}

__global__ void bf16_amax_kernel(const bf16_t *in, size_t n, float *amax) {
  float m = 0.0f;
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * blockDim.x)
    m = fmaxf(m, fabsf(bf16_to_f32(in[i])));
  m = wave_max(m);
  if ((threadIdx.x & 63) == 0) atomic_max_nonneg(amax, m);
}

// Fp8Scaling::channel / ::block_128 weights (quantize_bf16_rows_kernel and
// quantize_weight_block_128_kernel, cuda/linear.cu:300-316, 352-380): one workgroup per row, or
// per 128 x 128 block; scale = max(amax / 448, 2^-24), q = e4m3(w / scale) (a true division, as
// the reference's).
__device__ __forceinline__ float block_max_256(float m) {
  __shared__ float wave_maxima[4];
  m = wave_max(m);
  if ((threadIdx.x & 63) == 0) wave_maxima[threadIdx.x >> 6] = m;
  __syncthreads();
  return fmaxf(fmaxf(wave_maxima[0], wave_maxima[1]), fmaxf(wave_maxima[2], wave_maxima[3]));
}

__global__ __launch_bounds__(256) void quantize_rows_kernel(const bf16_t *in, fp8_t *out, int k,
                                                            float *scales) {
  const size_t row = blockIdx.x;
  const bf16_t *src = in + row * k;
  float m = 0.0f;
  for (int c = threadIdx.x; c < k; c += 256) m = fmaxf(m, fabsf(bf16_to_f32(src[c])));
  const float scale = fmaxf(block_max_256(m) / 448.0f, 0x1p-24f);
  if (threadIdx.x == 0) scales[row] = scale;
  for (int c = threadIdx.x; c < k; c += 256)
    out[row * k + c] = static_cast<fp8_t>(f32x2_to_e4m3x2(bf16_to_f32(src[c]) / scale, 0.0f) & 0xffu);
}

__global__ __launch_bounds__(256) void quantize_block128_kernel(const bf16_t *in, fp8_t *out, int n,
                                                                int k, int kbp, float *scales) {
  const int kb = blockIdx.x, nb = blockIdx.y;
  const int c = kb * 128 + (threadIdx.x & 127);
  const int r0 = nb * 128 + (threadIdx.x >> 7);
  float m = 0.0f;
  for (int r = r0; r < min(n, nb * 128 + 128); r += 2)
    if (c < k) m = fmaxf(m, fabsf(bf16_to_f32(in[static_cast<size_t>(r) * k + c])));
  const float scale = fmaxf(block_max_256(m) / 448.0f, 0x1p-24f);
  if (threadIdx.x == 0) scales[static_cast<size_t>(nb) * kbp + kb] = scale;
  for (int r = r0; r < min(n, nb * 128 + 128); r += 2)
    if (c < k) {
      const size_t i = static_cast<size_t>(r) * k + c;
      out[i] = static_cast<fp8_t>(f32x2_to_e4m3x2(bf16_to_f32(in[i]) / scale, 0.0f) & 0xffu);
    }
}

__global__ void zero_f32_kernel(float *p) { *p = 0.0f; }

unsigned grid_for(size_t n) {
  const size_t blocks = (n + 255) / 256;
  return static_cast<unsigned>(blocks < 8192 ? (blocks == 0 ? 1 : blocks) : 8192);
}

}  // namespace

void fill_normal_bf16(bf16_t *out, size_t n, uint64_t seed, float mean, float stddev,
                      hipStream_t stream) {
  fill_normal_bf16_kernel<<<grid_for(n), 256, 0, stream>>>(out, n, seed, mean, stddev);
  hip_check(hipGetLastError(), "launch normal fill");
}

void fill_fp8_weight(fp8_t *out, size_t n, uint64_t seed, float stddev, float *scale_out,
                     float *amax_scratch, hipStream_t stream) {
  zero_f32_kernel<<<1, 1, 0, stream>>>(amax_scratch);
  weight_amax_kernel<<<grid_for(n), 256, 0, stream>>>(n, seed, stddev, amax_scratch);
  weight_quantize_kernel<<<grid_for(n), 256, 0, stream>>>(out, n, seed, stddev, amax_scratch,
                                                         scale_out);
  hip_check(hipGetLastError(), "launch fp8 weight fill");
}

void quantize_weight_bf16_to_fp8(const bf16_t *in, fp8_t *out, size_t n, float *scale_out,
                                 float *amax_scratch, hipStream_t stream) {
  zero_f32_kernel<<<1, 1, 0, stream>>>(amax_scratch);
  bf16_amax_kernel<<<grid_for(n), 256, 0, stream>>>(in, n, amax_scratch);
  bf16_to_fp8_weight_kernel<<<grid_for(n), 256, 0, stream>>>(in, out, n, amax_scratch, scale_out);
  hip_check(hipGetLastError(), "launch weight quantisation");
}

size_t fp8_weight_scale_elements(int scaling, int n, int k) {
  if (scaling == 0) return 1;
  if (scaling == 1) return static_cast<size_t>(n);
  if (scaling == 2) {
    const size_t kbp = ((static_cast<size_t>(k) + 127) / 128 + 3) & ~static_cast<size_t>(3);
    return kbp * ((static_cast<size_t>(n) + 127) / 128);
  }
  throw std::runtime_error("invalid FP8 scaling");
}

void quantize_weight_bf16_to_fp8_scaled(const bf16_t *in, fp8_t *out, int n, int k, int scaling,
                                        float *scales, float *amax_scratch, hipStream_t stream) {
  if (n <= 0 || k <= 0) throw std::runtime_error("invalid FP8 weight shape");
  if (scaling == 0) {
    quantize_weight_bf16_to_fp8(in, out, static_cast<size_t>(n) * k, scales, amax_scratch, stream);
    return;
  }
  if (scaling == 1) {
    quantize_rows_kernel<<<n, 256, 0, stream>>>(in, out, k, scales);
  } else if (scaling == 2) {
    const int kb = (k + 127) / 128;
    const int kbp = (kb + 3) & ~3;
    hip_check(hipMemsetAsync(scales, 0, sizeof(float) * fp8_weight_scale_elements(2, n, k), stream),
              "clear FP8 block weight scales");
    quantize_block128_kernel<<<dim3(kb, (n + 127) / 128), 256, 0, stream>>>(in, out, n, k, kbp,
                                                                           scales);
  } else {
    throw std::runtime_error("invalid FP8 scaling");
  }
  hip_check(hipGetLastError(), "launch scaled weight quantisation");
}

// cuda/qkv.cu:44-64: sliding tables use theta 1e4 over all D/2 frequencies; the global
// ("proportional") tables use theta 1e6 and rotate only the first D/8 half-indices. The angle is
// the fp32 product position * fp32 frequency; sin/cos are evaluated in double and rounded to bf16.
void rope_table(int dimension, bool proportional, int positions, std::vector<bf16_t> &cosine,
                std::vector<bf16_t> &sine) {
  cosine.assign(static_cast<size_t>(positions) * dimension, 0);
  sine.assign(static_cast<size_t>(positions) * dimension, 0);
  auto to_bf16 = [](float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<bf16_t>(u >> 16);
  };
  std::vector<float> frequency(static_cast<size_t>(dimension / 2));
  for (int i = 0; i < dimension / 2; ++i) {
    double f = 0.0;
    if (proportional) {
      if (i < dimension / 8) f = std::pow(1000000.0, -2.0 * i / dimension);
    } else {
      f = std::pow(10000.0, -2.0 * i / dimension);
    }
    frequency[static_cast<size_t>(i)] = static_cast<float>(f);
  }
  for (int p = 0; p < positions; ++p)
    for (int i = 0; i < dimension; ++i) {
      const float angle = static_cast<float>(p) * frequency[static_cast<size_t>(i % (dimension / 2))];
      cosine[static_cast<size_t>(p) * dimension + i] = to_bf16(static_cast<float>(std::cos(static_cast<double>(angle))));
      sine[static_cast<size_t>(p) * dimension + i] = to_bf16(static_cast<float>(std::sin(static_cast<double>(angle))));
    }
}

}  // namespace carat_hip
