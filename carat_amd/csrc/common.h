// Shared device/host helpers for the carat MI355X (gfx950) verify-path kernels.
//
// Storage types: bf16 is carried as uint16_t bit patterns, OCP e4m3 as uint8_t. All arithmetic is
// fp32. Conversions round to nearest even exactly like the reference's __float2bfloat16_rn and
// __nv_fp8_e4m3(float) (saturating to +-448).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>

namespace carat_hip {

using bf16_t = uint16_t;
using fp8_t = uint8_t;

constexpr int kWave = 64;

typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

inline void hip_check(hipError_t result, const char *operation) {
  if (result != hipSuccess)
    throw std::runtime_error(std::string(operation) + ": " + hipGetErrorString(result));
}

// A striped amax has 1 .. kWave floats (one per lane of the reading wave).
inline void check_amax_stripes(int stripes) {
  if (stripes < 1 || stripes > kWave) throw std::runtime_error("amax stripes must be 1 .. 64");
}

// ---------------------------------------------------------------------------------------------
// conversions
// ---------------------------------------------------------------------------------------------

__device__ __forceinline__ float bf16_to_f32(bf16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Round to nearest even with quiet NaNs (a NaN keeps its upper payload and gains the quiet bit):
// gfx950's v_cvt_pk_bf16_f32, which equals that rule bit for bit on every one of the 2^32 inputs
// (checked exhaustively on MI355X).
__device__ __forceinline__ bf16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(bf16_t, static_cast<__bf16>(f));
}

// Two values -> packed bf16 pair (a in the low half), one conversion instruction.
__device__ __forceinline__ uint32_t f32x2_to_bf16x2(float a, float b) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{a, b}), bf16x2));
}

__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// Rounds a pair of values to bf16 precision in place (one conversion for both).
__device__ __forceinline__ void round_bf16x2(float &a, float &b) {
  const uint32_t packed = f32x2_to_bf16x2(a, b);
  a = __uint_as_float(packed << 16);
  b = __uint_as_float(packed & 0xffff0000u);
}

// Two fp32 values -> two e4m3 bytes (low 16 bits of the result), RNE with saturation. The
// hardware conversion rounds to nearest even; the clamp provides the saturating behaviour.
__device__ __forceinline__ uint32_t f32x2_to_e4m3x2(float a, float b) {
  a = fminf(fmaxf(a, -448.0f), 448.0f);
  b = fminf(fmaxf(b, -448.0f), 448.0f);
  return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false)) & 0xffffu;
}

// Four fp32 -> four e4m3 bytes packed little-endian into one dword.
__device__ __forceinline__ uint32_t f32x4_to_e4m3x4(float a, float b, float c, float d) {
  a = fminf(fmaxf(a, -448.0f), 448.0f);
  b = fminf(fmaxf(b, -448.0f), 448.0f);
  c = fminf(fmaxf(c, -448.0f), 448.0f);
  d = fminf(fmaxf(d, -448.0f), 448.0f);
  int packed = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  packed = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, packed, true);
  return static_cast<uint32_t>(packed);
}

__device__ __forceinline__ float e4m3_to_f32(uint32_t byte) {
  return __builtin_amdgcn_cvt_f32_fp8(static_cast<int>(byte), 0);
}

// Per-tensor activation scale from an amax, cuda/linear.cu:107,143 (multiplier 1).
__device__ __forceinline__ float fp8_scale_from_amax(float amax) {
  return amax > 0.0f ? amax / 448.0f : 1.0f;
}

// ---------------------------------------------------------------------------------------------
// wave / block reductions (wave64)
// ---------------------------------------------------------------------------------------------

// Wave64 reductions on the DPP network (VALU lane moves, no LDS round trip per step): butterflies
// inside each quad and row of 16 lanes, then the row totals are carried up with row broadcasts
// into lane 63, whose value every lane receives. DPP controls (GFX9): quad_perm(1,0,3,2) = 0xB1,
// quad_perm(2,3,0,1) = 0x4E, row_half_mirror = 0x141, row_mirror = 0x140, row_bcast15 = 0x142,
// row_bcast31 = 0x143.
template <int kCtrl, int kRowMask = 0xF>
__device__ __forceinline__ float dpp_move(float old, float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old),
                                                              __builtin_bit_cast(int, v), kCtrl,
                                                              kRowMask, 0xF, false));
}

__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_move<0xB1>(0.0f, v);
  v += dpp_move<0x4E>(0.0f, v);
  v += dpp_move<0x141>(0.0f, v);
  v += dpp_move<0x140>(0.0f, v);       // every lane: its row's sum
  v += dpp_move<0x142, 0xA>(0.0f, v);  // rows 1, 3 += rows 0, 2
  v += dpp_move<0x143, 0xC>(0.0f, v);  // row 3 += rows 0 + 1
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_move<0xB1>(v, v));
  v = fmaxf(v, dpp_move<0x4E>(v, v));
  v = fmaxf(v, dpp_move<0x141>(v, v));
  v = fmaxf(v, dpp_move<0x140>(v, v));
  v = fmaxf(v, dpp_move<0x142, 0xA>(v, v));
  v = fmaxf(v, dpp_move<0x143, 0xC>(v, v));
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// RMSNorm's 1 / sqrt(mean square + eps) (cuda/ops.cu:27-85).
__device__ __forceinline__ float inverse_rms(float square_sum, int width, float eps) {
  return rsqrtf(square_sum / static_cast<float>(width) + eps);
}

// Block-wide sum; `scratch` needs blockDim.x / 64 floats. All threads get the result.
__device__ __forceinline__ float block_sum(float v, float *scratch) {
  v = wave_sum(v);
  const int wave = threadIdx.x / kWave;
  const int waves = blockDim.x / kWave;
  __syncthreads();
  if ((threadIdx.x & (kWave - 1)) == 0) scratch[wave] = v;
  __syncthreads();
  float total = 0.0f;
  for (int w = 0; w < waves; ++w) total += scratch[w];
  return total;
}

__device__ __forceinline__ float block_max(float v, float *scratch) {
  v = wave_max(v);
  const int wave = threadIdx.x / kWave;
  const int waves = blockDim.x / kWave;
  __syncthreads();
  if ((threadIdx.x & (kWave - 1)) == 0) scratch[wave] = v;
  __syncthreads();
  float total = scratch[0];
  for (int w = 1; w < waves; ++w) total = fmaxf(total, scratch[w]);
  return total;
}

// Float amax accumulated with an integer atomic max on the bit pattern (valid for values >= 0).
__device__ __forceinline__ void atomic_max_nonneg(float *address, float value) {
  atomicMax(reinterpret_cast<unsigned int *>(address), __float_as_uint(value));
}

// Per-tensor amax held as `stripes` floats, each updated with atomic max: thousands of waves that
// finish together would otherwise serialise on one address (~10-20 ns per atomic). Stripes sit
// kAmaxStripeFloats floats (256 bytes) apart, each on its own cache line, since atomics to one
// line serialise as well. The value is the max over the stripes. `stripes` = 1 is the plain
// single-float form (one float of storage).
constexpr int kAmaxStripeFloats = 64;
constexpr int kMaxAmaxStripes = kWave;
__device__ __forceinline__ void amax_publish(float *amax, int stripes, float value) {
  const unsigned stripe =
      stripes > 1 ? (blockIdx.x * 4u + (threadIdx.x >> 6) + blockIdx.y * 131u + blockIdx.z * 37u) %
                        static_cast<unsigned>(stripes)
                  : 0u;
  atomic_max_nonneg(amax + stripe * kAmaxStripeFloats, value);
}

// Striped amax reads: at most one stripe per lane, so a read is one load per lane, issued
// wherever the caller likes, and one wave reduction where the value is needed.
__device__ __forceinline__ float amax_lane(const float *amax, int stripes) {
  const int i = threadIdx.x & (kWave - 1);
  return i < stripes ? amax[i * kAmaxStripeFloats] : 0.0f;
}
// Wave-cooperative read of a striped amax (every lane of the wave must call it).
__device__ __forceinline__ float amax_read(const float *amax, int stripes) {
  return wave_max(amax_lane(amax, stripes));
}

// Grid-wide agreement on a per-tensor amax among co-resident workgroups (the fused activation
// quantisations). One wave per workgroup calls it, every lane, with the workgroup's amax: the
// workgroup publishes its amax on a stripe (a returning atomic, complete before the arrival),
// then arrives on one of eight arrival counters (workgroup index mod 8, one per XCD under the
// round-robin dispatch); the last arrival of each counter arrives on the global counter, and the
// last of those reads every stripe and releases the tensor's amax (bit 31 set) in the release
// word, which the others poll. Arrivals on one address serialise, so the two-level count keeps
// the chain short (measured on MI355X, one-shot kernels: +1.5 us at 120 workgroups and +1.8 us
// at 224, against +2.0 and +3.3 us with a single counter; measured with relaxed atomics). The
// only values exchanged are these agent-scope atomics; the memory-model order comes from the
// arrivals (acquire-release: each carries its workgroup's stripe update to the last arrival of
// its counter and on to the global last arrival), so it does not rest on how the hardware
// happens to order relaxed read-modify-writes to different addresses. The released amax travels
// in the release word itself (relaxed write and polls: one location). Measured in the verify
// step (MI355X, same runners): this order +0.20 ms per verify over the separate quantisation
// kernel; with an acquire on every poll and a release on the word +0.51 ms; all relaxed +0.09 ms. `sync` holds kFusedSyncWords words kAmaxStripeFloats floats apart
// (global counter, release word, eight counters), zeroed beforehand; `workgroups` is the number
// that arrive. A wait past `spins` polls (kFusedQuantizeSpins in production, far beyond any real
// wait) sets *fault (the result is then not to be used) and returns. The arriving workgroups must be resident at once, or the early ones wait
// for the bound.
constexpr int kFusedQuantizeSpins = 1 << 17;
constexpr int kFusedSyncWords = 10;
__device__ __forceinline__ float fused_amax_release(float *amax, int stripes, unsigned *sync,
                                                    int32_t *fault, unsigned workgroups,
                                                    float workgroup_amax,
                                                    int spins = kFusedQuantizeSpins) {
  const int lane = threadIdx.x & (kWave - 1);
  unsigned *release = sync + kAmaxStripeFloats;
  const unsigned flat = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
  int last = 0;
  if (lane == 0) {
    unsigned *stripe = reinterpret_cast<unsigned *>(amax) + (flat % stripes) * kAmaxStripeFloats;
    const unsigned before = __hip_atomic_fetch_max(stripe, __float_as_uint(workgroup_amax),
                                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __asm__ volatile("s_waitcnt vmcnt(0)" ::"v"(before) : "memory");
    const unsigned group = flat % 8u;
    const unsigned group_size = (workgroups - group + 7u) / 8u;  // workgroups of this counter
    const unsigned groups = workgroups < 8u ? workgroups : 8u;
    const unsigned arrived = __hip_atomic_fetch_add(sync + (2 + group) * kAmaxStripeFloats, 1u,
                                                    __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    if (arrived + 1 == group_size)
      last = __hip_atomic_fetch_add(sync, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) + 1 == groups;
  }
  last = __shfl(last, 0, kWave);
  if (last) {
    const unsigned bits =
        lane < stripes ? __hip_atomic_fetch_max(reinterpret_cast<unsigned *>(amax) + lane * kAmaxStripeFloats,
                                                0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                       : 0u;
    const float total = wave_max(__uint_as_float(bits));
    // The waiting workgroups use only the value of the release word itself, so writing and
    // polling it needs no ordering beyond the word's own coherence.
    if (lane == 0)
      (void)__hip_atomic_exchange(release, __float_as_uint(total) | 0x80000000u, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
    return total;
  }
  unsigned seen = 0;
  if (lane == 0) {
    for (int spin = 0; spin < spins; ++spin) {
      seen = __hip_atomic_fetch_or(release, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (seen & 0x80000000u) break;
      __builtin_amdgcn_s_sleep(2);
    }
    if (!(seen & 0x80000000u))
      (void)__hip_atomic_fetch_or(fault, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  return __uint_as_float(__shfl(static_cast<int>(seen & 0x7fffffffu), 0, kWave));
}

// ---------------------------------------------------------------------------------------------
// argmax keys: an order-preserving 64-bit key (value bits << 32 | ~index) so that an unsigned
// max picks the largest value and, among equal values, the LOWEST index -- the tie rule of the
// reference's `better` (cuda/ops.cu:895-898). NaN maps below every other key (never wins), -0 is
// folded onto +0 so the two compare equal, and the initial key is (-inf, index 0): an element
// equal to -inf can then never displace it, exactly like the reference's (-inf, 0) start value.
// ---------------------------------------------------------------------------------------------

__host__ __device__ __forceinline__ uint32_t orderable_float_bits(float value) {
  uint32_t u;
  __builtin_memcpy(&u, &value, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0u;  // NaN: below everything
  if (u == 0x80000000u) u = 0u;                     // -0 == +0
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__host__ __device__ __forceinline__ uint64_t argmax_key(float value, uint32_t index) {
  return (static_cast<uint64_t>(orderable_float_bits(value)) << 32) |
         static_cast<uint64_t>(0xffffffffu - index);
}

__host__ __device__ __forceinline__ uint32_t argmax_key_index(uint64_t key) {
  return 0xffffffffu - static_cast<uint32_t>(key & 0xffffffffu);
}

// (-inf, 0): orderable(-inf) = ~0xff800000 = 0x007fffff.
constexpr uint64_t kArgmaxInitialKey = (static_cast<uint64_t>(0x007fffffu) << 32) | 0xffffffffull;

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) {
    const uint64_t other = __shfl_xor(v, offset, kWave);
    v = other > v ? other : v;
  }
  return v;
}

// vmcnt-only wait (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14]).
template <int N> __device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// lgkmcnt-only wait: this wave's LDS operations have completed (vmcnt and expcnt left open).
__device__ __forceinline__ void wait_lgkmcnt0() {
  __builtin_amdgcn_s_waitcnt(0xF | (0x3 << 14) | (0x7 << 4));
}

}  // namespace carat_hip
