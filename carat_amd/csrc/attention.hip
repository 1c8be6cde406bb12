// Verify / decode attention for gfx950.
//
// One workgroup (4 wave64s) owns one (request, kv head, key chunk). The G*T query rows of a kv head
// (G query heads per kv head, T tokens) form the 16-column B operand of v_mfma_f32_16x16x32_bf16;
// K rows are the A operand, so scores come out as S^T[key][query row] with every lane owning one
// query column -- the online-softmax max/sum reductions are two xor shuffles. P.V uses V^T as the A
// operand: each wave parks its V rows in LDS and reads them back transposed. fp8 K/V are
// dequantised to bf16 in registers (exact: e4m3 is a subset of bf16) and the per-tensor scales are
// folded into the scores and the output.
//
// Semantics (reference): cuda/prefill_gemm_attention.cu:126-349,552-730 (verify; no 1/sqrt(D)
// scaling, sliding window of `capacity` rows) and cuda/gemm_attention.cu:88-132,618-676 (decode).
// The reference materialises bf16 scores and probabilities; this kernel keeps scores in fp32 and
// rounds only the probabilities fed to the P.V MFMA to bf16.
#include "attention.h"

#include <algorithm>
#include <type_traits>

namespace carat_hip {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef short s4_t __attribute__((ext_vector_type(4)));

// Waves per workgroup (stages per wave follow from 64 KiB of LDS per workgroup). Measured on
// MI355X: four waves with two 16-key stages beat two waves with four (sliding verify 48.7 vs
// 61.1 us, global 305 vs 349 us) -- the per-key work of the verify rows needs the waves.
constexpr int kAttentionWaves = 4;
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) { return f32x2_to_bf16x2(lo, hi); }

// e4m3 -> bf16 is exact (bf16 has the wider exponent and mantissa): gfx950 converts a pair of
// e4m3 bytes straight to a bf16 pair (unit scale; checked on MI355X against the float route for
// every code).
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
template <bool kHigh>
__device__ __forceinline__ uint32_t e4m3x2_to_bf16x2(uint32_t word) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(word, 1.0f, kHigh));
}

// 8 e4m3 bytes -> 8 bf16 (exact).
__device__ __forceinline__ u32x4 e4m3x8_to_bf16x8(u32x2 raw) {
  return u32x4{e4m3x2_to_bf16x2<false>(raw.x), e4m3x2_to_bf16x2<true>(raw.x),
               e4m3x2_to_bf16x2<false>(raw.y), e4m3x2_to_bf16x2<true>(raw.y)};
}

// Max / sum over the four lane groups of a column (lanes l, l^16, l^32, l^48) with gfx950's
// cross-row lane swaps: VALU only, no LDS round trip. Each step combines the same two values in
// every lane that holds them (the swap returns them in either order; max and + commute), so the
// result is the one the xor-shuffle reduction gives, bit for bit.
__device__ __forceinline__ float groups_max(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float groups_sum(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

struct KeyRange {
  int lo;
  int hi;  // inclusive
};

__device__ __forceinline__ KeyRange key_range(const AttentionArgs &a, int p) {
  KeyRange range;
  if (a.mode == AttentionMode::decode) {
    range.lo = 0;
    range.hi = min(p + 1, a.capacity) - 1;
  } else if (a.mode == AttentionMode::sliding) {
    range.lo = max(0, p - a.window + 1);
    range.hi = p + a.tokens - 1;
  } else {
    range.lo = 0;
    range.hi = p + a.tokens - 1;
  }
  return range;
}

// Waves per SIMD (= workgroups per CU) the kernel is built for: three where the registers allow
// it (D = 128, one query tile: <= 168 VGPRs), two at D = 128 with two query tiles and at D = 256
// (<= 256 registers; measured on MI355X at 24 x 16 pairs: 88 us against 105 us at one), one at
// D = 512. The LDS and K-prefetch budgets follow from it.
template <int D, int NQ>
constexpr int kAttentionOccupancy = D <= 128 ? (NQ == 1 ? 3 : 2) : D <= 256 ? 2 : 1;

// The QKV post-processing of one (request r, kv head h) inside the attention kernel, with the
// arithmetic of qkv_post_kernel (cuda/qkv.cu:387-530) unit for unit, so the results are the same
// bits: a unit is one (row, head) of the packed projection -- the G query heads of kv head h and
// its K and V heads, for each of the request's T rows -- handled by one wave, lane l owning
// elements 2l, 2l + 1; units go round-robin over the waves. load() issues every load of the
// wave's units (split-K partials, norm weights, RoPE rows, scale operands) and finish() waits for
// them and writes the query rows to `q_tile` ([local_head * T + t][D]), the K/V rows to this
// step's k_new/v_new rows and, when the QKV arguments carry a cache, to the cache row
// (p + t) % capacity. The kernel issues load() before its first K/V stages, so the in-order
// memory counter lets finish() wait for these few loads alone.
constexpr int kFusedQkvMaxTokens = 8;
constexpr int kFusedQkvUnitsPerWave = 8;

// kQueryOnly: the assistant's decode step, whose projection holds only query heads (it reads the
// target's cache): units are the query rows, the RoPE position is p + position_offset + t, bf16
// projections carry no scale operands (scale 1), and the rows also go to q_out (written by the
// first key chunk of the pair) for the stage checks.
template <int D, int S, bool kQueryOnly = false>
struct FusedQkv {
  static constexpr int E = D / 64;
  static constexpr int U = kFusedQkvUnitsPerWave;
  static_assert(E == 2, "two elements per lane");
  float part[U][S][E], wv[U][E], cs[U][E], sn[U][E];
  float amax_part, w_scale;

  __device__ __forceinline__ static uint32_t load_u32(const bf16_t *p) {
    return *reinterpret_cast<const uint32_t *>(p);
  }
  __device__ __forceinline__ static void unpack(uint32_t w, float (&v)[E]) {
    v[0] = __uint_as_float(w << 16);
    v[1] = __uint_as_float(w & 0xffff0000u);
  }

  // unit u: query row (local head u / T, token u % T), then the T K rows, then the T V rows
  __device__ __forceinline__ static void unit(int u, int G, int T, int &kind, int &t) {
    kind = u < G * T ? 0 : 1 + (u - G * T) / T;
    t = u < G * T ? u % T : (u - G * T) % T;
  }
  __device__ __forceinline__ static int unit_count(const QkvArgs &q, int G, int T) {
    return kQueryOnly ? G * T : G * T + (q.key_equals_value ? 1 : 2) * T;
  }

  __device__ __forceinline__ void load(const AttentionArgs &a, int r, int h, int p) {
    const QkvArgs &q = a.qkv;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    const int hq = a.query_heads, hkv = a.kv_heads, G = hq / hkv, T = a.tokens;
    const int query_width = hq * D, kv_width = hkv * D;
    const int packed_width = kQueryOnly ? query_width : query_width + kv_width * (q.key_equals_value ? 1 : 2);
    const int units = unit_count(q, G, T);
    amax_part = q.x_amax != nullptr ? amax_lane(q.x_amax, q.amax_stripes) : 0.0f;
    w_scale = q.w_scale != nullptr ? *q.w_scale : 1.0f;
    // Branch-free: past the last unit a wave re-loads the last one (its values are not used), so
    // no control-flow merge makes the compiler wait for these loads before the K/V stages go out.
#pragma unroll
    for (int i = 0; i < U; ++i) {
      const int u = min(wave + i * waves, units - 1);
      int kind, t;
      unit(u, G, T, kind, t);
      const int column0 = kind == 0 ? (h * G + u / T) * D
                          : kind == 1 ? query_width + h * D
                                      : query_width + kv_width + h * D;
      const int row = r * T + t;
      const int c0 = column0 + lane * E;
#pragma unroll
      for (int k = 0; k < S; ++k) {
        const float2 v = *reinterpret_cast<const float2 *>(
            q.partials + (static_cast<size_t>(k) * q.rows + row) * packed_width + c0);
        part[i][k][0] = v.x;
        part[i][k][1] = v.y;
      }
      const size_t rope = static_cast<size_t>(p + q.position_offset + t) * D + lane * E;
      unpack(load_u32((kind == 1 ? q.k_norm : q.q_norm) + lane * E), wv[i]);
      unpack(load_u32(q.cosine + rope), cs[i]);
      unpack(load_u32(q.sine + rope), sn[i]);
    }
  }

  __device__ __forceinline__ void finish(const AttentionArgs &a, int r, int h, int p, int slot,
                                         bf16_t *q_tile, bool store_q = false) {
    const QkvArgs &q = a.qkv;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    const int hq = a.query_heads, hkv = a.kv_heads, G = hq / hkv, T = a.tokens;
    const int units = unit_count(q, G, T);
    const float scale =
        q.x_amax != nullptr ? w_scale * fp8_scale_from_amax(wave_max(amax_part)) : w_scale;
    // per unit: split-K sum, bf16, RMSNorm (Q, K with weight; V without), RoPE (Q, K). The
    // arithmetic of every unit comes first, branch-free (both the rotated and the plain result),
    // so the units' dependency chains interleave; past the last unit a wave redoes the last one.
    uint32_t roped[U], plain[U];
#pragma unroll
    for (int i = 0; i < U; ++i) {
      float x[E];
      float square_sum = 0.0f;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        float sum = part[i][0][e];
#pragma unroll
        for (int k = 1; k < S; ++k) sum += part[i][k][e];
        x[e] = round_bf16(sum * scale);
        square_sum += x[e] * x[e];
      }
      const float inv = inverse_rms(wave_sum(square_sum), D, q.eps);
      float normalized[E], out[E];
#pragma unroll
      for (int e = 0; e < E; ++e) normalized[e] = round_bf16(x[e] * inv * wv[i][e]);
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const int d = lane * E + e;
        const float partner = __shfl_xor(normalized[e], 32, kWave);
        const float rotated = d < D / 2 ? -partner : partner;
        out[e] = normalized[e] * cs[i][e] + rotated * sn[i][e];
      }
      roped[i] = f32x2_to_bf16x2(out[0], out[1]);
      plain[i] = f32x2_to_bf16x2(x[0] * inv, x[1] * inv);
    }
    // stores: Q rows to the tile, K (RoPE) and V (no weight; K = V: the K head's plain result)
    // rows to this step's rows and the cache
#pragma unroll
    for (int i = 0; i < U; ++i) {
      const int u = wave + i * waves;
      if (u >= units) break;  // wave-uniform
      int kind, t;
      unit(u, G, T, kind, t);
      const int row = r * T + t;
      auto write_kv = [&](bf16_t *new_rows, bf16_t *cache, uint32_t vals) {
        *reinterpret_cast<uint32_t *>(new_rows + (static_cast<size_t>(row) * hkv + h) * D + lane * E) = vals;
        if (cache != nullptr)
          *reinterpret_cast<uint32_t *>(
              cache + ((static_cast<size_t>(slot) * hkv + h) * q.capacity + (p + t) % q.capacity) * D +
              lane * E) = vals;
      };
      if (kind == 0) {
        *reinterpret_cast<uint32_t *>(q_tile + u * D + lane * E) = roped[i];
        if (kQueryOnly && store_q)
          *reinterpret_cast<uint32_t *>(
              q.q_out + (static_cast<size_t>(row) * hq + h * G + u / T) * D + lane * E) = roped[i];
        continue;
      }
      if (kQueryOnly) continue;
      if (kind == 1)
        write_kv(q.k_new, q.k_cache, roped[i]);
      if (kind == 2 || (kind == 1 && q.key_equals_value)) write_kv(q.v_new, q.v_cache, plain[i]);
    }
  }
};

// kFuseSplits > 0: the QKV post-processing of the step over that many split-K partials is fused
// into the prologue (AttentionArgs::fuse_qkv).
template <int D, int NQ, bool kFp8, AttentionMode kMode, int kWaves, int kFuseSplits = 0>
__global__ __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(kAttentionOccupancy<D, NQ>)))
void attention_kernel(const AttentionArgs a) {
  constexpr int kThreads = kWaves * 64;
  // 16 keys per wave iteration. A workgroup stays at 64 KiB of LDS, so two co-reside on a CU and
  // an uneven grid (384 workgroups on 256 CUs) still shares the HBM stream evenly instead of
  // running a second round.
  constexpr int KPI = 16;                  // keys per wave iteration
  constexpr int KT = KPI / 16;             // 16-key tiles per iteration
  constexpr int DS = D / 32;               // QK MFMA steps over D
  constexpr int DT = D / 16;               // PV output tiles over D
  // K/V rows stream HBM -> LDS by DMA (global_load_lds_dwordx4) in their stored format (bf16 or
  // e4m3), into per-wave stages. One wave instruction moves kRowsPerDma whole rows (1 KiB
  // contiguous when the rows are). Inside a row the 16-byte chunks are XOR-swizzled by the row
  // index (chunk c of row k sits at position c ^ (k mod kChunksPerRow)), so the 16 rows that one
  // K-operand read touches at the same chunk land in 16 different bank groups.
  constexpr int kSrcRowBytes = D * (kFp8 ? 1 : 2);
  constexpr int kChunksPerRow = kSrcRowBytes / 16;
  constexpr int kRowsPerDma = 64 / kChunksPerRow;
  constexpr int kDmaPerTensor = KPI / kRowsPerDma;
  constexpr int kStageBytes = KPI * kSrcRowBytes;  // one V stage
  // K rows go straight to VGPRs, already in the A operand layout: for MFMA step s, lane (key c,
  // group g) holds bytes [(4 s + g) w, +w) of its key row, w = 16 (bf16) or 8 (e4m3), so one load
  // instruction covers a contiguous 4w bytes of each of the 16 keys. Only V, which the P.V MFMA
  // needs transposed, is staged in LDS.
  // Stages per wave: V within 48 KiB per workgroup at three workgroups per CU (64 KiB at two,
  // 144 KiB at one) and the prefetched K within 48 (64, 128) VGPRs, at most four (six for e4m3).
  using KRaw = std::conditional_t<kFp8, u32x2, u32x4>;  // one K operand slice as stored
  constexpr int kKRegsPerStage = DS * static_cast<int>(sizeof(KRaw)) / 4;
  constexpr int kOccupancy = kAttentionOccupancy<D, NQ>;
  constexpr int kLdsBudget = kOccupancy == 3 ? 48 * 1024 : kOccupancy == 2 ? 64 * 1024 : 144 * 1024;
  constexpr int kRegBudget = kOccupancy == 3 ? 48 : kOccupancy == 2 ? 64 : 128;
  // At D = 512 the Q operand (64 VGPRs per query tile) lives in LDS instead, read once per MFMA
  // step, so that two K stages fit in the registers.
  constexpr bool kQInLds = D >= 512;
  constexpr int kQBytes = kQInLds ? NQ * DS * 64 * 16 : 0;
  constexpr int kStagesLds = (kLdsBudget - kQBytes) / (kWaves * kStageBytes);
  constexpr int kStagesRegs = kRegBudget / kKRegsPerStage;
  constexpr int kLoadsPerStage = kDmaPerTensor + DS;  // V DMAs + K loads, in issue order
  constexpr int kStagesVm = 63 / kLoadsPerStage + 1;   // the vmcnt wait counts at most 63 loads
  constexpr int kStagesFit0 = kStagesLds < kStagesRegs ? kStagesLds : kStagesRegs;
  constexpr int kStagesFit = kStagesFit0 < kStagesVm ? kStagesFit0 : kStagesVm;
  // e4m3 K/V rows carry half the bytes per stage, so a stage's latency covers less data: six of
  // them fit the same LDS and registers (measured on MI355X, config 3 e4m3: 233 -> 207 us).
  constexpr int kStageCap = kFp8 ? 6 : 4;
  constexpr int kStages = kStagesFit > kStageCap ? kStageCap : (kStagesFit < 1 ? 1 : kStagesFit);
  constexpr int kWaveBytes = kStages * kStageBytes;
  // wave merge: m and l per (wave, query row), then the O rows at a padded stride (no bank
  // conflicts between the rows of one store)
  constexpr int kCoStride = D + 4;
  constexpr int kCombineBytes = (2 * kWaves * NQ * 16 + kWaves * NQ * 16 * kCoStride) * 4;
  constexpr int kLoopBytes = kWaves * kWaveBytes + kQBytes;  // V stages, then Q (kQInLds)
  // the fused QKV post-processing's query rows [16][D] bf16 sit past the stages
  constexpr int kQTileBytes = kFuseSplits > 0 ? 16 * D * 2 : 0;
  constexpr int kLdsBytes = (kLoopBytes > kCombineBytes ? kLoopBytes : kCombineBytes) + kQTileBytes;
  static_assert(KPI % kRowsPerDma == 0 && kRowsPerDma * kChunksPerRow == 64, "DMA row tiling");
  __shared__ __attribute__((aligned(16))) unsigned char lds[kLdsBytes];

  const int lane = threadIdx.x & 63;
  // wave-uniform (SGPR) so the DMA destinations derived from it go straight into M0
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int group = lane >> 4;
  const int col = lane & 15;

  const int G = a.query_heads / a.kv_heads;
  const int T = a.tokens;
  const int qrows = G * T;
  // Workgroup -> (key chunk, kv head, request, query tile). Workgroups go to the 8 XCDs
  // round-robin; the query tiles of one item take consecutive slots of the same XCD, so they run
  // together and read the item's K/V rows through that XCD's L2 once.
  const int qtiles = (qrows + NQ * 16 - 1) / (NQ * 16);
  const int max_chunks = (a.max_keys + a.chunk_keys - 1) / a.chunk_keys;
  const int xcd_slot = static_cast<int>(blockIdx.x) >> 3;
  const int item = (xcd_slot / qtiles) * 8 + (static_cast<int>(blockIdx.x) & 7);
  const int q0 = (xcd_slot % qtiles) * NQ * 16;
  if (item >= max_chunks * a.kv_heads * a.requests) return;
  const int chunk = item % max_chunks;
  const int h = (item / max_chunks) % a.kv_heads;
  const int r = item / (max_chunks * a.kv_heads);
  const int p = a.positions[r];
  const int slot = a.slots[r];
  const KeyRange range = key_range(a, p);
  const int total_keys = range.hi - range.lo + 1;
  if (total_keys <= 0) return;
  // Ring index without a per-key division: every cached key of the range lies in [wrap, wrap+2C).
  const int wrap = kMode == AttentionMode::sliding ? (range.lo / a.capacity) * a.capacity : 0;
  const int n_chunks = (total_keys + a.chunk_keys - 1) / a.chunk_keys;
  if (chunk >= n_chunks) return;
  int chunk_lo = range.lo + chunk * a.chunk_keys;
  int chunk_hi = min(range.hi, chunk_lo + a.chunk_keys - 1);
  if constexpr (kMode != AttentionMode::decode) {
    // Only the keys some row of this query tile sees: a tile inside one head covers tokens
    // [t_lo, t_hi] (deep prefill steps: the causal triangle and the sliding band per tile). A
    // tile without visible keys in this chunk still writes its (empty) partial below.
    const int rows_here = min(NQ * 16, qrows - q0);
    const bool one_head = q0 / T == (q0 + rows_here - 1) / T;
    const int t_lo = one_head ? q0 % T : 0;
    const int t_hi = one_head ? (q0 + rows_here - 1) % T : T - 1;
    chunk_hi = min(chunk_hi, p + t_hi);
    if (kMode == AttentionMode::sliding) chunk_lo = max(chunk_lo, p + t_lo - a.window + 1);
  }

  const unsigned char *kc = static_cast<const unsigned char *>(a.k_cache);
  const unsigned char *vc = static_cast<const unsigned char *>(a.v_cache);
  const unsigned char *kn = static_cast<const unsigned char *>(a.k_new);
  const unsigned char *vn = static_cast<const unsigned char *>(a.v_new);
  // Row indices fit in 31 bits (checked on the host); addresses are formed as integers so the
  // cache/new-row choice is a pair of selects.
  const int cache_head = (slot * a.kv_heads + h) * a.capacity;
  const int new_head = r * T * a.kv_heads + h;  // + (key - p) * kv_heads
  const uint64_t k_cache_base = reinterpret_cast<uint64_t>(kc), v_cache_base = reinterpret_cast<uint64_t>(vc);
  const uint64_t k_new_base = reinterpret_cast<uint64_t>(kn), v_new_base = reinterpret_cast<uint64_t>(vn);

  unsigned char *wave_lds = lds + wave * kWaveBytes;
  const int first = chunk_lo + wave * KPI;
  const int stride = kWaves * KPI;
  const int iterations = first > chunk_hi ? 0 : (chunk_hi - first) / stride + 1;

  // Loads of iteration `it` (clamped to the last one, so the issue is branch-free) into stage
  // `st`: V rows by DMA into the wave's LDS stage, this lane's K slices into kreg[st]. Keys past
  // the chunk re-read its last row; they are masked in the softmax.
  KRaw kreg[kStages][DS];
  auto source_row = [&](int key) {
    const bool fresh = kMode != AttentionMode::decode && key >= p;
    int physical = key - wrap;
    if (kMode == AttentionMode::sliding) physical -= physical >= a.capacity ? a.capacity : 0;
    return fresh ? new_head + (key - p) * a.kv_heads : cache_head + physical;
  };
  auto issue = [&](int it, int st) {
    // (a wave without iterations re-reads a valid row of the chunk; its loads are never used)
    const int kbase = first + max(0, min(it, iterations - 1)) * stride;
    unsigned char *vst = wave_lds + st * kStageBytes;
#pragma unroll
    for (int j = 0; j < kDmaPerTensor; ++j) {
      const int row_local = j * kRowsPerDma + lane / kChunksPerRow;
      const int position = lane % kChunksPerRow;
      const int chunk_index = position ^ (row_local % kChunksPerRow);
      const int key = min(kbase + row_local, chunk_hi);
      const bool fresh = kMode != AttentionMode::decode && key >= p;
      const uint64_t offset = static_cast<uint64_t>(static_cast<uint32_t>(source_row(key))) * kSrcRowBytes +
                              static_cast<uint32_t>(chunk_index * 16);
      __builtin_amdgcn_global_load_lds(
          reinterpret_cast<const void *>((fresh ? v_new_base : v_cache_base) + offset),
          reinterpret_cast<void __attribute__((address_space(3))) *>(
              reinterpret_cast<uintptr_t>(vst + j * 1024)),
          16, 0, 0);
    }
    const int key = min(kbase + col, chunk_hi);
    const bool fresh = kMode != AttentionMode::decode && key >= p;
    const uint64_t k_address = (fresh ? k_new_base : k_cache_base) +
                               static_cast<uint64_t>(static_cast<uint32_t>(source_row(key))) * kSrcRowBytes +
                               static_cast<uint32_t>(group * static_cast<int>(sizeof(KRaw)));
#pragma unroll
    for (int s = 0; s < DS; ++s)
      kreg[st][s] = *reinterpret_cast<const __attribute__((address_space(1))) KRaw *>(
          k_address + s * 4 * sizeof(KRaw));
  };

  // The first stages of K/V rows go out before the query operands are loaded, so the two
  // round trips overlap.
  // With a single stage, iteration 0's loads go out here and each later one after the previous
  // iteration's compute.
  constexpr int kEarlyStages = kStages > 1 ? kStages - 1 : 1;
  auto issue_early = [&] {
    if (iterations > 0) {
#pragma unroll
      for (int st = 0; st < kEarlyStages; ++st) issue(st, st);
    }
  };
  // With the QKV post-processing fused, this step's K/V rows are written by the workgroup itself
  // first, and only stages issued after those stores may read them (key >= p).
  constexpr bool kFuseQkv = kFuseSplits > 0;
  // decode: the assistant's query-only projection (no K/V rows to store)
  constexpr bool kQueryOnly = kMode == AttentionMode::decode;
  FusedQkv<(kFuseSplits > 0 ? D : 128), (kFuseSplits > 0 ? kFuseSplits : 1), kQueryOnly> fused;
  // Fused QKV: every wave's loads of stages 0 .. 2 kStages - 3 (the early ones and those issued
  // in loop iterations 0 .. kStages - 2) stay below p when the range starts 2 kStages - 2
  // strides before it; the K/V rows' stores then need no wait of their own: a wave's in-order
  // memory counter has retired them once iteration kStages - 2 waited for its stage, and the
  // workgroup barrier at iteration kStages - 1 makes that so for every wave before any fresh key
  // is loaded. For shorter ranges the early stages are issued again after the stores.
  const bool kv_async = kFuseQkv && (kQueryOnly || chunk_lo + (2 * kStages - 2) * stride <= p);
  if constexpr (kFuseQkv) {
    // The prologue's loads go out before the stages (so that waiting for them does not wait for
    // the stages), and the stages unconditionally: a branch here would merge into a full wait.
    fused.load(a, r, h, p);
#pragma unroll
    for (int st = 0; st < kEarlyStages; ++st) issue(st, st);
  } else {
    issue_early();
  }

  // ---- Q operands: column = query row, K-group = d slice. Query row qr = local_head * T + t.
  // In registers, or (kQInLds) in LDS as q_lds[nq][s][lane], each wave loading every kWaves-th
  // step.
  constexpr int kQRegSteps = kQInLds ? 1 : DS;
  u32x4 qop[NQ][kQRegSteps];
  u32x4 *q_lds = reinterpret_cast<u32x4 *>(lds + kWaves * kWaveBytes);
  int row_t[NQ];
  if constexpr (kFuseQkv) {
    static_assert(NQ == 1 && !kQInLds && !kFp8, "fused QKV shape");
    // the query rows [qr = local_head * T + t][D] bf16, in LDS of their own
    bf16_t *q_tile = reinterpret_cast<bf16_t *>(lds + kLdsBytes - kQTileBytes);
    // the prologue's loads went out before the early stages: waiting for them leaves the stages
    // in flight
    wait_vmcnt<kEarlyStages * kLoadsPerStage>();
    fused.finish(a, r, h, p, slot, q_tile, chunk == 0);
    if (kv_async) {
      wait_lgkmcnt0();  // the query rows are in LDS (the K/V stores stay in flight)
      __builtin_amdgcn_s_barrier();
    } else {
      wait_vmcnt<0>();  // this step's K/V rows are stored (and the early stages have landed)
      __syncthreads();
      issue_early();    // again: they may have read fresh rows before the stores
    }
    const int qr = col;
    const bool valid = qr < qrows;
    row_t[0] = valid ? qr % T : -1;
#pragma unroll
    for (int s = 0; s < DS; ++s)
      qop[0][s] = valid ? *reinterpret_cast<const u32x4 *>(q_tile + qr * D + s * 32 + group * 8)
                        : u32x4{0u, 0u, 0u, 0u};
  } else {
#pragma unroll
  for (int nq = 0; nq < NQ; ++nq) {
    const int qr = q0 + nq * 16 + col;
    const bool valid = qr < qrows;
    const int local_head = valid ? qr / T : 0;
    const int t = valid ? qr % T : 0;
    row_t[nq] = valid ? t : -1;
    const bf16_t *qrow =
        a.q + ((static_cast<size_t>(r) * T + t) * a.query_heads + h * G + local_head) * D;
    if constexpr (kQInLds) {
      for (int s = wave; s < DS; s += kWaves)
        q_lds[(nq * DS + s) * 64 + lane] = valid ? *reinterpret_cast<const u32x4 *>(qrow + s * 32 + group * 8)
                                                 : u32x4{0u, 0u, 0u, 0u};
    } else {
#pragma unroll
      for (int s = 0; s < DS; ++s)
        qop[nq][s] = valid ? *reinterpret_cast<const u32x4 *>(qrow + s * 32 + group * 8)
                           : u32x4{0u, 0u, 0u, 0u};
    }
  }
  }
  if constexpr (kQInLds) __syncthreads();
  auto q_operand = [&](int nq, int s) -> u32x4 {
    if constexpr (kQInLds)
      return q_lds[(nq * DS + s) * 64 + lane];
    else
      return qop[nq][s];
  };

  float m_run[NQ], l_run[NQ];
  v4f o[NQ][DT];
#pragma unroll
  for (int nq = 0; nq < NQ; ++nq) {
    m_run[nq] = -INFINITY;
    l_run[nq] = 0.0f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[nq][dt] = v4f{0.f, 0.f, 0.f, 0.f};
  }

  const float score_scale = kFp8 ? a.k_scale * kLog2e : kLog2e;  // scores kept in log2 units
  // V^T operand. Row i of output tile dt stands for d = i * DT + dt (the output rows are
  // permuted the same way), so lane (i = col, group g) needs, of each key row 4g + e, the DT
  // contiguous elements from d = col * DT on: per block of 8 tiles, one wide LDS read per key row
  // (16 bytes of bf16, 8 of e4m3) instead of one read per element. Per-lane offsets inside a V
  // stage, fixed for the whole loop (swizzled chunk positions, see the DMA).
  static_assert(KT == 1, "one 16-key tile per wave iteration");
  static_assert(DT % 8 == 0, "V operand blocks of 8 tiles");
  constexpr int kVBlocks = DT / 8;
  constexpr int kEltBytes = kFp8 ? 1 : 2;
  int v_off[4][kVBlocks];
#pragma unroll
  for (int e = 0; e < 4; ++e)
#pragma unroll
    for (int b = 0; b < kVBlocks; ++b) {
      const int key = 4 * group + e;
      const int byte = (col * DT + 8 * b) * kEltBytes;
      v_off[e][b] = key * kSrcRowBytes + (((byte >> 4) ^ (key % kChunksPerRow)) << 4) + (byte & 15);
    }

  // K operand of MFMA step s from the K slices of stage st (bf16; e4m3 widened exactly).
  auto k_operand = [&](int st, int s) -> u32x4 {
    if constexpr (kFp8)
      return e4m3x8_to_bf16x8(kreg[st][s]);
    else
      return kreg[st][s];
  };
  // A operands of tiles 8b .. 8b + 7: pairs[j] = {V[4g][d], V[4g+1][d]}, {V[4g+2][d], V[4g+3][d]}
  // (bf16) at d = col * DT + 8b + j; e4m3 rows are widened exactly first.
  auto v_block = [&](const unsigned char *vst, int b, u32x2 (&pairs)[8]) {
    u32x4 raw[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if constexpr (kFp8)
        raw[e] = e4m3x8_to_bf16x8(*reinterpret_cast<const u32x2 *>(vst + v_off[e][b]));
      else
        raw[e] = *reinterpret_cast<const u32x4 *>(vst + v_off[e][b]);
    }
    {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
        pairs[j] = u32x2{__builtin_amdgcn_perm(raw[1][j / 2], raw[0][j / 2], sel),
                         __builtin_amdgcn_perm(raw[3][j / 2], raw[2][j / 2], sel)};
      }
    }
  };
  auto process = [&](int kbase, int st, const unsigned char *vst) {
    // ---- scores S^T[key][qrow] (log2 units)
    v4f sc[NQ][KT];
#pragma unroll
    for (int nq = 0; nq < NQ; ++nq)
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) {
        v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < DS; ++s)
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, k_operand(st, s)),
                                                        __builtin_bit_cast(v8bf, q_operand(nq, s)), acc,
                                                        0, 0, 0);
        sc[nq][kt] = acc;
      }

    // ---- mask + online softmax per query column. Tiles strictly inside every query row's
    // visible window (the bulk of the range) skip the mask (a wave-uniform branch).
    bool interior = kbase + 15 <= chunk_hi;
    if (kMode != AttentionMode::decode) interior = interior && kbase + 15 <= p;
    if (kMode == AttentionMode::sliding) interior = interior && kbase >= p + T - a.window;
#pragma unroll
    for (int nq = 0; nq < NQ; ++nq) {
      const int t = row_t[nq];
      float block_max = -INFINITY;
      if (interior) {
#pragma unroll
        for (int kt = 0; kt < KT; ++kt)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            sc[nq][kt][e] *= score_scale;
            block_max = fmaxf(block_max, sc[nq][kt][e]);
          }
      } else {
#pragma unroll
        for (int kt = 0; kt < KT; ++kt)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int key = kbase + kt * 16 + group * 4 + e;
            bool visible = key <= chunk_hi && t >= 0;
            if (kMode != AttentionMode::decode) visible = visible && key <= p + t;
            if (kMode == AttentionMode::sliding) visible = visible && key >= p + t - a.window + 1;
            const float v = visible ? sc[nq][kt][e] * score_scale : -INFINITY;
            sc[nq][kt][e] = v;
            block_max = fmaxf(block_max, v);
          }
      }
      block_max = groups_max(block_max);
      // The reference max m_run only moves when the column's max grew by more than 2^8: the
      // probabilities are then at most 256 (exact relative rounding in bf16, no fp32 overflow)
      // and the accumulators, which live in AGPRs, are rescaled rarely. exp2(-inf) = 0 covers
      // masked keys; m_use keeps a column with no visible key yet away from -inf - -inf.
      const bool grow = block_max > m_run[nq] + 8.0f;
      const float m_new = grow ? block_max : m_run[nq];
      const float m_use = m_new == -INFINITY ? 0.0f : m_new;
      const float alpha = grow ? __builtin_amdgcn_exp2f(m_run[nq] - m_use) : 1.0f;
      float local_sum = 0.0f;
#pragma unroll
      for (int kt = 0; kt < KT; ++kt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float pe = __builtin_amdgcn_exp2f(sc[nq][kt][e] - m_use);
          sc[nq][kt][e] = pe;
          local_sum += pe;
        }
      local_sum = groups_sum(local_sum);
      l_run[nq] = l_run[nq] * alpha + local_sum;
      m_run[nq] = m_new;
      if (__builtin_amdgcn_ballot_w64(grow) != 0) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[nq][dt] *= alpha;
      }
    }

    __asm__ volatile("" ::: "memory");

    // ---- O^T[d][qrow] += V^T[d][keys] . P^T[keys][qrow], 16 keys per MFMA (16x16x16). The
    // score tile's output layout (lane (q, group g) holds keys 4g..4g+3) is exactly the B operand
    // layout, so the probabilities feed the MFMA without a shuffle; the A operand holds
    // V[keys 4g..4g+3][d] for d = col * DT + dt.
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
      s4_t pop[NQ];
#pragma unroll
      for (int nq = 0; nq < NQ; ++nq) {
        const v4f pv = sc[nq][kt];
        pop[nq] = __builtin_bit_cast(s4_t, u32x2{pack_bf16x2(pv[0], pv[1]), pack_bf16x2(pv[2], pv[3])});
      }
#pragma unroll
      for (int b = 0; b < kVBlocks; ++b) {
        u32x2 pairs[8];
        v_block(vst, b, pairs);
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
          for (int nq = 0; nq < NQ; ++nq)
            o[nq][8 * b + j] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
                __builtin_bit_cast(s4_t, pairs[j]), pop[nq], o[nq][8 * b + j], 0, 0, 0);
      }
    }
  };

  // Per-wave pipeline (no workgroup barrier: the stages are private to the wave). The in-order
  // vmcnt counter tracks the loads: with kStages - 1 stages issued ahead, waiting for
  // (kStages - 1) * kLoadsPerStage outstanding means stage `it` has landed. The loop is unrolled
  // by kStages so that every K register slot is a compile-time index.
  if (iterations > 0) {
    for (int it0 = 0; it0 < iterations; it0 += kStages) {
#pragma unroll
      for (int j = 0; j < kStages; ++j) {
        const int it = it0 + j;
        if (it >= iterations) break;
        // fused QKV: every wave's K/V row stores have retired (see kv_async)
        if (kFuseQkv && !kQueryOnly && kv_async && it == kStages - 1) __builtin_amdgcn_s_barrier();
        __asm__ volatile("" ::: "memory");  // the previous iteration's LDS reads stay above
        if constexpr (kStages > 1) issue(it + kStages - 1, (j + kStages - 1) % kStages);
        wait_vmcnt<(kStages - 1) * kLoadsPerStage>();
        __asm__ volatile("" ::: "memory");
        process(first + it * stride, j, wave_lds + j * kStageBytes);
        if constexpr (kStages == 1) {
          __asm__ volatile("" ::: "memory");
          if (it + 1 < iterations) issue(it + 1, 0);
        }
      }
    }
  }
  wait_vmcnt<0>();  // the clamped tail DMAs must land before the LDS is reused below

  // ---- combine the waves through LDS: per wave m, l (per query row) and O rows.
  __syncthreads();
  float *cm = reinterpret_cast<float *>(lds);                // [wave][NQ*16]
  float *cl = cm + kWaves * NQ * 16;                         // [wave][NQ*16]
  float *co = cl + kWaves * NQ * 16;                         // [wave][NQ*16][kCoStride]
#pragma unroll
  for (int nq = 0; nq < NQ; ++nq) {
    const int qr = nq * 16 + col;
    if (group == 0) {
      cm[wave * NQ * 16 + qr] = m_run[nq];
      cl[wave * NQ * 16 + qr] = l_run[nq];
    }
    // row 4g + e of every output tile: d = (4g + e) * DT + dt, DT contiguous floats
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float *dst = co + (static_cast<size_t>(wave) * NQ * 16 + qr) * kCoStride + (group * 4 + e) * DT;
#pragma unroll
      for (int dt = 0; dt < DT; dt += 4)
        *reinterpret_cast<v4f *>(dst + dt) =
            v4f{o[nq][dt][e], o[nq][dt + 1][e], o[nq][dt + 2][e], o[nq][dt + 3][e]};
    }
  }
  __syncthreads();

  // One thread per (query row, 8 consecutive d): the row's wave factors once, then 8 outputs in
  // the same arithmetic order per element as ever; `lr` is the workgroup's row, qr = q0 + lr the
  // item's.
  const int rows_total = qtiles * NQ * 16;
  const bool single = n_chunks == 1;
  float *part = nullptr;
  if (!single) {
    part = a.partials +
           ((static_cast<size_t>(r) * a.kv_heads + h) * max_chunks + chunk) * rows_total * (D + 2);
  }
  const int local_rows = min(NQ * 16, qrows - q0);
  float amax = 0.0f;
  constexpr int kGroups8 = D / 8;
  for (int idx = threadIdx.x; idx < local_rows * kGroups8; idx += kThreads) {
    const int lr = idx / kGroups8;
    const int qr = q0 + lr;
    const int d0 = (idx % kGroups8) * 8;
    float m = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) m = fmaxf(m, cm[w * NQ * 16 + lr]);
    float l = 0.0f, acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (m != -INFINITY) {
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float f = exp2f(cm[w * NQ * 16 + lr] - m);
        l += f * cl[w * NQ * 16 + lr];
        const float *src = co + (static_cast<size_t>(w) * NQ * 16 + lr) * kCoStride + d0;
        const v4f lo = *reinterpret_cast<const v4f *>(src);
        const v4f hi = *reinterpret_cast<const v4f *>(src + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc[e] += f * lo[e];
          acc[4 + e] += f * hi[e];
        }
      }
    }
    if (single) {
      const int local_head = qr / T;
      const int t = qr % T;
      uint32_t packed[4];
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        float v0 = l > 0.0f ? acc[e] / l : 0.0f;
        float v1 = l > 0.0f ? acc[e + 1] / l : 0.0f;
        if constexpr (kFp8) {
          v0 *= a.v_scale;
          v1 *= a.v_scale;
        }
        const bf16_t h0 = f32_to_bf16(v0), h1 = f32_to_bf16(v1);
        amax = fmaxf(amax, fmaxf(fabsf(bf16_to_f32(h0)), fabsf(bf16_to_f32(h1))));
        packed[e / 2] = static_cast<uint32_t>(h0) | (static_cast<uint32_t>(h1) << 16);
      }
      *reinterpret_cast<u32x4 *>(
          a.out + ((static_cast<size_t>(r) * T + t) * a.query_heads + h * G + local_head) * D + d0) =
          u32x4{packed[0], packed[1], packed[2], packed[3]};
    } else {
      float *dst = part + static_cast<size_t>(qr) * (D + 2) + d0;
#pragma unroll
      for (int e = 0; e < 8; ++e) dst[e] = acc[e];
      if (d0 == 0) {
        part[static_cast<size_t>(qr) * (D + 2) + D] = m;
        part[static_cast<size_t>(qr) * (D + 2) + D + 1] = l;
      }
    }
  }

  // One amax update per workgroup (a chunk that wrote partials has no output yet).
  if (a.out_amax != nullptr && single) {
    __shared__ float wave_amax[kWaves];
    amax = block_max(amax, wave_amax);
    if (threadIdx.x == 0) amax_publish(a.out_amax, a.amax_stripes, amax);
  }
}

// Merges the chunk partials (m, l, unnormalised O) of every (request, kv head) that was split:
// one workgroup per (kCombineRows query rows, kv head, request), one thread per output dimension,
// one amax update per workgroup. Up to kCombineFast chunks, every value of the workgroup's rows
// is loaded at once (one memory round trip); longer ranges go row by row, kMaxMergedChunks at a
// time.
constexpr int kMaxMergedChunks = 16;
constexpr int kCombineRows = 4;
constexpr int kCombineFast = 8;

// Online merge of n chunk partials (log2-unit maxima) into (m, l, acc).
template <int N>
__device__ __forceinline__ void merge_chunks(const float (&mc)[N], const float (&lc)[N],
                                             const float (&oc)[N], float &m, float &l, float &acc) {
  float m_new = m;
#pragma unroll
  for (int c = 0; c < N; ++c) m_new = fmaxf(m_new, mc[c]);
  if (m_new == -INFINITY) return;
  const float alpha = exp2f(m - m_new);  // m = -inf -> 0
  l *= alpha;
  acc *= alpha;
#pragma unroll
  for (int c = 0; c < N; ++c) {
    if (mc[c] == -INFINITY) continue;
    const float f = exp2f(mc[c] - m_new);
    l += f * lc[c];
    acc += f * oc[c];
  }
  m = m_new;
}

template <int D, bool kFp8>
__global__ __launch_bounds__(D) void attention_combine_kernel(const AttentionArgs a, int nq) {
  const int h = blockIdx.y;
  const int r = blockIdx.z;
  const int d = threadIdx.x;
  const int G = a.query_heads / a.kv_heads;
  const int T = a.tokens;
  const int p = a.positions[r];
  const KeyRange range = key_range(a, p);
  const int total_keys = range.hi - range.lo + 1;
  const int n_chunks = total_keys <= 0 ? 0 : (total_keys + a.chunk_keys - 1) / a.chunk_keys;
  if (n_chunks <= 1) return;  // single-chunk pairs were finished by the main kernel
  const int rows_total = nq * 16;
  const size_t max_chunks = static_cast<size_t>((a.max_keys + a.chunk_keys - 1) / a.chunk_keys);
  const size_t chunk_stride = static_cast<size_t>(rows_total) * (D + 2);
  const float *pair = a.partials + (static_cast<size_t>(r) * a.kv_heads + h) * max_chunks * chunk_stride;
  const int row0 = blockIdx.x * kCombineRows;
  float m[kCombineRows], l[kCombineRows], acc[kCombineRows];
#pragma unroll
  for (int i = 0; i < kCombineRows; ++i) {
    m[i] = -INFINITY;
    l[i] = 0.0f;
    acc[i] = 0.0f;
  }
  if (n_chunks <= kCombineFast) {
    float mc[kCombineRows][kCombineFast], lc[kCombineRows][kCombineFast], oc[kCombineRows][kCombineFast];
#pragma unroll
    for (int i = 0; i < kCombineRows; ++i) {
      const int qr = min(row0 + i, G * T - 1);
#pragma unroll
      for (int c = 0; c < kCombineFast; ++c) {
        const bool valid = c < n_chunks;
        const float *pr = pair + static_cast<size_t>(valid ? c : 0) * chunk_stride + static_cast<size_t>(qr) * (D + 2);
        mc[i][c] = valid ? pr[D] : -INFINITY;
        lc[i][c] = pr[D + 1];
        oc[i][c] = pr[d];
      }
    }
#pragma unroll
    for (int i = 0; i < kCombineRows; ++i) merge_chunks(mc[i], lc[i], oc[i], m[i], l[i], acc[i]);
  } else {
    for (int i = 0; i < kCombineRows; ++i) {
      const int qr = min(row0 + i, G * T - 1);
      for (int c0 = 0; c0 < n_chunks; c0 += kMaxMergedChunks) {
        float mc[kMaxMergedChunks], lc[kMaxMergedChunks], oc[kMaxMergedChunks];
#pragma unroll
        for (int c = 0; c < kMaxMergedChunks; ++c) {
          const bool valid = c0 + c < n_chunks;
          const float *pr = pair + static_cast<size_t>(valid ? c0 + c : c0) * chunk_stride +
                            static_cast<size_t>(qr) * (D + 2);
          mc[c] = valid ? pr[D] : -INFINITY;
          lc[c] = pr[D + 1];
          oc[c] = pr[d];
        }
        merge_chunks(mc, lc, oc, m[i], l[i], acc[i]);
      }
    }
  }
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < kCombineRows; ++i) {
    const int qr = row0 + i;
    if (qr >= G * T) break;
    float value = l[i] > 0.0f ? acc[i] / l[i] : 0.0f;
    if constexpr (kFp8) value *= a.v_scale;
    const int local_head = qr / T;
    const int t = qr % T;
    const bf16_t hv = f32_to_bf16(value);
    a.out[((static_cast<size_t>(r) * T + t) * a.query_heads + h * G + local_head) * D + d] = hv;
    amax = fmaxf(amax, fabsf(bf16_to_f32(hv)));
  }
  if (a.out_amax != nullptr) {
    __shared__ float wave_amax[D / 64];
    amax = block_max(amax, wave_amax);
    if (threadIdx.x == 0) amax_publish(a.out_amax, a.amax_stripes, amax);
  }
}

// ---------------------------------------------------------------------------------------------
// D-split verify attention for D = 512 with 17..48 query rows per kv head (the Gemma-4 global
// layers: 8 query heads per kv head x 5 rows). One workgroup per (request, kv head, key chunk)
// holds every query row; wave w owns dimensions [128 w, 128 w + 128) of Q, K and V. Each wave's
// partial scores over its dimensions are summed through LDS (fixed order, so every wave holds
// the same scores and runs the same softmax), and each wave accumulates the output for its own
// dimensions. The K/V rows are read once per item instead of once per 16-row query tile.
// ---------------------------------------------------------------------------------------------
constexpr int kSplitD = 512;
constexpr int kSplitTiles = 3;  // 16-row query tiles (<= 48 rows)

// Two workgroups per CU (256 registers per lane, 56 KiB of LDS each) with two K/V stages:
// measured on MI355X at 24 x 4 kv heads x 8192 keys, 398 us against 632-645 us at one workgroup
// per CU with three or four stages.
template <AttentionMode kMode>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void attention_dsplit_kernel(const AttentionArgs a) {
  constexpr int D = kSplitD, NT = kSplitTiles, kWaves = 4, KPI = 16;
  constexpr int DW = D / kWaves;             // dimensions per wave
  constexpr int DSW = DW / 32;               // QK MFMA steps per wave
  constexpr int DTW = DW / 16;               // PV output tiles per wave
  constexpr int kRowBytes = D * 2;           // one bf16 K/V row
  constexpr int kSliceBytes = DW * 2;        // a wave's part of a row
  constexpr int kSliceChunks = kSliceBytes / 16;
  constexpr int kRowsPerDma = 64 / kSliceChunks;
  constexpr int kDma = KPI / kRowsPerDma;
  constexpr int kStages = 2;
  constexpr int kStageBytes = KPI * kSliceBytes;
  constexpr int kLoadsPerStage = kDma + DSW;
  constexpr int kScoreBytes = 2 * kWaves * NT * 64 * 16;  // [parity][wave][tile][lane] v4f
  static_assert(kRowsPerDma * kSliceChunks == 64 && KPI % kRowsPerDma == 0, "DMA row tiling");
  static_assert((kStages - 1) * kLoadsPerStage < 64, "vmcnt range");
  __shared__ __attribute__((aligned(16))) unsigned char lds[kWaves * kStages * kStageBytes + kScoreBytes];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int group = lane >> 4;
  const int col = lane & 15;
  const int G = a.query_heads / a.kv_heads;
  const int T = a.tokens;
  const int qrows = G * T;
  const int max_chunks = (a.max_keys + a.chunk_keys - 1) / a.chunk_keys;
  const int item = blockIdx.x;
  if (item >= max_chunks * a.kv_heads * a.requests) return;
  const int chunk = item % max_chunks;
  const int h = (item / max_chunks) % a.kv_heads;
  const int r = item / (max_chunks * a.kv_heads);
  const int p = a.positions[r];
  const int slot = a.slots[r];
  const KeyRange range = key_range(a, p);
  const int total_keys = range.hi - range.lo + 1;
  if (total_keys <= 0) return;
  const int wrap = kMode == AttentionMode::sliding ? (range.lo / a.capacity) * a.capacity : 0;
  const int n_chunks = (total_keys + a.chunk_keys - 1) / a.chunk_keys;
  if (chunk >= n_chunks) return;
  const int chunk_lo = range.lo + chunk * a.chunk_keys;
  const int chunk_hi = min(range.hi, chunk_lo + a.chunk_keys - 1);
  const int iterations = (chunk_hi - chunk_lo) / KPI + 1;

  const int cache_head = (slot * a.kv_heads + h) * a.capacity;
  const int new_head = r * T * a.kv_heads + h;
  const uint64_t k_cache_base = reinterpret_cast<uint64_t>(a.k_cache);
  const uint64_t v_cache_base = reinterpret_cast<uint64_t>(a.v_cache);
  const uint64_t k_new_base = reinterpret_cast<uint64_t>(a.k_new);
  const uint64_t v_new_base = reinterpret_cast<uint64_t>(a.v_new);
  const int slice = wave * kSliceBytes;
  auto source_row = [&](int key) {
    const bool fresh = key >= p;
    int physical = key - wrap;
    if (kMode == AttentionMode::sliding) physical -= physical >= a.capacity ? a.capacity : 0;
    return fresh ? new_head + (key - p) * a.kv_heads : cache_head + physical;
  };
  // V rows of a stage: row k's 16-byte chunk c at position c ^ swz(k) (the four key groups that
  // one PV operand read touches land in four different 32-byte windows).
  auto swz = [](int key) { return ((key >> 2) & 3) << 1; };

  unsigned char *wave_lds = lds + wave * kStages * kStageBytes;
  v4f *scores_lds = reinterpret_cast<v4f *>(lds + kWaves * kStages * kStageBytes);
  u32x4 kreg[kStages][DSW];
  auto issue = [&](int it, int st) {
    const int kbase = chunk_lo + min(it, iterations - 1) * KPI;
    unsigned char *vst = wave_lds + st * kStageBytes;
#pragma unroll
    for (int j = 0; j < kDma; ++j) {
      const int row_local = j * kRowsPerDma + lane / kSliceChunks;
      const int position = lane % kSliceChunks;
      const int key = min(kbase + row_local, chunk_hi);
      const bool fresh = key >= p;
      const uint64_t offset = static_cast<uint64_t>(static_cast<uint32_t>(source_row(key))) * kRowBytes +
                              slice + ((position ^ swz(row_local)) << 4);
      __builtin_amdgcn_global_load_lds(
          reinterpret_cast<const void *>((fresh ? v_new_base : v_cache_base) + offset),
          reinterpret_cast<void __attribute__((address_space(3))) *>(
              reinterpret_cast<uintptr_t>(vst + j * 1024)),
          16, 0, 0);
    }
    const int key = min(kbase + col, chunk_hi);
    const bool fresh = key >= p;
    const uint64_t k_address = (fresh ? k_new_base : k_cache_base) +
                               static_cast<uint64_t>(static_cast<uint32_t>(source_row(key))) * kRowBytes +
                               slice + group * 16;
#pragma unroll
    for (int s = 0; s < DSW; ++s)
      kreg[st][s] = *reinterpret_cast<const __attribute__((address_space(1))) u32x4 *>(k_address + s * 64);
  };

#pragma unroll
  for (int st = 0; st < kStages - 1; ++st) issue(st, st);

  // Q operand (B of the QK MFMA) for this wave's dimensions: lane (query row, group g) holds
  // dims [32 s + 8 g, +8) of the slice. Query row qr = local_head * T + t.
  u32x4 qop[NT][DSW];
  int row_t[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int qr = nt * 16 + col;
    const bool valid = qr < qrows;
    const int local_head = valid ? qr / T : 0;
    const int t = valid ? qr % T : 0;
    row_t[nt] = valid ? t : -1;
    const bf16_t *qrow = a.q + ((static_cast<size_t>(r) * T + t) * a.query_heads + h * G + local_head) * D +
                         wave * DW;
#pragma unroll
    for (int s = 0; s < DSW; ++s)
      qop[nt][s] = valid ? *reinterpret_cast<const u32x4 *>(qrow + s * 32 + group * 8) : u32x4{0u, 0u, 0u, 0u};
  }

  float m_run[NT], l_run[NT];
  v4f o[NT][DTW];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    m_run[nt] = -INFINITY;
    l_run[nt] = 0.0f;
#pragma unroll
    for (int dt = 0; dt < DTW; ++dt) o[nt][dt] = v4f{0.f, 0.f, 0.f, 0.f};
  }
  // V[key 4 g + e][d = 16 dt + col] of a stage: byte (16 dt + col) * 2 of row 4 g + e, i.e.
  // chunk 2 dt + col / 8 at position (2 dt + col / 8) ^ swz(4 g + e) = (2 dt) ^ swz | col / 8 (swz
  // is even), so the per-lane part is one offset per e.
  int v_lane[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int key = 4 * group + e;
    v_lane[e] = key * kSliceBytes + ((col >> 3) << 4) + (col & 7) * 2;
  }
  const int v_xor = swz(4 * group) << 4;  // the same for the four keys of the group

  // Unrolled by kStages so that every K register slot is a compile-time index.
  for (int it0 = 0; it0 < iterations; it0 += kStages)
#pragma unroll
  for (int st = 0; st < kStages; ++st) {
    const int it = it0 + st;
    if (it >= iterations) break;
    __asm__ volatile("" ::: "memory");
    issue(it + kStages - 1, (st + kStages - 1) % kStages);
    wait_vmcnt<(kStages - 1) * kLoadsPerStage>();
    __asm__ volatile("" ::: "memory");
    const int kbase = chunk_lo + it * KPI;
    // ---- partial scores over this wave's dimensions
    v4f part[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < DSW; ++s)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, kreg[st][s]),
                                                      __builtin_bit_cast(v8bf, qop[nt][s]), acc, 0, 0, 0);
      part[nt] = acc;
    }
    v4f *buf = scores_lds + (it & 1) * kWaves * NT * 64;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) buf[(wave * NT + nt) * 64 + lane] = part[nt];
    // LDS writes done, then a bare barrier: a fence here would also drain the K/V loads in flight.
    // The other parity's buffer is free: every wave read it before this iteration's barrier.
    wait_lgkmcnt0();
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
    v4f sc[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      v4f sum = buf[nt * 64 + lane];
#pragma unroll
      for (int w = 1; w < kWaves; ++w) sum += buf[(w * NT + nt) * 64 + lane];
      sc[nt] = sum;
    }
    // ---- mask + online softmax (the same rules as attention_kernel)
    bool interior = kbase + 15 <= chunk_hi && kbase + 15 <= p;
    if (kMode == AttentionMode::sliding) interior = interior && kbase >= p + T - a.window;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int t = row_t[nt];
      float block_max = -INFINITY;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int key = kbase + group * 4 + e;
        bool visible = interior || (key <= chunk_hi && key <= p + t);
        if (kMode == AttentionMode::sliding && !interior) visible = visible && key >= p + t - a.window + 1;
        visible = visible && t >= 0;
        const float v = visible ? sc[nt][e] * kLog2e : -INFINITY;
        sc[nt][e] = v;
        block_max = fmaxf(block_max, v);
      }
      block_max = groups_max(block_max);
      const bool grow = block_max > m_run[nt] + 8.0f;
      const float m_new = grow ? block_max : m_run[nt];
      const float m_use = m_new == -INFINITY ? 0.0f : m_new;
      const float alpha = grow ? __builtin_amdgcn_exp2f(m_run[nt] - m_use) : 1.0f;
      float local_sum = 0.0f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float pe = __builtin_amdgcn_exp2f(sc[nt][e] - m_use);
        sc[nt][e] = pe;
        local_sum += pe;
      }
      local_sum = groups_sum(local_sum);
      l_run[nt] = l_run[nt] * alpha + local_sum;
      m_run[nt] = m_new;
      if (__builtin_amdgcn_ballot_w64(grow) != 0) {
#pragma unroll
        for (int dt = 0; dt < DTW; ++dt) o[nt][dt] *= alpha;
      }
    }
    // ---- O^T[d][q] += V^T[d][keys] . P^T[keys][q] for this wave's dimensions
    s4_t pop[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
      pop[nt] = __builtin_bit_cast(s4_t, u32x2{pack_bf16x2(sc[nt][0], sc[nt][1]),
                                               pack_bf16x2(sc[nt][2], sc[nt][3])});
    const unsigned char *vst = wave_lds + st * kStageBytes;
#pragma unroll
    for (int dt = 0; dt < DTW; ++dt) {
      const int chunk_off = ((2 * dt) << 4) ^ v_xor;
      uint32_t v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = *reinterpret_cast<const uint16_t *>(vst + v_lane[e] + chunk_off);
      const u32x2 vv = {v[0] | (v[1] << 16), v[2] | (v[3] << 16)};
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
        o[nt][dt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s4_t, vv), pop[nt],
                                                              o[nt][dt], 0, 0, 0);
    }
  }
  wait_vmcnt<0>();  // the clamped tail loads land before the workgroup ends

  // ---- output: every wave holds the same m, l; lane (query col, group g) holds dimensions
  // 16 dt + 4 g + {0..3} of its slice.
  const bool single = n_chunks == 1;
  const int rows_total = NT * 16;
  float *part_out = single ? nullptr
                           : a.partials + ((static_cast<size_t>(r) * a.kv_heads + h) * max_chunks + chunk) *
                                              rows_total * (D + 2);
  float amax = 0.0f;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int qr = nt * 16 + col;
    if (qr >= qrows) continue;
    if (single) {
      const int local_head = qr / T;
      const int t = qr % T;
      bf16_t *dst = a.out + ((static_cast<size_t>(r) * T + t) * a.query_heads + h * G + local_head) * D +
                    wave * DW + group * 4;
#pragma unroll
      for (int dt = 0; dt < DTW; ++dt) {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = l_run[nt] > 0.0f ? o[nt][dt][e] / l_run[nt] : 0.0f;
          v[e] = bf16_to_f32(f32_to_bf16(v[e]));
          amax = fmaxf(amax, fabsf(v[e]));
        }
        *reinterpret_cast<uint2 *>(dst + dt * 16) = uint2{f32x2_to_bf16x2(v[0], v[1]), f32x2_to_bf16x2(v[2], v[3])};
      }
    } else {
      float *dst = part_out + static_cast<size_t>(qr) * (D + 2);
#pragma unroll
      for (int dt = 0; dt < DTW; ++dt)
        *reinterpret_cast<v4f *>(dst + wave * DW + dt * 16 + group * 4) = o[nt][dt];
      if (wave == 0 && group == 0) {
        dst[D] = m_run[nt];
        dst[D + 1] = l_run[nt];
      }
    }
  }
  if (a.out_amax != nullptr && single) {
    __shared__ float wave_amax[kWaves];
    amax = block_max(amax, wave_amax);
    if (threadIdx.x == 0) amax_publish(a.out_amax, a.amax_stripes, amax);
  }
}

void launch_dsplit(const AttentionArgs &a, hipStream_t stream) {
  const int64_t items = static_cast<int64_t>((a.max_keys + a.chunk_keys - 1) / a.chunk_keys) *
                        a.kv_heads * a.requests;
  if (items > (int64_t{1} << 31) - 1) throw std::runtime_error("attention grid too large");
  const dim3 grid(static_cast<unsigned>(items));
  if (a.timing_start != nullptr) hip_check(hipEventRecord(a.timing_start, stream), "record probe");
  if (a.mode == AttentionMode::sliding)
    attention_dsplit_kernel<AttentionMode::sliding><<<grid, 256, 0, stream>>>(a);
  else
    attention_dsplit_kernel<AttentionMode::global><<<grid, 256, 0, stream>>>(a);
  if (a.timing_stop != nullptr) hip_check(hipEventRecord(a.timing_stop, stream), "record probe");
  if ((a.max_keys + a.chunk_keys - 1) / a.chunk_keys > 1) {
    const int qrows = (a.query_heads / a.kv_heads) * a.tokens;
    attention_combine_kernel<kSplitD, false>
        <<<dim3((qrows + kCombineRows - 1) / kCombineRows, a.kv_heads, a.requests), kSplitD, 0, stream>>>(
            a, kSplitTiles);
  }
}

template <int D, int NQ, bool kFp8>
void launch_mode(const AttentionArgs &a, dim3 grid, hipStream_t stream) {
  switch (a.mode) {
  case AttentionMode::sliding:
    attention_kernel<D, NQ, kFp8, AttentionMode::sliding, kAttentionWaves>
        <<<grid, kAttentionWaves * 64, 0, stream>>>(a);
    break;
  case AttentionMode::global:
    attention_kernel<D, NQ, kFp8, AttentionMode::global, kAttentionWaves>
        <<<grid, kAttentionWaves * 64, 0, stream>>>(a);
    break;
  case AttentionMode::decode:
    attention_kernel<D, NQ, kFp8, AttentionMode::decode, kAttentionWaves>
        <<<grid, kAttentionWaves * 64, 0, stream>>>(a);
    break;
  }
}

// Verify attention with the step's QKV post-processing fused (attention_can_fuse_qkv).
template <int S>
void launch_fused(const AttentionArgs &a, dim3 grid, hipStream_t stream) {
  if (a.mode == AttentionMode::sliding)
    attention_kernel<128, 1, false, AttentionMode::sliding, kAttentionWaves, S>
        <<<grid, kAttentionWaves * 64, 0, stream>>>(a);
  else if (a.mode == AttentionMode::decode)
    attention_kernel<128, 1, false, AttentionMode::decode, kAttentionWaves, S>
        <<<grid, kAttentionWaves * 64, 0, stream>>>(a);
  else
    attention_kernel<128, 1, false, AttentionMode::global, kAttentionWaves, S>
        <<<grid, kAttentionWaves * 64, 0, stream>>>(a);
}

template <int D, int NQ>
void launch_typed(const AttentionArgs &a, dim3 grid, hipStream_t stream) {
  if (a.timing_start != nullptr) hip_check(hipEventRecord(a.timing_start, stream), "record probe");
  if constexpr (D == 128 && NQ == 1) {
    if (a.fuse_qkv) {
      if (a.qkv.splits == 1)
        launch_fused<1>(a, grid, stream);
      else
        launch_fused<2>(a, grid, stream);
    }
  }
  if (!a.fuse_qkv) {
    if (a.fp8_kv)
      launch_mode<D, NQ, true>(a, grid, stream);
    else
      launch_mode<D, NQ, false>(a, grid, stream);
  }
  if (a.timing_stop != nullptr) hip_check(hipEventRecord(a.timing_stop, stream), "record probe");
  if ((a.max_keys + a.chunk_keys - 1) / a.chunk_keys > 1) {
    const int qrows = (a.query_heads / a.kv_heads) * a.tokens;
    const int tiles = (qrows + NQ * 16 - 1) / (NQ * 16) * NQ;  // 16-row tiles of the partials
    const dim3 combine_grid((qrows + kCombineRows - 1) / kCombineRows, a.kv_heads, a.requests);
    if (a.fp8_kv)
      attention_combine_kernel<D, true><<<combine_grid, D, 0, stream>>>(a, tiles);
    else
      attention_combine_kernel<D, false><<<combine_grid, D, 0, stream>>>(a, tiles);
  }
}

}  // namespace

bool attention_can_fuse_qkv(const AttentionArgs &a) {
  const QkvArgs &q = a.qkv;
  if (a.mode == AttentionMode::decode) {
    // the assistant's query-only projection, one row per request, any number of key chunks
    const int G = a.kv_heads > 0 ? a.query_heads / a.kv_heads : 0;
    return a.dimension == 128 && !a.fp8_kv && G > 0 && G <= 16 && a.tokens == 1 &&
           G <= kAttentionWaves * kFusedQkvUnitsPerWave && a.chunk_keys > 0 &&
           q.partials != nullptr && (q.splits == 1 || q.splits == 2) &&
           (q.x_amax == nullptr) == (q.w_scale == nullptr) && q.kv_heads == 0 &&
           q.rows == a.requests && q.tokens == 1 && q.query_heads == a.query_heads &&
           q.dimension == 128 && q.q_norm != nullptr && q.cosine != nullptr && q.sine != nullptr &&
           q.positions == a.positions && q.q_out != nullptr && q.q_out == a.q;
  }
  const int G = a.kv_heads > 0 ? a.query_heads / a.kv_heads : 0;
  const int units = G * a.tokens + (q.key_equals_value ? 1 : 2) * a.tokens;
  return (a.mode == AttentionMode::sliding || a.mode == AttentionMode::global) && a.dimension == 128 &&
         !a.fp8_kv && G > 0 && G * a.tokens <= 16 && a.tokens <= kFusedQkvMaxTokens &&
         units <= kAttentionWaves * kFusedQkvUnitsPerWave && a.chunk_keys > 0 &&
         (a.max_keys + a.chunk_keys - 1) / a.chunk_keys == 1 && q.partials != nullptr &&
         (q.splits == 1 || q.splits == 2) && q.x_amax != nullptr && q.w_scale != nullptr &&
         q.rows == a.requests * a.tokens && q.tokens == a.tokens && q.query_heads == a.query_heads &&
         q.kv_heads == a.kv_heads && q.dimension == 128 && q.q_norm != nullptr &&
         q.k_norm != nullptr && q.cosine != nullptr && q.sine != nullptr && q.positions == a.positions &&
         q.slots == a.slots && q.position_offset == 0 && q.k_new == a.k_new && q.v_new == a.v_new &&
         (q.k_cache == nullptr || (q.v_cache != nullptr && q.capacity > 0));
}

size_t attention_partials_floats(int requests, int kv_heads, int max_keys, int chunk_keys,
                                 int query_rows, int dimension) {
  const size_t chunks = static_cast<size_t>((max_keys + chunk_keys - 1) / chunk_keys);
  const size_t rows = static_cast<size_t>((query_rows + 31) / 32) * 32;  // whole workgroup tiles
  return static_cast<size_t>(requests) * kv_heads * chunks * rows * (dimension + 2);
}


int attention_default_chunk(AttentionMode mode, int max_keys, int requests, int kv_heads,
                            bool fp8_kv, int dimension) {
  // One workgroup per (request, kv head) streams the whole key range when that already gives
  // >= 256 workgroups: two or three co-reside per CU, so an uneven count still shares the HBM
  // stream evenly, and no partials or merge kernel are needed (measured on MI355X, 24 slots x 16
  // kv heads: global verify 290 us in one chunk, 287 us in four 2048-key chunks plus the merge;
  // sliding verify 50 us whole, 54 us in two chunks plus the merge). Smaller batches split the
  // range so that up to 512 workgroups stream it.
  //
  // Two exceptions at D = 128, where three workgroups fit a CU: with one workgroup per pair the
  // 128 CUs holding two of them fall behind the 128 holding one, and two chunks per pair put
  // exactly three workgroups on every CU (768 workgroups). e4m3 K/V verify (a workgroup moves
  // half the bytes per key; cold HBM, 24 x 16 pairs x 8155 keys: the single-workgroup CUs finish
  // 134 us in, the last workgroups at 182 us; two chunks: 152 us plus the merge), and the
  // assistant's decode over the global cache (one query row per head, no amax for the merge to
  // publish: 3.31 -> 3.26 ms per draft). bf16 verify gains nothing from it (13.61 ms either way).
  const int whole = ((max_keys + 255) / 256) * 256;
  const int pairs = std::max(1, requests * kv_heads);
  const bool balance = (fp8_kv && mode != AttentionMode::decode) || (!fp8_kv && mode == AttentionMode::decode);
  if (balance && dimension == 128 && pairs >= 256 && 2 * pairs <= 3 * 256 && max_keys >= 2048)
    return ((max_keys + 1) / 2 + 255) / 256 * 256;
  if (pairs >= 256) return whole;
  // the smallest 256-key multiple that keeps the workgroups at <= 512
  const long chunks = std::max(1L, 512L / pairs);
  const int chunk = static_cast<int>(((max_keys + chunks - 1) / chunks + 255) / 256 * 256);
  return std::min(std::max(chunk, 256), whole);
}

void launch_attention(const AttentionArgs &a, hipStream_t stream) {
  if (a.q == nullptr || a.k_cache == nullptr || a.v_cache == nullptr || a.out == nullptr ||
      a.slots == nullptr || a.positions == nullptr || a.requests <= 0 || a.tokens <= 0 ||
      a.tokens > 1024 || a.kv_heads <= 0 || a.query_heads % a.kv_heads != 0 || a.capacity <= 0 ||
      a.max_keys <= 0 || a.chunk_keys <= 0 || a.chunk_keys % 256 != 0)
    throw std::runtime_error("invalid verify attention shape");
  check_amax_stripes(a.amax_stripes);
  if (a.mode != AttentionMode::decode && (a.k_new == nullptr || a.v_new == nullptr))
    throw std::runtime_error("verify attention needs this step's K/V rows");
  if (a.mode == AttentionMode::sliding && (a.window <= 0 || a.window > a.capacity))
    throw std::runtime_error("sliding attention window must fit the ring");
  if (a.mode == AttentionMode::decode && a.tokens != 1)
    throw std::runtime_error("decode attention takes one query token");
  if (a.fuse_qkv && !attention_can_fuse_qkv(a))
    throw std::runtime_error("this attention call cannot take the QKV post-processing");
  if (a.fuse_qkv) check_amax_stripes(a.qkv.amax_stripes);
  const int qrows = (a.query_heads / a.kv_heads) * a.tokens;
  const int max_chunks = (a.max_keys + a.chunk_keys - 1) / a.chunk_keys;
  if (max_chunks > 1 && a.partials == nullptr)
    throw std::runtime_error("split attention needs a partial workspace");
  const int64_t slot_count = a.slot_count > 0 ? a.slot_count : a.requests;
  if (slot_count * a.kv_heads * a.capacity >= (int64_t{1} << 31) ||
      static_cast<int64_t>(a.requests) * a.tokens * a.kv_heads >= (int64_t{1} << 31))
    throw std::runtime_error("attention cache exceeds 2^31 rows");
  // One workgroup per (key chunk, kv head, request, query tile); the item count is padded to a
  // multiple of the 8 XCDs (see the kernel's mapping).
  const int64_t items = static_cast<int64_t>(max_chunks) * a.kv_heads * a.requests;
  auto grid_for = [&](int rows_per_workgroup) {
    const int64_t tiles = (qrows + rows_per_workgroup - 1) / rows_per_workgroup;
    const int64_t blocks = (items + 7) / 8 * 8 * tiles;
    if (blocks > (int64_t{1} << 31) - 1) throw std::runtime_error("attention grid too large");
    return dim3(static_cast<unsigned>(blocks));
  };
  if (qrows > 16384) throw std::runtime_error("attention supports at most 16384 query rows per kv head");
  if (a.dimension == 128 && qrows <= 16)
    launch_typed<128, 1>(a, grid_for(16), stream);
  else if (a.dimension == 128)
    launch_typed<128, 2>(a, grid_for(32), stream);
  else if (a.dimension == 256)
    launch_typed<256, 1>(a, grid_for(16), stream);
  else if (a.dimension == 512 && !a.fp8_kv && a.mode != AttentionMode::decode && qrows > 16 &&
           qrows <= 16 * kSplitTiles)
    launch_dsplit(a, stream);
  else if (a.dimension == 512)
    launch_typed<512, 1>(a, grid_for(16), stream);
  else
    throw std::runtime_error("attention head dimension " + std::to_string(a.dimension) +
                             " not instantiated (128, 256, 512)");
  hip_check(hipGetLastError(), "launch verify attention");
}

}  // namespace carat_hip
