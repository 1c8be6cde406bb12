// Skinny weight-streaming GEMM for gfx950: Y[M][N] = X[M][K] . W[N][K]^T, M <= 128 per token block.
//
// Roles: weights are the MFMA A operand (16 features per tile), tokens the B operand (16 per tile).
// Every weight byte is used by exactly one wave, so weights stream HBM -> VGPRs directly, P steps
// ahead, from the packed layout (gemm.h) in which a workgroup's weights for one K step are one
// contiguous run and each wave load instruction reads 1 KiB contiguous. The activations are
// shared by all waves of a workgroup and stay row-major: bf16 GEMMs read their producer's output;
// for e4m3 weights they are quantised once with the producer's per-tensor amax (scale =
// amax / 448, q = e4m3(x * (1 / scale)), cuda/linear.cu:107-110,143-186) by prepare_x_kernel or
// by the producing row kernel itself. Each step's 128-byte slice of every token row is DMA'd
// global -> LDS (global_load_lds_dwordx4). Loads are issued branch-free
// (tail steps re-issue the last step's addresses, which hit in cache) so the in-order vmcnt counter
// keeps P steps in flight.
//
// Operand K order inside a 128-byte step (identical for A and B, so the dot product is unchanged):
// lane group g holds bytes [g*16, g*16+16) and [64+g*16, 64+g*16+16); for bf16 these are the K
// slices of the two 16x16x32 MFMAs, for fp8 the one 16x16x128 MFMA.
#include "gemm.h"

#include <algorithm>

namespace carat_hip {
namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kStepBytes = 128;    // bytes of one weight row per K step
constexpr int kTileBytes = 2048;   // one 16-token B operand tile of one step

// GELU, tanh form (cuda/ops.cu:228-284): 0.5 v (1 + tanh(u)), u = sqrt(2/pi) (v + 0.044715 v^3).
// Since 1 + tanh(u) = 2 / (1 + e^(-2u)), this is v / (1 + 2^(-2u log2 e)): one v_exp_f32 and one
// v_rcp_f32, branch-free (a library tanhf inlines a branchy sequence per element). Both saturate
// correctly: e^(-2u) -> inf gives 0, -> 0 gives v.
__device__ __forceinline__ float gelu_tanh(float v) {
  const float u = 0.7978845608028654f * (v + 0.044715f * v * v * v);
  return v * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-2.8853900817779268f * u));
}


// ---------------------------------------------------------------------------------------------
// weight packing: one thread per 16-byte chunk of the packed layout
// ---------------------------------------------------------------------------------------------
struct PackGeometry {
  int n, row_bytes, f, waves, gate_up, steps, group_tiles, blocks, step_major;
};

// Logical (row, byte offset) of packed 16-byte chunk `chunk`.
__device__ __forceinline__ void packed_chunk_source(const PackGeometry &g, size_t chunk, int &row,
                                                    int &byte) {
  const int lane = static_cast<int>(chunk & 63);
  const int half = static_cast<int>((chunk >> 6) & 1);
  size_t rest = chunk >> 7;
  const int tile = static_cast<int>(rest % g.group_tiles);
  rest /= g.group_tiles;
  const int step = static_cast<int>(g.step_major ? rest / g.blocks : rest % g.steps);
  const int block = static_cast<int>(g.step_major ? rest % g.blocks : rest / g.steps);
  const int col = lane & 15;
  if (g.gate_up) {
    const int h = g.f / 2;
    const int wave = tile / g.f;
    const int f = tile % g.f;
    const int gate_row = block * (16 * g.waves * h) + (wave * h + (f % h)) * 16 + col;
    row = f < h ? gate_row : g.n / 2 + gate_row;
  } else {
    row = block * (16 * g.group_tiles) + tile * 16 + col;
  }
  byte = step * kStepBytes + half * 64 + (lane >> 4) * 16;
}

template <bool kPack>
__global__ __launch_bounds__(256) void pack_weight_kernel(const unsigned char *src,
                                                          unsigned char *dst, PackGeometry g,
                                                          size_t chunks) {
  for (size_t chunk = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; chunk < chunks;
       chunk += static_cast<size_t>(gridDim.x) * blockDim.x) {
    int row, byte;
    packed_chunk_source(g, chunk, row, byte);
    const size_t logical = static_cast<size_t>(row) * g.row_bytes + byte;
    if constexpr (kPack)
      *reinterpret_cast<u32x4 *>(dst + chunk * 16) = *reinterpret_cast<const u32x4 *>(src + logical);
    else
      *reinterpret_cast<u32x4 *>(dst + logical) = *reinterpret_cast<const u32x4 *>(src + chunk * 16);
  }
}

void check_layout(const WeightLayout &l) {
  const int f = l.tiles_per_wave;
  if (l.n <= 0 || l.row_bytes <= 0 || l.row_bytes % kStepBytes != 0 ||
      (f != 1 && f != 2 && f != 4) || (l.gate_up && f == 1) || l.waves < 1 || l.waves > 4 ||
      l.n % (16 * l.waves * f) != 0)
    throw std::runtime_error("invalid packed weight layout");
}

void launch_pack(const void *src, void *dst, const WeightLayout &l, bool pack, hipStream_t stream) {
  check_layout(l);
  if (src == nullptr || dst == nullptr) throw std::runtime_error("null weight pointer");
  const PackGeometry g{l.n, l.row_bytes, l.tiles_per_wave, l.waves, l.gate_up ? 1 : 0,
                       l.row_bytes / kStepBytes, l.waves * l.tiles_per_wave,
                       l.n / (16 * l.waves * l.tiles_per_wave), l.step_major ? 1 : 0};
  const size_t chunks = static_cast<size_t>(l.n) * l.row_bytes / 16;
  const unsigned blocks = static_cast<unsigned>(std::min<size_t>((chunks + 255) / 256, 65536));
  if (pack)
    pack_weight_kernel<true><<<blocks, 256, 0, stream>>>(
        static_cast<const unsigned char *>(src), static_cast<unsigned char *>(dst), g, chunks);
  else
    pack_weight_kernel<false><<<blocks, 256, 0, stream>>>(
        static_cast<const unsigned char *>(src), static_cast<unsigned char *>(dst), g, chunks);
  hip_check(hipGetLastError(), "launch weight packing");
}

// ---------------------------------------------------------------------------------------------
// e4m3 activation operand: out[token][k], row-major like the bf16 producer output, quantised with
// the producer's per-tensor scale amax / 448 (cuda/linear.cu:107-110, 143-186). Quantising once
// here keeps the per-workgroup operand traffic of the GEMM at one byte per element; the GEMM
// gathers each token's 128-byte step slice (one cache line) by DMA, as it gathers bf16 rows, and
// a producer that owns a token row writes whole lines of it.
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void prepare_x_kernel(const bf16_t *x, int ldx, int m, int k,
                                                        const float *x_amax, int amax_stripes,
                                                        int token_tiles, unsigned char *out) {
  const int pieces = k / 16;  // 16-byte output chunks per token
  const int chunk = blockIdx.x * blockDim.x + threadIdx.x;  // one 16-byte chunk per thread
  const int tokens = token_tiles * 16;
  const int token = blockIdx.y * tokens + chunk / pieces;
  const int piece = chunk % pieces;
  // The row slice goes out before the amax: neither load waits for the other. Lanes past the
  // tokens re-read a valid slice (token m - 1) and store nothing.
  const bf16_t *src = x + static_cast<size_t>(min(token, m - 1)) * ldx + piece * 16;
  const u32x4 lo = *reinterpret_cast<const u32x4 *>(src);
  const u32x4 hi = *reinterpret_cast<const u32x4 *>(src + 8);
  const float inv = 1.0f / fp8_scale_from_amax(amax_read(x_amax, amax_stripes));
  if (chunk >= tokens * pieces || token >= m) return;
  u32x4 value;
  const uint32_t w[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
#pragma unroll
  for (int q = 0; q < 4; ++q)
    value[q] = f32x4_to_e4m3x4(__uint_as_float(w[2 * q] << 16) * inv,
                               __uint_as_float(w[2 * q] & 0xffff0000u) * inv,
                               __uint_as_float(w[2 * q + 1] << 16) * inv,
                               __uint_as_float(w[2 * q + 1] & 0xffff0000u) * inv);
  reinterpret_cast<u32x4 *>(out + static_cast<size_t>(token) * k)[piece] = value;
}

// Fp8Scaling::channel / ::block_128 activation operands (quantize_bf16_rows_kernel and
// quantize_activation_block_128_kernel, cuda/linear.cu:300-316, 382-401): scale =
// max(amax / 448, 2^-24) per token row (channel) or per token and 128-element K step (block_128),
// q = e4m3(x / scale), written in the row-major operand layout of prepare_x_kernel. Scales:
// channel x_scales[token]; block_128 x_scales[m_block][step][col][token tile] (token = tile * 16 +
// col of the block), so that a lane's token tiles of one step are contiguous. Tokens past m get a
// scale but no operand row (the GEMM re-reads row m - 1 for them and stores nothing).
__device__ __forceinline__ u32x4 quantize_chunk(u32x4 lo, u32x4 hi, float scale, bool live) {
  u32x4 value = {0u, 0u, 0u, 0u};
  if (!live) return value;
  const uint32_t w[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
#pragma unroll
  for (int q = 0; q < 4; ++q)
    value[q] = f32x4_to_e4m3x4(__uint_as_float(w[2 * q] << 16) / scale,
                               __uint_as_float(w[2 * q] & 0xffff0000u) / scale,
                               __uint_as_float(w[2 * q + 1] << 16) / scale,
                               __uint_as_float(w[2 * q + 1] & 0xffff0000u) / scale);
  return value;
}

__device__ __forceinline__ float chunk_amax(u32x4 lo, u32x4 hi) {
  const uint32_t w[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
  float m = 0.0f;
#pragma unroll
  for (int q = 0; q < 8; ++q)
    m = fmaxf(m, fmaxf(fabsf(__uint_as_float(w[q] << 16)), fabsf(__uint_as_float(w[q] & 0xffff0000u))));
  return m;
}

// channel: one workgroup per token of the padded token blocks (scales for all, rows for live ones)
__global__ __launch_bounds__(256) void prepare_x_rows_kernel(const bf16_t *x, int ldx, int m, int k,
                                                             unsigned char *out, float *x_scales) {
  const int token = blockIdx.x;
  const bool live = token < m;
  const bf16_t *src = x + static_cast<size_t>(min(token, m - 1)) * ldx;
  const int chunks = k / 16;
  float amax = 0.0f;
  for (int c = threadIdx.x; c < chunks; c += 256)
    amax = fmaxf(amax, chunk_amax(*reinterpret_cast<const u32x4 *>(src + c * 16),
                                  *reinterpret_cast<const u32x4 *>(src + c * 16 + 8)));
  __shared__ float wave_maxima[4];
  amax = wave_max(amax);
  if ((threadIdx.x & 63) == 0) wave_maxima[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(wave_maxima[0], wave_maxima[1]), fmaxf(wave_maxima[2], wave_maxima[3]));
  const float scale = fmaxf(amax / 448.0f, 0x1p-24f);
  if (threadIdx.x == 0) x_scales[token] = scale;
  for (int c = threadIdx.x; c < chunks; c += 256) {
    const u32x4 value = quantize_chunk(*reinterpret_cast<const u32x4 *>(src + c * 16),
                                       *reinterpret_cast<const u32x4 *>(src + c * 16 + 8), scale, live);
    if (live) reinterpret_cast<u32x4 *>(out + static_cast<size_t>(token) * k)[c] = value;
  }
}

// block_128: one wave per (token block, step, token tile); lane (group, col) holds both halves
__global__ __launch_bounds__(256) void prepare_x_blocks_kernel(const bf16_t *x, int ldx, int m, int k,
                                                               int token_tiles, unsigned char *out,
                                                               float *x_scales) {
  const int steps = k / kStepBytes;
  const int w = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (w >= steps * token_tiles) return;  // wave-uniform
  const int m_block = blockIdx.y;
  const int step = w / token_tiles, tile = w % token_tiles;
  const int lane = threadIdx.x & 63, group = lane >> 4, col = lane & 15;
  const int token = m_block * token_tiles * 16 + tile * 16 + col;
  const bf16_t *src = x + static_cast<size_t>(min(token, m - 1)) * ldx + step * 128 + group * 16;
  const u32x4 lo0 = *reinterpret_cast<const u32x4 *>(src);
  const u32x4 hi0 = *reinterpret_cast<const u32x4 *>(src + 8);
  const u32x4 lo1 = *reinterpret_cast<const u32x4 *>(src + 64);
  const u32x4 hi1 = *reinterpret_cast<const u32x4 *>(src + 72);
  float amax = fmaxf(chunk_amax(lo0, hi0), chunk_amax(lo1, hi1));
  amax = fmaxf(amax, __shfl_xor(amax, 16, kWave));
  amax = fmaxf(amax, __shfl_xor(amax, 32, kWave));
  const float scale = fmaxf(amax / 448.0f, 0x1p-24f);
  const bool live = token < m;
  if (live) {
    u32x4 *dst = reinterpret_cast<u32x4 *>(out + static_cast<size_t>(token) * k + step * 128) + group;
    dst[0] = quantize_chunk(lo0, hi0, scale, true);
    dst[4] = quantize_chunk(lo1, hi1, scale, true);
  }
  if (group == 0)
    x_scales[((static_cast<size_t>(m_block) * steps + step) * 16 + col) * token_tiles + tile] = scale;
}

// ---------------------------------------------------------------------------------------------
// main kernel: W waves; wave w owns F feature tiles (16 features each) x TT token tiles. The F
// tiles come from kBlocks consecutive blocks of the packed layout (F / kBlocks tiles per wave
// each): with one token block a workgroup is one layout block; with many (prefill steps) a
// workgroup takes several blocks of a one-tile-per-wave layout, so that each activation operand
// read from LDS feeds several MFMAs.
// ---------------------------------------------------------------------------------------------
// kScale: Fp8Scaling of the e4m3 operands: 0 tensor (the consumer or the epilogue applies
// scale(x_amax) * w_scale), 1 channel (the epilogue scales by x_scales[token] * w_scales[feature]),
// 2 block_128 (each 128-byte K step, one scale block, is accumulated scaled by
// x_scales(token, step) * w_scales(feature / 128, step)).
template <bool kFp8, GemmEpilogue kEpi, int TT, int F, int W, int P, int kBlocks = 1, int kOcc = 1,
          int kScale = 0>
__global__ __launch_bounds__(W * 64) __attribute__((amdgpu_waves_per_eu(kOcc)))
void gemm_kernel(const GemmArgs a) {
  static_assert(F % kBlocks == 0 && (kBlocks == 1 || kEpi != GemmEpilogue::gelu_gate),
                "blocks per workgroup");
  static_assert(kScale == 0 || kFp8, "scaled operands are e4m3");
  constexpr int FL = F / kBlocks;  // tiles per wave in the packed layout
  // Activation operand, one LDS stage per K step, filled by DMA (global_load_lds_dwordx4):
  //  - e4m3 weights: the prepared row-major operand (prepare_x_kernel), 1 B/element;
  //  - bf16 weights: the row-major bf16 X itself;
  //  either way the 128-byte slice of every token row that matches the weight step, its 16-byte
  //  chunks XOR-swizzled by the row index (chunk c of row t at position c ^ (t mod 8)), so one
  //  chunk of 16 consecutive rows spreads over distinct banks; the B operand is read from there
  //  directly.
  constexpr int kXRowBytes = 128;
  constexpr int kXChunks = kXRowBytes / 16;
  constexpr int kXStage = TT * 16 * kXRowBytes;   // = TT * kTileBytes for both operand kinds
  constexpr int kThreads = W * 64;
  // 1 KiB wave units of DMA per stage, spread round-robin over the waves; the last round's
  // surplus units repeat the final one (identical bytes to the same LDS address).
  constexpr int kXUnits = kXStage / 1024;
  constexpr int kXDma = (kXUnits + W - 1) / W;  // 16-byte DMA chunks per thread per step
  // block_128: each step also loads the lane's TT activation scales (contiguous), counted in the
  // in-order vector-memory stream, and the F weight-block scales of its tiles, whose addresses are
  // wave-uniform (scalar loads, outside that count; were they vector loads, the waits below would
  // only be stricter).
  constexpr int kXsVec = TT >= 4 ? 4 : TT;
  constexpr int kXsLoads = kScale == 2 ? TT / kXsVec : 0;
  constexpr int kLoadsPerStep = kXDma + 2 * F + kXsLoads;
  __shared__ __attribute__((aligned(16))) unsigned char lds[P * kXStage];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int group = lane >> 4;
  const int col = lane & 15;

  // Workgroup -> (feature block, K split, token block) on a one-dimensional grid. Workgroups go
  // to the 8 XCDs round-robin; the token blocks of one (feature block, split) take consecutive
  // slots of the same XCD, so that weight block streams from HBM about once and the other token
  // blocks re-read it from the XCD's L2. With one token block this is the plain feature-fastest
  // order.
  const int blocks_n = a.n / (16 * W * F);  // workgroup feature blocks (kBlocks layout blocks)
  const int m_blocks = (a.m + TT * 16 - 1) / (TT * 16);
  const int xslot = static_cast<int>(blockIdx.x) >> 3;
  const int wb = (xslot / m_blocks) * 8 + (static_cast<int>(blockIdx.x) & 7);
  if (wb >= blocks_n * a.k_splits) return;
  const int m_block = xslot % m_blocks;
  const int n_block = wb % blocks_n;
  const int split = wb / blocks_n;
  const int row_bytes = a.k * (kFp8 ? 1 : 2);
  const int total_steps = row_bytes / kStepBytes;
  const int steps = total_steps / a.k_splits;  // host guarantees an exact split
  const int step0 = split * steps;

  // This wave's tiles of the packed weight; feature0[f] is the first output feature of tile f.
  // gelu_gate: tiles [0, F/2) are gate rows, [F/2, F) the matching up rows of the packed
  // [gate | up] weight (cuda/ops.cu:264-270 packing).
  constexpr int kGroupBytes = W * FL * kTileBytes;  // one K step of one layout block
  // step-major weights: one K step of all layout blocks is contiguous
  const int layout_blocks = a.n / (16 * W * FL);
  const size_t step_stride = a.w_layout.step_major ? static_cast<size_t>(layout_blocks) * kGroupBytes
                                                   : static_cast<size_t>(kGroupBytes);
  const unsigned char *wrow[F];
  int feature0[F];
#pragma unroll
  for (int f = 0; f < F; ++f) {
    const int block = n_block * kBlocks + f / FL;  // layout block
    const int tile = wave * FL + f % FL;            // tile within the layout block
    if constexpr (kEpi == GemmEpilogue::gelu_gate) {
      constexpr int H = F / 2;
      feature0[f] = n_block * (16 * W * H) + (wave * H + (f % H)) * 16;
    } else {
      feature0[f] = block * (16 * W * FL) + tile * 16;
    }
    const size_t run = a.w_layout.step_major
                           ? static_cast<size_t>(step0) * layout_blocks + block
                           : static_cast<size_t>(block) * total_steps + step0;
    wrow[f] = static_cast<const unsigned char *>(a.w) + run * kGroupBytes + tile * kTileBytes + lane * 16;
  }
  // Weight scale row of tile f (gelu_gate: the up tiles are rows n/2 + feature0).
  auto scale_row = [&](int f) {
    if constexpr (kEpi == GemmEpilogue::gelu_gate) return f < F / 2 ? feature0[f] : a.n / 2 + feature0[f];
    else return feature0[f];
  };
  // This thread's DMA sources for stage chunk id = unit(i) * 64 + lane: row id / 8 of the
  // row-major activations (bf16 X, or the prepared e4m3 operand) at swizzled position id % 8
  // (rows past M re-read row M - 1; their outputs are never stored).
  auto xunit = [&](int i) { return min(i * W + wave, kXUnits - 1); };
  const unsigned char *xsrc[kXDma];
#pragma unroll
  for (int i = 0; i < kXDma; ++i) {
    const int id = xunit(i) * 64 + lane;
    const int row = id / kXChunks;
    const int chunk = (id % kXChunks) ^ (row % kXChunks);
    const int token = min(m_block * TT * 16 + row, a.m - 1);
    const unsigned char *row_base =
        kFp8 ? a.xprep + static_cast<size_t>(token) * row_bytes
             : reinterpret_cast<const unsigned char *>(a.x + static_cast<size_t>(token) * a.ldx);
    xsrc[i] = row_base + static_cast<size_t>(step0) * kXRowBytes + chunk * 16;
  }

  u32x4 wreg[P][F][2];
  float xsreg[P][kScale == 2 ? TT : 1];
  float wsreg[P][kScale == 2 ? F : 1];
  const float *xs_src = nullptr;
  // constant address space: wave-uniform addresses load through the scalar cache (reads only)
  typedef const __attribute__((address_space(4))) float *const_floats;
  const_floats ws_src[kScale == 2 ? F : 1];
  if constexpr (kScale == 2) {
    xs_src = a.x_scales + ((static_cast<size_t>(m_block) * total_steps + step0) * 16 + col) * TT;
#pragma unroll
    for (int f = 0; f < F; ++f)
      ws_src[f] = reinterpret_cast<const_floats>(reinterpret_cast<uintptr_t>(
          a.w_scales + static_cast<size_t>(scale_row(f) / 128) * a.w_scale_kblocks + step0));
  }
  v4f acc[F][TT];
#pragma unroll
  for (int f = 0; f < F; ++f)
#pragma unroll
    for (int j = 0; j < TT; ++j) acc[f][j] = v4f{0.f, 0.f, 0.f, 0.f};

  auto issue = [&](int step, int slot) {
    const int s = step < steps ? step : steps - 1;  // branch-free tail: repeat the last step
    unsigned char *stage = lds + slot * kXStage;
#pragma unroll
    for (int i = 0; i < kXDma; ++i)
      __builtin_amdgcn_global_load_lds(
          reinterpret_cast<const void *>(xsrc[i] + static_cast<size_t>(s) * kXRowBytes),
          reinterpret_cast<void __attribute__((address_space(3))) *>(
              reinterpret_cast<uintptr_t>(stage + xunit(i) * 1024)),
          16, 0, 0);
#pragma unroll
    for (int f = 0; f < F; ++f) {
      const unsigned char *src = wrow[f] + static_cast<size_t>(s) * step_stride;
      wreg[slot][f][0] = *reinterpret_cast<const u32x4 *>(src);
      wreg[slot][f][1] = *reinterpret_cast<const u32x4 *>(src + 1024);
    }
    if constexpr (kScale == 2) {
      const float *xs = xs_src + static_cast<size_t>(s) * 16 * TT;
#pragma unroll
      for (int i = 0; i < kXsLoads; ++i) {
        if constexpr (kXsVec == 4) {
          const v4f v = *reinterpret_cast<const v4f *>(xs + i * 4);
#pragma unroll
          for (int e = 0; e < 4; ++e) xsreg[slot][i * 4 + e] = v[e];
        } else {
          const float2 v = *reinterpret_cast<const float2 *>(xs + i * 2);
          xsreg[slot][i * 2] = v.x;
          xsreg[slot][i * 2 + 1] = v.y;
        }
      }
#pragma unroll
      for (int f = 0; f < F; ++f) wsreg[slot][f] = ws_src[f][s];
    }
  };

  auto mfma = [&](int slot, int f, int j, u32x4 b0, u32x4 b1) {
    const u32x4 a0 = wreg[slot][f][0];
    const u32x4 a1 = wreg[slot][f][1];
    if constexpr (kFp8) {
      const v8i av = {static_cast<int>(a0.x), static_cast<int>(a0.y), static_cast<int>(a0.z),
                      static_cast<int>(a0.w), static_cast<int>(a1.x), static_cast<int>(a1.y),
                      static_cast<int>(a1.z), static_cast<int>(a1.w)};
      const v8i bv = {static_cast<int>(b0.x), static_cast<int>(b0.y), static_cast<int>(b0.z),
                      static_cast<int>(b0.w), static_cast<int>(b1.x), static_cast<int>(b1.y),
                      static_cast<int>(b1.z), static_cast<int>(b1.w)};
      acc[f][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, acc[f][j], 0, 0, 0, 0,
                                                                  0, 0);
    } else {
      acc[f][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
          __builtin_bit_cast(v8bf, a0), __builtin_bit_cast(v8bf, b0), acc[f][j], 0, 0, 0);
      acc[f][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
          __builtin_bit_cast(v8bf, a1), __builtin_bit_cast(v8bf, b1), acc[f][j], 0, 0, 0);
    }
  };

  // Token tile j+1's B operand is read from LDS while tile j's MFMAs run (the scheduling
  // barriers keep the compiler from sinking the reads next to their use).
  // B operand of token tile j, half h, from the swizzled stage (row j*16+col, chunk h*4+group
  // of the 128-byte row slice).
  auto b_operand = [&](int slot, int j, int h) -> u32x4 {
    const int row = j * 16 + col;
    const int chunk = (h * 4 + group) ^ (row % kXChunks);
    return *reinterpret_cast<const u32x4 *>(lds + slot * kXStage + row * kXRowBytes + chunk * 16);
  };

  // block_128: one step's product of weight tile f and token tile j, unscaled (a fresh
  // accumulator); its scale xs(token, step) * ws(f, step) is applied one token tile later, so that
  // the multiply-adds of tile j - 1 run under tile j's MFMAs.
  auto mfma_block = [&](int slot, int f, u32x4 b0, u32x4 b1) -> v4f {
    const u32x4 a0 = wreg[slot][f][0];
    const u32x4 a1 = wreg[slot][f][1];
    const v8i av = {static_cast<int>(a0.x), static_cast<int>(a0.y), static_cast<int>(a0.z),
                    static_cast<int>(a0.w), static_cast<int>(a1.x), static_cast<int>(a1.y),
                    static_cast<int>(a1.z), static_cast<int>(a1.w)};
    const v8i bv = {static_cast<int>(b0.x), static_cast<int>(b0.y), static_cast<int>(b0.z),
                    static_cast<int>(b0.w), static_cast<int>(b1.x), static_cast<int>(b1.y),
                    static_cast<int>(b1.z), static_cast<int>(b1.w)};
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, v4f{0.f, 0.f, 0.f, 0.f}, 0, 0,
                                                           0, 0, 0, 0);
  };

  auto compute = [&](int slot) {
    u32x4 c0 = b_operand(slot, 0, 0);
    u32x4 c1 = b_operand(slot, 0, 1);
    v4f pending[kScale == 2 ? F : 1];
#pragma unroll
    for (int j = 0; j < TT; ++j) {
      u32x4 n0 = c0, n1 = c1;
      if (j + 1 < TT) {
        n0 = b_operand(slot, j + 1, 0);
        n1 = b_operand(slot, j + 1, 1);
      }
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (kScale == 2) {
        v4f current[F];
#pragma unroll
        for (int f = 0; f < F; ++f) current[f] = mfma_block(slot, f, c0, c1);
        if (j > 0) {
#pragma unroll
          for (int f = 0; f < F; ++f) {
            const float sc = xsreg[slot][j - 1] * wsreg[slot][f];
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[f][j - 1][e] += pending[f][e] * sc;
          }
        }
#pragma unroll
        for (int f = 0; f < F; ++f) pending[f] = current[f];
      } else {
#pragma unroll
        for (int f = 0; f < F; ++f) mfma(slot, f, j, c0, c1);
      }
      __builtin_amdgcn_sched_barrier(0);
      c0 = n0;
      c1 = n1;
    }
    if constexpr (kScale == 2) {
#pragma unroll
      for (int f = 0; f < F; ++f) {
        const float sc = xsreg[slot][TT - 1] * wsreg[slot][f];
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[f][TT - 1][e] += pending[f][e] * sc;
      }
    }
  };

  // The output scale's operands are loaded before the weight stream starts and reduced after it,
  // so their latency does not add to the kernel's tail.
  float x_amax_lane = 0.0f, w_scale = 1.0f;
  if constexpr (kFp8 && kScale == 0) {
    x_amax_lane = amax_lane(a.x_amax, a.amax_stripes);
    w_scale = *a.w_scale;
  }

  // prologue: steps 0 .. P-2
#pragma unroll
  for (int i = 0; i < P - 1; ++i) issue(i, i);
  const int rounds = (steps + P - 1) / P;
  for (int r = 0; r < rounds; ++r) {
#pragma unroll
    for (int i = 0; i < P; ++i) {
      const int s = r * P + i;
      // Step s landed for this wave (steps s+1 .. s+P-2 stay in flight); the bare barrier (no
      // fence: a fence would drain every outstanding load) makes it so for every wave, and frees
      // stage (s-1) % P, whose LDS reads all completed before their MFMAs.
      wait_vmcnt<(P - 2) * kLoadsPerStep>();
      __builtin_amdgcn_s_barrier();
      issue(s + P - 1, (i + P - 1) % P);
      if (s < steps) compute(i);
    }
  }

  float out_scale = 1.0f;
  if constexpr (kFp8 && kScale == 0) out_scale = fp8_scale_from_amax(wave_max(x_amax_lane)) * w_scale;
  // channel: the lane's token scales and its features' scales
  float ch_x[kScale == 1 ? TT : 1];
  v4f ch_w[kScale == 1 ? F : 1];
  if constexpr (kScale == 1) {
#pragma unroll
    for (int j = 0; j < TT; ++j)
      ch_x[j] = a.x_scales[min(m_block * TT * 16 + col + j * 16, a.m - 1)];
#pragma unroll
    for (int f = 0; f < F; ++f) ch_w[f] = *reinterpret_cast<const v4f *>(a.w_scales + scale_row(f) + group * 4);
  }
  // output scale of element e of acc[f][j]
  auto scale_of = [&](int f, int j, int e) -> float {
    if constexpr (kScale == 1) return ch_x[j] * ch_w[f][e];
    else if constexpr (kScale == 2) return 1.0f;
    else return out_scale;
  };

  // ------------------------------------------------------------------ epilogues
  // acc[f][j]: lane (col = token, group g) holds features feature0[f] + 4g + {0..3}.
  const int token_base = m_block * TT * 16 + col;
  if constexpr (kEpi == GemmEpilogue::partial_f32) {
#pragma unroll
    for (int j = 0; j < TT; ++j) {
      const int token = token_base + j * 16;
      if (token >= a.m) continue;
      float *dst = a.partial + (static_cast<size_t>(split) * a.m + token) * a.n;
#pragma unroll
      for (int f = 0; f < F; ++f) {
        v4f v = acc[f][j];
        if constexpr (kScale == 1) {
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] *= scale_of(f, j, e);
        }
        *reinterpret_cast<v4f *>(dst + feature0[f] + group * 4) = v;
      }
    }
  } else if constexpr (kEpi == GemmEpilogue::store_bf16) {
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < TT; ++j) {
      const int token = token_base + j * 16;
      if (token >= a.m) continue;
      bf16_t *dst = a.y + static_cast<size_t>(token) * a.ldy;
#pragma unroll
      for (int f = 0; f < F; ++f) {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = acc[f][j][e] * scale_of(f, j, e);
          amax = fmaxf(amax, fabsf(v[e]));
        }
        *reinterpret_cast<uint2 *>(dst + feature0[f] + group * 4) =
            uint2{f32x2_to_bf16x2(v[0], v[1]), f32x2_to_bf16x2(v[2], v[3])};
      }
    }
    if (a.y_amax != nullptr) {
      // Rounding is monotonic and symmetric, so the amax of the rounded outputs is the rounded
      // amax of the unrounded ones.
      amax = round_bf16(wave_max(amax));
      if (lane == 0) amax_publish(a.y_amax, a.amax_stripes, amax);
    }
  } else if constexpr (kEpi == GemmEpilogue::gelu_gate) {
    constexpr int H = F / 2;
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < TT; ++j) {
      const int token = token_base + j * 16;
      if (token >= a.m) continue;
      bf16_t *dst = a.y + static_cast<size_t>(token) * a.ldy;
#pragma unroll
      for (int f = 0; f < H; ++f) {
        float g[4], u[4], v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          g[e] = acc[f][j][e] * scale_of(f, j, e);
          u[e] = acc[f + H][j][e] * scale_of(f + H, j, e);
        }
        round_bf16x2(g[0], g[1]);
        round_bf16x2(g[2], g[3]);
        round_bf16x2(u[0], u[1]);
        round_bf16x2(u[2], u[3]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = gelu_tanh(g[e]) * u[e];
          amax = fmaxf(amax, fabsf(v[e]));
        }
        *reinterpret_cast<uint2 *>(dst + feature0[f] + group * 4) =
            uint2{f32x2_to_bf16x2(v[0], v[1]), f32x2_to_bf16x2(v[2], v[3])};
      }
    }
    if (a.y_amax != nullptr) {
      // amax of the rounded outputs = rounded amax (rounding is monotonic and symmetric)
      amax = round_bf16(wave_max(amax));
      if (lane == 0) amax_publish(a.y_amax, a.amax_stripes, amax);
    }
  } else {
    // argmax over bf16-rounded logits (cuda/linear.cu:735-737 writes bf16 logits; ops.cu:895-898
    // tie rule). One partial key per (workgroup, token); argmax_reduce_kernel finishes the row.
    __syncthreads();
    uint64_t *wave_keys = reinterpret_cast<uint64_t *>(lds);  // [W][TT*16]
#pragma unroll
    for (int j = 0; j < TT; ++j) {
      uint64_t best = kArgmaxInitialKey;
#pragma unroll
      for (int f = 0; f < F; ++f)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint64_t key = argmax_key(round_bf16(acc[f][j][e] * scale_of(f, j, e)),
                                          static_cast<uint32_t>(feature0[f] + group * 4 + e));
          best = key > best ? key : best;
        }
      uint64_t other = __shfl_xor(best, 16, kWave);
      best = other > best ? other : best;
      other = __shfl_xor(best, 32, kWave);
      best = other > best ? other : best;
      if (group == 0) wave_keys[wave * TT * 16 + j * 16 + col] = best;
    }
    __syncthreads();
    for (int t = threadIdx.x; t < TT * 16; t += kThreads) {
      uint64_t best = wave_keys[t];
#pragma unroll
      for (int w = 1; w < W; ++w) {
        const uint64_t other = wave_keys[w * TT * 16 + t];
        best = other > best ? other : best;
      }
      const int token = m_block * TT * 16 + t;
      if (token < a.m) a.argmax_partials[static_cast<size_t>(token) * blocks_n + n_block] = best;
    }
  }
}

// Row argmax reduction over the per-workgroup partial keys of one row.
__global__ __launch_bounds__(256) void argmax_reduce_kernel(const uint64_t *partials, int parts,
                                                            int32_t *out, int32_t *table,
                                                            int stride, int column) {
  const int row = blockIdx.x;
  uint64_t best = kArgmaxInitialKey;
  for (int i = threadIdx.x; i < parts; i += blockDim.x) {
    const uint64_t k = partials[static_cast<size_t>(row) * parts + i];
    best = k > best ? k : best;
  }
  best = wave_max_u64(best);
  __shared__ uint64_t wave_best[4];
  if ((threadIdx.x & 63) == 0) wave_best[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t b = wave_best[0];
    for (int w = 1; w < 4; ++w) b = wave_best[w] > b ? wave_best[w] : b;
    const int32_t index = static_cast<int32_t>(argmax_key_index(b));
    if (out != nullptr) out[row] = index;
    if (table != nullptr) table[row * stride + column] = index;
  }
}

// Pipeline depth per tiles-per-wave (measured on MI355X: 3 stages suffice from F = 2 on).
template <int F> constexpr int kStages = F == 1 ? 4 : 3;

template <bool kFp8, GemmEpilogue kEpi, int TT, int kS>
void launch_tiles(const GemmArgs &a, bool many, bool group4, dim3 grid, hipStream_t stream) {
  const int w = a.w_layout.waves;
  // one- and two-wave layouts (few-row weights) are built for one 32-row token block only
  if ((w == 1 || w == 2) && !(TT == 2 && kS == 0))
    throw std::runtime_error("a few-row weight layout serves at most 32 rows per call");
  // Many token blocks (prefill steps): the weights mostly come from L2, and two workgroups per CU
  // (two weight stages, <= 256 registers) keep the MFMAs fed while one of them waits.
  switch (a.w_layout.tiles_per_wave) {
  case 1:
    if constexpr (kEpi != GemmEpilogue::gelu_gate) {
      // (block_128 keeps one workgroup per CU: its per-step scale registers would spill at two)
      if constexpr (TT == 8 && kS != 2) {
        if (group4) {  // four one-tile layout blocks per workgroup
          if (w == 3) gemm_kernel<kFp8, kEpi, TT, 4, 3, 2, 4, 2, kS><<<grid, 192, 0, stream>>>(a);
          else gemm_kernel<kFp8, kEpi, TT, 4, 4, 2, 4, 2, kS><<<grid, 256, 0, stream>>>(a);
          return;
        }
      }
      if constexpr (TT == 2 && kS == 0) {  // few-row layouts (gemm_weight_layout few_rows)
        if (w == 1) { gemm_kernel<kFp8, kEpi, TT, 1, 1, kStages<1>, 1, 1, kS><<<grid, 64, 0, stream>>>(a); return; }
        if (w == 2) { gemm_kernel<kFp8, kEpi, TT, 1, 2, kStages<1>, 1, 1, kS><<<grid, 128, 0, stream>>>(a); return; }
      }
      if (w == 3) gemm_kernel<kFp8, kEpi, TT, 1, 3, kStages<1>, 1, 1, kS><<<grid, 192, 0, stream>>>(a);
      else gemm_kernel<kFp8, kEpi, TT, 1, 4, kStages<1>, 1, 1, kS><<<grid, 256, 0, stream>>>(a);
      return;
    }
    break;
  case 2:
    if constexpr (TT == 2 && kS == 0) {
      if (w == 1) { gemm_kernel<kFp8, kEpi, TT, 2, 1, kStages<2>, 1, 1, kS><<<grid, 64, 0, stream>>>(a); return; }
      if (w == 2) { gemm_kernel<kFp8, kEpi, TT, 2, 2, kStages<2>, 1, 1, kS><<<grid, 128, 0, stream>>>(a); return; }
    }
    if (w == 3) gemm_kernel<kFp8, kEpi, TT, 2, 3, kStages<2>, 1, 1, kS><<<grid, 192, 0, stream>>>(a);
    else gemm_kernel<kFp8, kEpi, TT, 2, 4, kStages<2>, 1, 1, kS><<<grid, 256, 0, stream>>>(a);
    return;
  case 4:
    if constexpr (TT == 8 && kS != 2) {
      if (many) {
        if (w == 3) gemm_kernel<kFp8, kEpi, TT, 4, 3, 2, 1, 2, kS><<<grid, 192, 0, stream>>>(a);
        else gemm_kernel<kFp8, kEpi, TT, 4, 4, 2, 1, 2, kS><<<grid, 256, 0, stream>>>(a);
        return;
      }
    }
    if (w == 3) gemm_kernel<kFp8, kEpi, TT, 4, 3, kStages<4>, 1, 1, kS><<<grid, 192, 0, stream>>>(a);
    else gemm_kernel<kFp8, kEpi, TT, 4, 4, kStages<4>, 1, 1, kS><<<grid, 256, 0, stream>>>(a);
    return;
  }
  throw std::runtime_error("unsupported weight layout for this GEMM");
}

template <bool kFp8, GemmEpilogue kEpi, int kS>
void launch_scaled(const GemmArgs &a, bool small_m, bool group4, dim3 grid, hipStream_t stream) {
  if (small_m)
    launch_tiles<kFp8, kEpi, 2, kS>(a, false, group4, grid, stream);
  else
    launch_tiles<kFp8, kEpi, 8, kS>(a, a.m > 8 * 16, group4, grid, stream);
}

template <bool kFp8, GemmEpilogue kEpi>
void launch_shape(const GemmArgs &a, bool small_m, bool group4, dim3 grid, hipStream_t stream) {
  if constexpr (kFp8) {
    if (a.scaling == 1) return launch_scaled<kFp8, kEpi, 1>(a, small_m, group4, grid, stream);
    if (a.scaling == 2) return launch_scaled<kFp8, kEpi, 2>(a, small_m, group4, grid, stream);
  }
  launch_scaled<kFp8, kEpi, 0>(a, small_m, group4, grid, stream);
}

template <bool kFp8>
void launch_gemm(const GemmArgs &a, hipStream_t stream) {
  if (a.x == nullptr || a.w == nullptr || a.m <= 0 || a.m > kGemmMaxRows || a.k <= 0 || a.n <= 0 ||
      a.k_splits <= 0 || a.ldx < a.k || (kFp8 && a.xprep == nullptr))
    throw std::runtime_error("invalid skinny GEMM shape");
  check_amax_stripes(a.amax_stripes);
  const int row_bytes = a.k * (kFp8 ? 1 : 2);
  if (row_bytes % kStepBytes != 0) throw std::runtime_error("GEMM K must fill 128-byte steps");
  if (a.ldx % 8 != 0) throw std::runtime_error("GEMM activation stride must be 16-byte aligned");
  if (a.scaling < 0 || a.scaling > 2 || (!kFp8 && a.scaling != 0))
    throw std::runtime_error("invalid FP8 scaling");
  if (kFp8 && a.scaling == 0 && (a.x_amax == nullptr || a.w_scale == nullptr))
    throw std::runtime_error("FP8 GEMM needs activation amax and weight scale");
  if (a.scaling != 0 && (a.w_scales == nullptr || a.x_scales == nullptr || a.xprep_ready))
    throw std::runtime_error("scaled FP8 GEMM needs weight and activation scale arrays");
  const int total_steps = row_bytes / kStepBytes;
  if (total_steps % a.k_splits != 0) throw std::runtime_error("GEMM split-K must divide K steps");
  const bool small_m = a.m <= 32;
  const int tt = gemm_token_tiles(a.m);
  const int tokens_per_block = tt * 16;
  const int m_blocks = (a.m + tokens_per_block - 1) / tokens_per_block;
  check_layout(a.w_layout);
  const bool gelu = a.epilogue == GemmEpilogue::gelu_gate;
  if (a.w_layout.n != a.n || a.w_layout.row_bytes != row_bytes || a.w_layout.gate_up != gelu)
    throw std::runtime_error("GEMM weight layout does not match the call");
  const int blocks_n = gemm_blocks_n(a.w_layout);
  switch (a.epilogue) {
  case GemmEpilogue::store_bf16:
  case GemmEpilogue::gelu_gate:
    if (a.y == nullptr || a.k_splits != 1) throw std::runtime_error("GEMM store needs y, 1 split");
    break;
  case GemmEpilogue::partial_f32:
    if (a.partial == nullptr) throw std::runtime_error("GEMM partial output missing");
    break;
  case GemmEpilogue::argmax:
    if (a.argmax_partials == nullptr || a.k_splits != 1 || (a.argmax_out == nullptr && !a.argmax_deferred))
      throw std::runtime_error("GEMM argmax needs partial keys, output, 1 split");
    if (static_cast<size_t>(blocks_n) * a.m > a.argmax_partial_capacity)
      throw std::runtime_error("GEMM argmax partial workspace too small");
    break;
  }
  if constexpr (kFp8) {
    const size_t chunks = static_cast<size_t>(total_steps) * tt * 128;
    if (chunks * 16 * m_blocks > a.xprep_capacity)
      throw std::runtime_error("GEMM activation workspace too small");
    const dim3 grid(static_cast<unsigned>((chunks + 255) / 256), m_blocks);
    if (a.scaling == 1) {
      if (static_cast<size_t>(m_blocks) * tokens_per_block > a.x_scales_capacity)
        throw std::runtime_error("GEMM activation scale workspace too small");
      prepare_x_rows_kernel<<<m_blocks * tokens_per_block, 256, 0, stream>>>(a.x, a.ldx, a.m, a.k,
                                                                            a.xprep, a.x_scales);
    } else if (a.scaling == 2) {
      if (static_cast<size_t>(m_blocks) * total_steps * tokens_per_block > a.x_scales_capacity)
        throw std::runtime_error("GEMM activation scale workspace too small");
      if (a.w_scale_kblocks < total_steps) throw std::runtime_error("GEMM weight block scales too few");
      const dim3 waves_grid(static_cast<unsigned>((total_steps * tt + 3) / 4), m_blocks);
      prepare_x_blocks_kernel<<<waves_grid, 256, 0, stream>>>(a.x, a.ldx, a.m, a.k, tt, a.xprep,
                                                             a.x_scales);
    } else if (!a.xprep_ready) {
prepare_x_kernel<<<grid, 256, 0, stream>>>(a.x, a.ldx, a.m, a.k, a.x_amax, a.amax_stripes, tt,
                                               a.xprep);
    }
  }
  // Several token blocks on a one-tile-per-wave layout: a workgroup takes four layout blocks,
  // so that its MFMAs per LDS operand read match the four-tile layouts (measured on MI355X at
  // 1024 rows: the one-tile workgroup is bound by its LDS operand reads).
  const bool group4 = m_blocks > 1 && a.scaling != 2 && a.w_layout.tiles_per_wave == 1 && blocks_n % 4 == 0 &&
                      (a.epilogue == GemmEpilogue::partial_f32 || a.epilogue == GemmEpilogue::store_bf16);
  const int wg_blocks = group4 ? blocks_n / 4 : blocks_n;
  const int64_t groups = (static_cast<int64_t>(wg_blocks) * a.k_splits + 7) / 8;
  const dim3 grid(static_cast<unsigned>(groups * 8 * m_blocks));
  if (a.timing_start != nullptr) hip_check(hipEventRecord(a.timing_start, stream), "record probe");
  switch (a.epilogue) {
  case GemmEpilogue::store_bf16:
    launch_shape<kFp8, GemmEpilogue::store_bf16>(a, small_m, group4, grid, stream);
    break;
  case GemmEpilogue::partial_f32:
    launch_shape<kFp8, GemmEpilogue::partial_f32>(a, small_m, group4, grid, stream);
    break;
  case GemmEpilogue::argmax:
    launch_shape<kFp8, GemmEpilogue::argmax>(a, small_m, group4, grid, stream);
    if (a.timing_stop != nullptr) hip_check(hipEventRecord(a.timing_stop, stream), "record probe");
    if (!a.argmax_deferred)
      argmax_reduce_kernel<<<a.m, 256, 0, stream>>>(a.argmax_partials, blocks_n, a.argmax_out,
                                                    a.argmax_table, a.argmax_table_stride,
                                                    a.argmax_table_column);
    break;
  case GemmEpilogue::gelu_gate:
    launch_shape<kFp8, GemmEpilogue::gelu_gate>(a, small_m, group4, grid, stream);
    break;
  }
  if (a.timing_stop != nullptr && a.epilogue != GemmEpilogue::argmax)
    hip_check(hipEventRecord(a.timing_stop, stream), "record probe");
  hip_check(hipGetLastError(), "launch skinny GEMM");
}

}  // namespace

WeightLayout gemm_weight_layout(int n, int row_bytes, bool gate_up, bool few_rows) {
  // The widest F (longest contiguous run per workgroup step) that still leaves >= 128
  // workgroups; measured on MI355X for the verify shapes (qkv 8192 and o/down 5376 rows take
  // F = 1, gate/up 43008 and the lm_head take F = 4). Gate/up weights feed the GELU epilogue,
  // which needs the whole K in one workgroup (no split-K): when 4-wave blocks leave CUs idle,
  // 3-wave blocks of the same F fill more of them (43008 rows: 224 workgroups instead of 168,
  // 51 us instead of 57 us per launch on MI355X).
  WeightLayout l;
  l.n = n;
  l.row_bytes = row_bytes;
  l.gate_up = gate_up;
  l.tiles_per_wave = gate_up ? 2 : 1;
  l.waves = 4;
  for (int f : {4, 2}) {
    if (n % (64 * f) == 0 && n / (64 * f) >= 128) {
      l.tiles_per_wave = f;
      break;
    }
  }
  if (n % (64 * l.tiles_per_wave) != 0) throw std::runtime_error("weight rows must fill 64-row tiles");
  const int unit = 16 * l.tiles_per_wave;  // rows per wave
  if (gate_up && n / (4 * unit) < 192 && n % (3 * unit) == 0 && n / (3 * unit) <= 256)
    l.waves = 3;
  // Split-K layouts: 3-wave blocks when 4-wave ones leave CUs idle after the split (o 5376 x
  // 4096: 224 workgroups instead of 168).
  if (!gate_up && l.tiles_per_wave == 1 && n % 48 == 0) {
    const int steps = row_bytes / 128;
    const int wg4 = (n / 64) * gemm_choose_splits(n / 64, steps);
    const int wg3 = (n / 48) * gemm_choose_splits(n / 48, steps);
    if (wg4 < 200 && wg3 > wg4 && wg3 <= 256) l.waves = 3;
  }
  // GEMMs of a few rows per call (the assistant's draft step, 24 rows) are latency-bound: when
  // the grid stays small, narrower workgroups (fewer waves, the same F) give more of them -- the
  // widest that reaches 240 workgroups with its split-K factor, else one wave.
  // Step-major storage: at any moment the workgroups stream one contiguous window of the weight
  // (the K step they are at) instead of 224-1024 runs a block's whole K range apart (measured on
  // MI355X, config-5 verify over four pairs of runners: 13.53 -> 13.18 ms median, every pair
  // faster; the GEMMs timed back to back alone do not change).
  l.step_major = true;
  if (few_rows) {
    const int steps = row_bytes / 128;
    auto workgroups = [&](int w) {
      const int blocks = n / (16 * w * l.tiles_per_wave);
      return gate_up ? blocks : blocks * gemm_choose_splits(blocks, steps);
    };
    if (workgroups(l.waves) < 240) {
      int pick = 1;
      for (int w = l.waves - 1; w >= 1; --w)
        if (n % (16 * w * l.tiles_per_wave) == 0 && workgroups(w) >= 240) {
          pick = w;
          break;
        }
      if (n % (16 * pick * l.tiles_per_wave) == 0) l.waves = pick;
    }
  }
  check_layout(l);
  return l;
}

int gemm_blocks_n(const WeightLayout &l) { return l.n / (16 * l.waves * l.tiles_per_wave); }

void pack_weight(const void *row_major, void *packed, const WeightLayout &layout,
                 hipStream_t stream) {
  launch_pack(row_major, packed, layout, true, stream);
}
void unpack_weight(const void *packed, void *row_major, const WeightLayout &layout,
                   hipStream_t stream) {
  launch_pack(packed, row_major, layout, false, stream);
}

size_t gemm_xprep_bytes(int m, int k) {
  const int tt = gemm_token_tiles(m);
  const int m_blocks = (m + tt * 16 - 1) / (tt * 16);
  return static_cast<size_t>(m_blocks) * (k / kStepBytes) * tt * kTileBytes;
}

size_t gemm_x_scale_floats(int m, int k) {
  const int tt = gemm_token_tiles(m);
  const int m_blocks = (m + tt * 16 - 1) / (tt * 16);
  return static_cast<size_t>(m_blocks) * tt * 16 * std::max(1, k / kStepBytes);
}

size_t gemm_argmax_partials(int m, const WeightLayout &layout) {
  return static_cast<size_t>(m) * gemm_blocks_n(layout);
}

int gemm_choose_splits(int n_blocks, int k_steps) {
  // The smallest divisor of k_steps that gives >= 240 workgroups (about one per CU), keeping
  // >= 12 steps per split so each weight stream outlasts its pipeline ramp; when none reaches
  // 240, the largest such divisor. Measured on MI355X: down 5376 x 21504 takes 3 splits, qkv
  // 8192 x 5376 and o 5376 x 4096 take 2.
  int best = 1;
  for (int s = 1; s <= k_steps; ++s) {
    if (k_steps % s != 0) continue;
    if (k_steps / s < 12) break;
    best = s;
    if (static_cast<long>(n_blocks) * s >= 240) break;
  }
  return best;
}

void launch_fp8_gemm(const GemmArgs &args, hipStream_t stream) { launch_gemm<true>(args, stream); }
void launch_bf16_gemm(const GemmArgs &args, hipStream_t stream) {
  launch_gemm<false>(args, stream);
}

}  // namespace carat_hip
