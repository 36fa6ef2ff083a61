// EXL3 dense linear for gfx950: decode kernel, fused small-M GEMV, output
// transform, and the C-ABI entry points exl3_linear_out / exl3_decode /
// exl3_linear_workspace_size.
//
// Small-M path (rows <= 8 per launch), two kernels:
//  1. gemv_kernel: one workgroup = 4 wavefronts = 32 output columns (two
//     tile columns) x a K range of up to 4*depth steps of 32 inputs.  It
//       a. issues all of its trellis loads first (dword loads; the 64 lanes
//          of a wavefront read two whole 16x16 tiles per tile row),
//       b. forms its activations meanwhile: t = H128(x * suh) for its K range
//          and every row, split into FP16 high and low parts at a per-row
//          power-of-two scale, stored in LDS in MFMA B-operand order,
//       c. decodes 16 trellis states per lane per step straight into MFMA
//          A-operand order and runs two v_mfma_f32_16x16x32_f16 per step,
//       d. reduces its four wavefronts through LDS in a fixed order and
//          writes one FP32 partial sum per (row, column).
//  2. gemv_output: sums the K-split partials in split order, applies the
//     output H128 and svh, rounds to the output dtype.
//
// Lane mapping.  The trellis' lane order is a 32-lane fragment order
// (encoder lane L holds tile rows {2q, 2q+1, 2q+8, 2q+9}, q = L & 3, of
// tile columns L >> 2 and (L >> 2) + 8).  MFMA lanes that share an A row
// sit 16 apart, so lane (g, m) = (lane >> 4, lane & 15) decodes encoder lane
// L = 4 * (m & 7) + g of tile column (m >> 3): its values 0-3 are A row m of
// the first MFMA (tile column m & 7 of that tile) and values 4-7 A row m of
// the second (tile column (m & 7) + 8), with k slots {2g, 2g+1, 2g+8, 2g+9}
// of two consecutive tile rows.  The activations are stored in LDS in the
// same k-slot order, so no lane shuffle of weights is ever needed.
#include <hip/hip_runtime.h>

#include <climits>
#include <string>

#include "../../include/vllm_mi355x.h"
#include "common.h"
#include "exl3_codec.h"

namespace exl3 {
namespace {

using vq::kBF16;
using vq::kFP16;
using vq::kFP32;

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kMaxGemvRows = 8;

// Formats the format admits (reference: csrc/exl3/gemm.cu:17-20,
// kernels/exl3/utils.py:283-285): even rates 1..8 bits for both codebooks,
// and 1.5 / 2.5 / 3.5 bits for mul1.
bool known_format(int64_t bits_x2, int64_t codebook) {
  if (codebook == 1) return bits_x2 >= 2 && bits_x2 <= 16 && bits_x2 % 2 == 0;
  if (codebook == 2) return bits_x2 >= 2 && bits_x2 <= 16 && (bits_x2 % 2 == 0 || bits_x2 <= 7);
  return false;
}

// Per-rate geometry of the small-M kernel.
template <int kBitsX2>
struct Gemv {
  static constexpr int kWords = LaneLoad<kBitsX2>::kWords;
  // steps (two tile rows each) each wavefront loads up front
  static constexpr int kDepth = 32 / (2 * kWords);
  static constexpr int kStepsPerGroup = 4 * kDepth;
};

int gemv_steps_per_group(int bits_x2) {
  switch (bits_x2) {
#define VQ_STEPS(B) case B: return Gemv<B>::kStepsPerGroup;
    VQ_STEPS(2) VQ_STEPS(3) VQ_STEPS(4) VQ_STEPS(5) VQ_STEPS(6) VQ_STEPS(7) VQ_STEPS(8)
    VQ_STEPS(10) VQ_STEPS(12) VQ_STEPS(14) VQ_STEPS(16)
#undef VQ_STEPS
  }
  return 16;
}

// Ring word `w` of a tile.
template <bool kAligned>
__device__ __forceinline__ uint32_t tile_word(const uint8_t* tile, int byte_offset) {
  if constexpr (kAligned) {
    return *reinterpret_cast<const uint32_t*>(tile + byte_offset);
  } else {
    const uint16_t* h = reinterpret_cast<const uint16_t*>(tile + byte_offset);
    return uint32_t(h[0]) | (uint32_t(h[1]) << 16);
  }
}

// Byte offsets (within a tile) of the words encoder lane L needs.
template <int kBitsX2>
__device__ __forceinline__ void lane_word_offsets(int L, int (&off)[Gemv<kBitsX2>::kWords]) {
  lane_word_index<kBitsX2>(L, off);
#pragma unroll
  for (int i = 0; i < Gemv<kBitsX2>::kWords; ++i) off[i] *= 4;
}

// ---- decode (inspection) kernel --------------------------------------------

template <int kBitsX2, int kCodebook, bool kAligned>
__global__ __launch_bounds__(kThreads) void decode_kernel(const uint8_t* __restrict__ trellis,
                                                          int64_t tiles_k, int64_t tiles_n,
                                                          uint16_t* __restrict__ out) {
  const int64_t gid = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  const int64_t tile = gid >> 5;
  if (tile >= tiles_k * tiles_n) return;
  const int L = int(gid & 31);
  const int64_t tr = tile / tiles_n;
  const int64_t tc = tile - tr * tiles_n;
  const uint8_t* src = trellis + tile * Ring<kBitsX2>::kTileBytes;
  int off[Gemv<kBitsX2>::kWords];
  lane_word_offsets<kBitsX2>(L, off);
  uint32_t words[Gemv<kBitsX2>::kWords];
#pragma unroll
  for (int i = 0; i < Gemv<kBitsX2>::kWords; ++i) words[i] = tile_word<kAligned>(src, off[i]);
  uint32_t pair[4];
  decode_words<kBitsX2, kCodebook>(L, words, pair);
  const int64_t cols = 16 * tiles_n;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint16_t v = uint16_t(pair[j >> 1] >> (16 * (j & 1)));
    const int64_t row = tr * 16 + 2 * (L & 3) + (j & 1) + 8 * ((j >> 1) & 1);
    const int64_t col = tc * 16 + (L >> 2) + 8 * (j >> 2);
    out[row * cols + col] = v;
  }
}

// ---- small-M kernel ----------------------------------------------------------

struct GemvArgs {
  const void* x;
  const uint16_t* suh;
  const uint8_t* trellis;
  float* partial;        // [splits][rows][np]
  int64_t logical_in;
  int64_t tiles_n;
  int64_t np;
  int x_dtype;
  int rows;              // 1..8
  int steps_total;       // padded_in / 32
  int steps_per_group;   // multiple of 4
};

// Power-of-two exponent e so that max * 2^e lies in [2^14, 2^15): the FP16
// high part then stays below 2^15 and the low part keeps ~11 more bits.
__device__ __forceinline__ int scale_exponent(uint32_t max_bits) {
  const int biased = int((max_bits >> 23) & 0xff);
  if (max_bits == 0u) return 0;
  const int e = 14 - (biased - 127);
  return e > 127 ? 127 : (e < -126 ? -126 : e);
}

// Float index, within the LDS activation block, of local input k of row r:
// the block is [step][g][row][8 slots] of FP32, later rewritten in place as
// [step][g][row][hi 8 halves | lo 8 halves] = [step][g][B column][8 halves].
__device__ __forceinline__ int act_index(int k, int r, int rows) {
  const int step = k >> 5;
  const int w = k & 31;
  const int tr = w >> 4;
  const int kk = w & 15;
  const int g = (kk & 7) >> 1;
  const int slot = 4 * tr + (kk & 1) + 2 * (kk >> 3);
  return ((step * 4 + g) * rows + r) * 8 + slot;
}

template <int kBitsX2, int kCodebook, bool kAligned>
__global__ __launch_bounds__(kThreads) void gemv_kernel(GemvArgs a) {
  using G = Gemv<kBitsX2>;
  using R = Ring<kBitsX2>;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ uint32_t row_max[kMaxGemvRows];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 4;
  const int m = lane & 15;
  const int L = 4 * (m & 7) + g;
  const int rows = a.rows;
  const int step0 = blockIdx.y * a.steps_per_group;
  const int nsteps = min(a.steps_per_group, a.steps_total - step0);
  const int per_wave = nsteps >> 2;

  // a. trellis loads of this wavefront's steps
  int off[G::kWords];
  lane_word_offsets<kBitsX2>(L, off);
  const int64_t row_bytes = a.tiles_n * R::kTileBytes;
  const uint8_t* column = a.trellis + (2 * int64_t(blockIdx.x) + (m >> 3)) * R::kTileBytes;
  uint32_t words[G::kDepth][2][G::kWords];
#pragma unroll
  for (int j = 0; j < G::kDepth; ++j) {
    if (j < per_wave) {
      const int64_t kt = 2 * int64_t(step0 + wave * per_wave + j);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint8_t* tile = column + (kt + h) * row_bytes;
#pragma unroll
        for (int i = 0; i < G::kWords; ++i) words[j][h][i] = tile_word<kAligned>(tile, off[i]);
      }
    }
  }

  // b. activations: t = H128(x * suh) over this group's K range, per row
  if (tid < kMaxGemvRows) row_max[tid] = 0u;
  __syncthreads();
  float* act = reinterpret_cast<float*>(smem);
  const int blocks = nsteps >> 2;
  const int64_t k0 = int64_t(step0) * 32;
  for (int task = wave; task < rows * blocks; task += 4) {
    const int r = task / blocks;
    const int b = task - r * blocks;
    const int kl0 = b * 128 + lane;
    const int kl1 = kl0 + 64;
    const int64_t kg0 = k0 + kl0;
    const int64_t kg1 = k0 + kl1;
    const int64_t xrow = int64_t(r) * a.logical_in;
    float v0 = kg0 < a.logical_in ? vq::load_act(a.x, a.x_dtype, xrow + kg0) * vq::f16_to_f32(a.suh[kg0]) : 0.0f;
    float v1 = kg1 < a.logical_in ? vq::load_act(a.x, a.x_dtype, xrow + kg1) * vq::f16_to_f32(a.suh[kg1]) : 0.0f;
    vq::h128_wave(v0, v1, lane);
    act[act_index(kl0, r, rows)] = v0;
    act[act_index(kl1, r, rows)] = v1;
    float mx = fmaxf(fabsf(v0), fabsf(v1));
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) mx = fmaxf(mx, __shfl_xor(mx, d));
    if (lane == 0) atomicMax(&row_max[r], __builtin_bit_cast(uint32_t, mx));
  }
  __syncthreads();
  const int chunks = nsteps * 4 * rows;
  for (int c = tid; c < chunks; c += kThreads) {
    const int e = scale_exponent(row_max[c % rows]);
    f32x4_t* p = reinterpret_cast<f32x4_t*>(act + c * 8);
    const f32x4_t v0 = p[0];
    const f32x4_t v1 = p[1];
    half8_t hi, lo;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float s = ldexpf(i < 4 ? v0[i] : v1[i - 4], e);
      const _Float16 h = _Float16(s);
      hi[i] = h;
      lo[i] = _Float16(s - float(h));
    }
    reinterpret_cast<half8_t*>(p)[0] = hi;
    reinterpret_cast<half8_t*>(p)[1] = lo;
  }
  __syncthreads();

  // c. decode + MFMA
  const int ncols = 2 * rows;
  f32x4_t acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
  f32x4_t acc2 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int j = 0; j < G::kDepth; ++j) {
    if (j < per_wave) {
      const int sl = wave * per_wave + j;
      uint32_t q0[4], q1[4];
      decode_words<kBitsX2, kCodebook>(L, words[j][0], q0);
      decode_words<kBitsX2, kCodebook>(L, words[j][1], q1);
      const u32x4_t a1 = {q0[0], q0[1], q1[0], q1[1]};
      const u32x4_t a2 = {q0[2], q0[3], q1[2], q1[3]};
      half8_t bop = {};
      if (m < ncols) bop = *reinterpret_cast<const half8_t*>(smem + ((sl * 4 + g) * ncols + m) * 16);
      acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, a1), bop, acc1, 0, 0, 0);
      acc2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, a2), bop, acc2, 0, 0, 0);
    }
  }

  // d. reduce the four wavefronts: red[wave][column 0..31][B column 0..15]
  __syncthreads();
  float* red = reinterpret_cast<float*>(smem);
  if (m < ncols) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 4 * g + i;
      const int col = (row & 7) + 16 * (row >> 3);
      red[(wave * 32 + col) * 16 + m] = acc1[i];
      red[(wave * 32 + col + 8) * 16 + m] = acc2[i];
    }
  }
  __syncthreads();
  for (int t = tid; t < 32 * rows; t += kThreads) {
    const int col = t & 31;
    const int r = t >> 5;
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      s += red[(w * 32 + col) * 16 + 2 * r] + red[(w * 32 + col) * 16 + 2 * r + 1];
    }
    a.partial[(int64_t(blockIdx.y) * rows + r) * a.np + 32 * int64_t(blockIdx.x) + col] =
        ldexpf(s, -scale_exponent(row_max[r]));
  }
}

// One wavefront per (row, 128-column block): sum the K-split partials in
// split order, H128, times svh, rounded to the output dtype.
__global__ __launch_bounds__(kThreads) void gemv_output(const float* __restrict__ partial, int splits,
                                                         int rows, int64_t np,
                                                         const uint16_t* __restrict__ svh,
                                                         int64_t logical_out, void* out, int out_dtype) {
  const int lane = threadIdx.x & 63;
  const int64_t task = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int64_t blocks = np / 128;
  if (task >= rows * blocks) return;
  const int64_t r = task / blocks;
  const int64_t c0 = (task - r * blocks) * 128 + lane;
  const int64_t c1 = c0 + 64;
  float v0 = 0.0f, v1 = 0.0f;
  for (int s = 0; s < splits; ++s) {
    const float* p = partial + (int64_t(s) * rows + r) * np;
    v0 += p[c0];
    v1 += p[c1];
  }
  vq::h128_wave(v0, v1, lane);
  if (c0 < logical_out) vq::store_act(out, out_dtype, r * logical_out + c0, v0 * vq::f16_to_f32(svh[c0]));
  if (c1 < logical_out) vq::store_act(out, out_dtype, r * logical_out + c1, v1 * vq::f16_to_f32(svh[c1]));
}

// ---- dispatch ----------------------------------------------------------------

template <int kBitsX2, int kCodebook>
int launch_format(bool aligned, const GemvArgs* gemv, dim3 grid, size_t lds, hipStream_t stream,
                  const uint8_t* trellis, int64_t tiles_k, int64_t tiles_n, uint16_t* decoded) {
  if (gemv) {
    if (aligned) {
      hipLaunchKernelGGL((gemv_kernel<kBitsX2, kCodebook, true>), grid, dim3(kThreads), lds, stream, *gemv);
    } else {
      hipLaunchKernelGGL((gemv_kernel<kBitsX2, kCodebook, false>), grid, dim3(kThreads), lds, stream, *gemv);
    }
    return vq::check_launch("exl3 gemv_kernel");
  }
  const int64_t threads = tiles_k * tiles_n * 32;
  const dim3 dgrid(unsigned((threads + kThreads - 1) / kThreads));
  if (aligned) {
    hipLaunchKernelGGL((decode_kernel<kBitsX2, kCodebook, true>), dgrid, dim3(kThreads), 0, stream,
                       trellis, tiles_k, tiles_n, decoded);
  } else {
    hipLaunchKernelGGL((decode_kernel<kBitsX2, kCodebook, false>), dgrid, dim3(kThreads), 0, stream,
                       trellis, tiles_k, tiles_n, decoded);
  }
  return vq::check_launch("exl3 decode_kernel");
}

int dispatch(int64_t bits_x2, int64_t codebook, bool aligned, const GemvArgs* gemv, dim3 grid,
             size_t lds, hipStream_t stream, const uint8_t* trellis, int64_t tiles_k,
             int64_t tiles_n, uint16_t* decoded) {
#define VQ_CASE(B, C)                                                                   \
  if (bits_x2 == B && codebook == C)                                                    \
    return launch_format<B, C>(aligned, gemv, grid, lds, stream, trellis, tiles_k, tiles_n, decoded);
  VQ_CASE(2, 1) VQ_CASE(4, 1) VQ_CASE(6, 1) VQ_CASE(8, 1)
  VQ_CASE(10, 1) VQ_CASE(12, 1) VQ_CASE(14, 1) VQ_CASE(16, 1)
  VQ_CASE(2, 2) VQ_CASE(3, 2) VQ_CASE(4, 2) VQ_CASE(5, 2) VQ_CASE(6, 2) VQ_CASE(7, 2)
  VQ_CASE(8, 2) VQ_CASE(10, 2) VQ_CASE(12, 2) VQ_CASE(14, 2) VQ_CASE(16, 2)
#undef VQ_CASE
  return vq::fail("Unsupported EXL3 rate/codebook combination");
}

int check_padded(int64_t n) {
  if (n <= 0 || n % 128 != 0 || n > INT_MAX) {
    return vq::fail("EXL3 padded dimensions must be positive H128 multiples fitting int32");
  }
  return vq::kOk;
}

int64_t gemv_splits(int64_t padded_in, int bits_x2) {
  const int64_t steps = padded_in / 32;
  const int64_t spg = gemv_steps_per_group(bits_x2);
  return (steps + spg - 1) / spg;
}

}  // namespace
}  // namespace exl3

extern "C" int64_t exl3_linear_workspace_size(int64_t max_rows, int64_t padded_in,
                                              int64_t padded_out) {
  if (max_rows < 0) {
    vq::fail("EXL3 max_rows must be nonnegative");
    return -1;
  }
  if (exl3::check_padded(padded_in) != vq::kOk || exl3::check_padded(padded_out) != vq::kOk) return -1;
  const int64_t small = max_rows < exl3::kMaxGemvRows ? max_rows : exl3::kMaxGemvRows;
  // K-split partials: at most ceil(padded_in / 512) splits (16 steps of 32
  // inputs per workgroup at the least).
  const int64_t splits = (padded_in + 511) / 512;
  return max_rows * (padded_in + padded_out) + small * splits * padded_out;
}

extern "C" int exl3_decode(const void* trellis, int64_t tiles_k, int64_t tiles_n,
                           int64_t trellis_words, int64_t bits_x2, int64_t codebook, void* out,
                           void* stream) {
  if (!trellis || !out) return vq::fail("EXL3 decode needs trellis and out buffers");
  if (trellis_words != 8 * bits_x2) return vq::fail("EXL3 packed word stride mismatch");
  if (tiles_k <= 0 || tiles_n <= 0) return vq::fail("EXL3 decode needs a nonempty trellis");
  if (!exl3::known_format(bits_x2, codebook)) {
    return vq::fail("Unsupported EXL3 rate/codebook combination");
  }
  const bool aligned = (reinterpret_cast<uintptr_t>(trellis) & 3) == 0;
  return exl3::dispatch(bits_x2, codebook, aligned, nullptr, dim3(), 0,
                        static_cast<hipStream_t>(stream), static_cast<const uint8_t*>(trellis),
                        tiles_k, tiles_n, static_cast<uint16_t*>(out));
}

extern "C" int exl3_linear_out(const void* x, int x_dtype, int64_t rows, int64_t x_cols,
                               const void* trellis, int64_t tiles_k, int64_t tiles_n,
                               int64_t trellis_words, const void* suh, int64_t suh_numel,
                               const void* svh, int64_t svh_numel, int64_t bits_x2,
                               int64_t codebook, int64_t logical_in, int64_t logical_out,
                               void* out, int out_dtype, int64_t out_rows, int64_t out_cols,
                               float* workspace, int64_t workspace_numel, void* stream) {
  using namespace vq;
  // Checks in the reference's order and wording (csrc/exl3/dense.cu:85-113).
  if (x_dtype != kBF16 && x_dtype != kFP16) return fail("x has incorrect dtype");
  if (out_dtype != kBF16 && out_dtype != kFP16 && out_dtype != kFP32) {
    return fail("EXL3 linear out must be BF16, FP16 or FP32");
  }
  if (trellis_words != 8 * bits_x2) return fail("EXL3 packed word stride mismatch");
  const int64_t padded_in = tiles_k * 16;
  const int64_t padded_out = tiles_n * 16;
  if (int rc = exl3::check_padded(padded_in)) return rc;
  if (int rc = exl3::check_padded(padded_out)) return rc;
  if (!(logical_in > 0 && logical_in <= padded_in && logical_out > 0 && logical_out <= padded_out)) {
    return fail("EXL3 logical dimensions must lie within the packed geometry");
  }
  if (!(x_cols == logical_in && out_rows == rows && out_cols == logical_out &&
        suh_numel == padded_in && svh_numel == padded_out)) {
    return fail("EXL3 linear input/output/scale geometry mismatch");
  }
  if (rows < 0 || rows > INT_MAX) return fail("EXL3 linear has too many rows");
  if (!exl3::known_format(bits_x2, codebook)) {
    return fail("Unsupported EXL3 rate/codebook combination");
  }
  const int64_t need = exl3_linear_workspace_size(rows, padded_in, padded_out);
  if (workspace_numel < need) return fail("EXL3 linear workspace is too small");
  if ((reinterpret_cast<uintptr_t>(workspace) & 15) != 0) {
    return fail("EXL3 linear workspace must be 16-byte aligned");
  }
  const int64_t x_bytes = rows * logical_in * dtype_bytes(x_dtype);
  const int64_t out_bytes = rows * logical_out * dtype_bytes(out_dtype);
  const int64_t ws_bytes = workspace_numel * 4;
  const int64_t tr_bytes = tiles_k * tiles_n * trellis_words * 2;
  const void* inputs[4] = {x, trellis, suh, svh};
  const int64_t input_bytes[4] = {x_bytes, tr_bytes, padded_in * 2, padded_out * 2};
  if (overlaps(out, out_bytes, workspace, ws_bytes)) {
    return fail("unsupported operation: some elements of the input tensor and the written-to "
                "tensor refer to a single memory location.");
  }
  for (int i = 0; i < 4; ++i) {
    if (overlaps(out, out_bytes, inputs[i], input_bytes[i]) ||
        overlaps(workspace, ws_bytes, inputs[i], input_bytes[i])) {
      return fail("unsupported operation: some elements of the input tensor and the written-to "
                  "tensor refer to a single memory location.");
    }
  }
  if (rows == 0) return kOk;

  const hipStream_t s = static_cast<hipStream_t>(stream);
  const bool aligned = (reinterpret_cast<uintptr_t>(trellis) & 3) == 0;
  const int steps_total = int(padded_in / 32);
  const int spg_max = exl3::gemv_steps_per_group(int(bits_x2));
  const int64_t splits0 = exl3::gemv_splits(padded_in, int(bits_x2));
  // Even split, rounded up to whole 128-input blocks (4 steps).
  int spg = int((steps_total + splits0 - 1) / splits0);
  spg = (spg + 3) / 4 * 4;
  if (spg > spg_max) spg = spg_max;
  const int64_t splits = (steps_total + spg - 1) / spg;
  if (splits > 65535) return fail("EXL3 linear K is too large");
  float* partial = workspace;
  for (int64_t r0 = 0; r0 < rows; r0 += exl3::kMaxGemvRows) {
    const int chunk = int(rows - r0 < exl3::kMaxGemvRows ? rows - r0 : exl3::kMaxGemvRows);
    exl3::GemvArgs a{};
    a.x = static_cast<const uint8_t*>(x) + r0 * logical_in * dtype_bytes(x_dtype);
    a.suh = static_cast<const uint16_t*>(suh);
    a.trellis = static_cast<const uint8_t*>(trellis);
    a.partial = partial;
    a.logical_in = logical_in;
    a.tiles_n = tiles_n;
    a.np = padded_out;
    a.x_dtype = x_dtype;
    a.rows = chunk;
    a.steps_total = steps_total;
    a.steps_per_group = spg;
    const dim3 grid(unsigned(padded_out / 32), unsigned(splits));
    size_t lds = size_t(spg) * 4 * chunk * 32;
    if (lds < 4 * 32 * 16 * 4) lds = 4 * 32 * 16 * 4;
    if (int rc = exl3::dispatch(bits_x2, codebook, aligned, &a, grid, lds, s, nullptr, 0, 0, nullptr)) {
      return rc;
    }
    const int64_t tasks = chunk * (padded_out / 128);
    hipLaunchKernelGGL(exl3::gemv_output, dim3(unsigned((tasks + 3) / 4)), dim3(exl3::kThreads), 0, s,
                       partial, int(splits), chunk, padded_out, static_cast<const uint16_t*>(svh),
                       logical_out,
                       static_cast<uint8_t*>(out) + r0 * logical_out * dtype_bytes(out_dtype),
                       out_dtype);
    if (int rc = check_launch("exl3 gemv_output")) return rc;
  }
  return kOk;
}
