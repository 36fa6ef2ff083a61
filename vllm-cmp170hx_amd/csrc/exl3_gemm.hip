// EXL3 dense linear for many rows (prefill), gfx950.
//
// Two launches on the caller's stream, where the reference's operator has
// three (csrc/exl3/dense.cu:115-148: linear_input, GEMM, linear_output); the
// GEMM runs on the matrix cores and applies the output transform itself:
//  1. prefill_input: one workgroup per row forms t = H128(x * suh) over the
//     whole row, picks a per-row power-of-two scale from the row maximum, and
//     writes t as FP16 high and low parts (t * 2^e = hi + lo, ~22 bits), in
//     the k order of the MFMA operands: within every 32-input step, group g
//     (8 halves) holds inputs {2g, 2g+1, 2g+8, 2g+9} of its two 16-input tile
//     rows.  Row r: [high: padded_in halves][low: padded_in halves]; the
//     low parts are written unless the GEMM reads the high parts alone.
//  2. the GEMM:
//     * a 16-byte aligned trellis: tile_gemm (exl3_tile.h), weights decoded
//       in registers straight into MFMA B operands, 128 x 256 tiles, on the
//       high and low parts (the default) or, under
//       exl3_set_tile_precision(1), the high parts alone (each rotated input
//       rounded once to FP16);
//     * other trellis bases: prefill_gemm, 256 x 256
//       output tiles, 16 wavefronts, four per SIMD (8 along M x 2 along N,
//       32 x 128 each = 1 x 4 v_mfma_f32_32x32x16_f16 tiles).  Per K step of
//       32 inputs the workgroup decodes the 32 x 256 weight slab (32 trellis
//       tiles, one encoder lane per thread) straight into LDS as W^T [n][k]
//       in FP16 (exact values, k in the activations' order) and stages the
//       activation tiles; every wavefront accumulates hi * W and lo * W into
//       one FP32 accumulator.  The slab and tiles are double-buffered: step
//       s + 1 is decoded and staged while the MFMAs of step s run (one
//       barrier a step), with its trellis words and activations loaded two
//       steps ahead.
//     Both epilogues unscale each row (2^-e) and apply the output transform:
//     H128 over each 128-column block, times svh, rounded to the output dtype.
//
// Workspace (FP32 elements): rows x padded_in floats holding the FP16 rows
// above, and one int row exponent per row after them.
#include <hip/hip_runtime.h>

#include <atomic>
#include <climits>
#include <type_traits>

#include "common.h"
#include "exl3_codec.h"
#include "exl3_internal.h"
#include "exl3_tile.h"

namespace exl3 {
namespace {

constexpr int kBM = 256;            // rows per workgroup
constexpr int kBN = 256;            // columns per workgroup
constexpr int kBK = 32;             // inputs per K step (two tile rows)
constexpr int kGemmThreads = 1024;  // 16 wavefronts, four per SIMD
constexpr int kWaves = kGemmThreads / 64;
constexpr int kBandsM = kWaves / 2;   // wavefronts along M (two 128-column bands along N)
constexpr int kMT = kBM / kBandsM / 32;                       // 32-row MFMA tiles per wavefront
constexpr int kTasks = 1024 / kGemmThreads;                   // decode tasks per thread (32 tiles x 32 lanes)
constexpr int kStageVecs = kBM * 32 * 2 / 16 / kGemmThreads;  // 16-byte activation vectors per thread and tile
static_assert(kMT >= 1 && kTasks >= 1 && kStageVecs >= 1, "workgroup shape");
constexpr int kLdsK = kBK + 8;      // LDS row stride in halves (80 bytes)

// ---- 1. activations ----------------------------------------------------------

// One workgroup (256 threads) per row.  A wavefront forms four 128-input
// blocks at a time (group G: blocks 4 G .. 4 G + 3, one per 16-lane row,
// eight consecutive inputs a lane, H128 in registers and DPP); wavefront w
// takes groups w, w + 4, ..., the first kCache of them kept in registers.
// Pass 1 finds the row maximum of |t|, pass 2 writes the scaled high parts
// (and the low parts when `lo`: the GEMM reads them) as dword pairs; groups past the register cache are formed again
// (the same operations, so the same values).  Inputs past logical_in form
// +0, as the reference's zero padding.
// Half offset of input k within its 32-input step, in the operand order.
__device__ __forceinline__ int64_t operand_order(int64_t k) {
  const int w = int(k & 31);
  const int g = (w & 7) >> 1;
  const int slot = 4 * (w >> 4) + (w & 1) + 2 * ((w >> 3) & 1);
  return (k & ~int64_t(31)) + g * 8 + slot;
}

template <int kCache>
__global__ __launch_bounds__(256) void prefill_input(const void* __restrict__ x, int x_dtype,
                                                     int64_t logical_in, int64_t padded_in,
                                                     const uint16_t* __restrict__ suh,
                                                     _Float16* __restrict__ act,
                                                     int* __restrict__ row_exp, bool lo) {
  __shared__ uint32_t row_max;
  const int64_t r = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int q = lane >> 4;  // the lane's block within a group
  const int l = lane & 15;  // its eight inputs within the block: 8 l ..
  const int64_t blocks = padded_in / 128;
  const int64_t groups = (blocks + 3) / 4;
  const uint16_t* xs = static_cast<const uint16_t*>(x) + r * logical_in;
  if (threadIdx.x == 0) row_max = 0u;
  __syncthreads();
  // the first input of the lane's eight in group G (clamped to the last block)
  auto first_k = [&](int64_t G) { return min(4 * G + q, blocks - 1) * 128 + 8 * l; };
  // eight 16-bit values p[k0 .. k0 + 7]: one 16-byte load where all are
  // inside len and the address allows it, else one load each (0 past len)
  auto load8 = [&](const uint16_t* p, int64_t k0, int64_t len, uint16_t (&h)[8]) {
    if (k0 + 8 <= len && (reinterpret_cast<uintptr_t>(p + k0) & 15) == 0) {
      const u32x4_t w = *reinterpret_cast<const u32x4_t*>(p + k0);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t word = w[j >> 1];
        h[j] = uint16_t(word >> (16 * (j & 1)));
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) h[j] = k0 + j < len ? p[k0 + j] : uint16_t(0);
    }
  };
  auto form = [&](int64_t G, float (&v)[8]) {
    const int64_t k0 = first_k(G);
    uint16_t xh[8], sh[8];
    load8(xs, k0, logical_in, xh);
    load8(suh, k0, padded_in, sh);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      v[j] = k0 + j < logical_in ? u16_act(xh[j], x_dtype) * vq::f16_to_f32(sh[j]) : 0.0f;
    }
    vq::h128_rows(v, l);
  };
  auto live = [&](int64_t G) { return 4 * G + q < blocks; };
  float mx = 0.0f;
  float c[kCache][8];
#pragma unroll
  for (int i = 0; i < kCache; ++i) form(min(int64_t(wave + 4 * i), groups - 1), c[i]);
#pragma unroll
  for (int i = 0; i < kCache; ++i) {
    if (wave + 4 * i < groups && live(wave + 4 * i)) {
#pragma unroll
      for (int j = 0; j < 8; ++j) mx = fmaxf(mx, fabsf(c[i][j]));
    }
  }
  for (int64_t G = wave + 4 * kCache; G < groups; G += 4) {
    float v[8];
    form(G, v);
    if (live(G)) {
#pragma unroll
      for (int j = 0; j < 8; ++j) mx = fmaxf(mx, fabsf(v[j]));
    }
  }
  mx = vq::wave_max(mx, lane);
  if (lane == 0) atomicMax(&row_max, __builtin_bit_cast(uint32_t, mx));
  __syncthreads();
  const int e = scale_exponent(row_max);
  if (threadIdx.x == 0) row_exp[r] = e;
  _Float16* h = act + r * 2 * padded_in;
  // inputs k0 + 2 i, k0 + 2 i + 1 are adjacent halves of the operand order
  // at (k0 & ~31) + 8 i + 4 ((k0 >> 4) & 1) + 2 ((k0 >> 3) & 1)
  auto store8 = [&](int64_t k0, const float (&v)[8]) {
    const int64_t base = (k0 & ~int64_t(31)) + 4 * ((k0 >> 4) & 1) + 2 * ((k0 >> 3) & 1);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float t0 = ldexpf(v[2 * i], e);
      const float t1 = ldexpf(v[2 * i + 1], e);
      const _Float16 h0 = _Float16(t0), h1 = _Float16(t1);
      const uint32_t hw = uint32_t(__builtin_bit_cast(uint16_t, h0)) | (uint32_t(__builtin_bit_cast(uint16_t, h1)) << 16);
      *reinterpret_cast<uint32_t*>(h + base + 8 * i) = hw;
      if (lo) {
        const _Float16 l0 = _Float16(t0 - float(h0)), l1 = _Float16(t1 - float(h1));
        const uint32_t lw = uint32_t(__builtin_bit_cast(uint16_t, l0)) | (uint32_t(__builtin_bit_cast(uint16_t, l1)) << 16);
        *reinterpret_cast<uint32_t*>(h + padded_in + base + 8 * i) = lw;
      }
    }
  };
#pragma unroll
  for (int i = 0; i < kCache; ++i) {
    if (wave + 4 * i < groups && live(wave + 4 * i)) store8(first_k(wave + 4 * i), c[i]);
  }
  for (int64_t G = wave + 4 * kCache; G < groups; G += 4) {
    float v[8];
    form(G, v);
    if (live(G)) store8(first_k(G), v);
  }
}

// ---- 2. decode-to-LDS MFMA GEMM -------------------------------------------------

struct PrefillArgs {
  const _Float16* act;    // [rows][high kp | low kp], operand order
  const int* row_exp;     // [rows]
  const uint8_t* trellis;
  const uint16_t* svh;    // [np]
  void* out;              // [rows][logical_out]
  int64_t rows;
  int64_t kp;
  int64_t np;
  int64_t tiles_n;
  int64_t logical_out;
  int out_dtype;
};

template <int kBitsX2, int kCodebook, bool kAligned>
__global__ __launch_bounds__(kGemmThreads) void prefill_gemm(PrefillArgs a) {
  using R = Ring<kBitsX2>;
  constexpr int kWords = LaneLoad<kBitsX2>::kWords;
  // two buffers of: the W^T slab [n][k] and the two activation tiles [m][k],
  // FP16, 80-byte rows.  Step s+1 is decoded and staged into one buffer while
  // the MFMAs of step s read the other: one barrier per step.
  __shared__ __attribute__((aligned(16))) _Float16 w_lds[2][kBN * kLdsK];
  __shared__ __attribute__((aligned(16))) _Float16 hi_lds[2][kBM * kLdsK];
  __shared__ __attribute__((aligned(16))) _Float16 lo_lds[2][kBM * kLdsK];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave % kBandsM;     // row band of kMT 32-row tiles
  const int wn = wave / kBandsM;     // 128-column band
  const int64_t row0 = int64_t(blockIdx.x) * kBM;
  const int64_t col0 = int64_t(blockIdx.y) * kBN;
  const int64_t tile_col0 = col0 / 16;
  const int steps = int(a.kp / kBK);

  // activation staging: thread t copies 16-byte vectors t + kGemmThreads v of
  // each tile (row = vector / 4, halves 8 (vector % 4) ..)
  int st_off[kStageVecs];
  const _Float16* hi_src[kStageVecs];
  const _Float16* lo_src[kStageVecs];
#pragma unroll
  for (int v = 0; v < kStageVecs; ++v) {
    const int vec = tid + kGemmThreads * v;
    st_off[v] = (vec >> 2) * kLdsK + 8 * (vec & 3);
    const int64_t src_row = min(row0 + (vec >> 2), a.rows - 1);
    hi_src[v] = a.act + src_row * 2 * a.kp + 8 * (vec & 3);
    lo_src[v] = hi_src[v] + a.kp;
  }

  // decode tasks: (tile row tr, tile column tc, encoder lane L), kTasks per thread
  int task_tr[kTasks], task_tc[kTasks], task_l[kTasks], off[kTasks][kWords];
  bool task_on[kTasks];
  const uint8_t* task_src[kTasks];
#pragma unroll
  for (int i = 0; i < kTasks; ++i) {
    const int task = tid + kGemmThreads * i;
    const int tile = task >> 5;
    task_tr[i] = tile >> 4;
    task_tc[i] = tile & 15;
    task_l[i] = task & 31;
    task_on[i] = tile_col0 + task_tc[i] < a.tiles_n;
    int idx[kWords];
    lane_word_index<kBitsX2>(task_l[i], idx);
#pragma unroll
    for (int w = 0; w < kWords; ++w) off[i][w] = 4 * idx[w];
    const int64_t tc = task_on[i] ? tile_col0 + task_tc[i] : 0;  // absent tiles read tile 0
    task_src[i] = a.trellis + (int64_t(task_tr[i]) * a.tiles_n + tc) * R::kTileBytes;
  }
  const int64_t step_bytes = 2 * a.tiles_n * R::kTileBytes;  // two tile rows

  f32x16_t acc[kMT][4];
#pragma unroll
  for (int i = 0; i < kMT; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16_t{};

  // two register slots of fetched step data: slot s & 1 holds step s, loaded
  // two steps before it is decoded
  uint32_t words[2][kTasks][kWords];
  u32x4_t hv[2][kStageVecs], lv[2][kStageVecs];
  auto fetch = [&](int slot, int step) {
#pragma unroll
    for (int i = 0; i < kTasks; ++i)
#pragma unroll
      for (int w = 0; w < kWords; ++w)
        words[slot][i][w] = tile_word<kAligned>(task_src[i] + step * step_bytes, off[i][w]);
#pragma unroll
    for (int v = 0; v < kStageVecs; ++v) {
      hv[slot][v] = *reinterpret_cast<const u32x4_t*>(hi_src[v] + int64_t(step) * kBK);
      lv[slot][v] = *reinterpret_cast<const u32x4_t*>(lo_src[v] + int64_t(step) * kBK);
    }
  };
  // decode task i of the step in register slot `slot` into W buffer `buf`
  auto decode_task = [&](int slot, int buf, int i) {
    uint32_t pair[4];
    decode_words<kBitsX2, kCodebook>(task_l[i], words[slot][i], pair);
    if (!task_on[i]) pair[0] = pair[1] = pair[2] = pair[3] = 0u;
    const int L = task_l[i];
    // values 0-3 (tile rows 2q, 2q+1, 2q+8, 2q+9 of column n) sit at operand
    // positions 8q + 4h .. + 3 of the step (h = tile row in the step), values
    // 4-7 the same of column n + 8: one 8-byte store each
    const int kb = 8 * (L & 3) + 4 * task_tr[i];
    const int n = task_tc[i] * 16 + (L >> 2);
    _Float16* w = w_lds[buf];
    *reinterpret_cast<uint64_t*>(w + n * kLdsK + kb) = uint64_t(pair[0]) | (uint64_t(pair[1]) << 32);
    *reinterpret_cast<uint64_t*>(w + (n + 8) * kLdsK + kb) = uint64_t(pair[2]) | (uint64_t(pair[3]) << 32);
  };
  auto stage = [&](int slot, int buf) {
#pragma unroll
    for (int v = 0; v < kStageVecs; ++v) {
      *reinterpret_cast<u32x4_t*>(hi_lds[buf] + st_off[v]) = hv[slot][v];
      *reinterpret_cast<u32x4_t*>(lo_lds[buf] + st_off[v]) = lv[slot][v];
    }
  };
  // the MFMAs of one k16 chunk of buffer `buf`: A = activations (rows l % 32,
  // k 8 (l / 32) + i), B = W (k 8 (l / 32) + i, columns l % 32)
  auto mfma_chunk = [&](int buf, int kc) {
    const int ko = kc * 16 + 8 * (lane >> 5);
    half8_t ah[kMT], al[kMT], b[4];
#pragma unroll
    for (int i = 0; i < kMT; ++i) {
      const int m = wm * 32 * kMT + i * 32 + (lane & 31);
      ah[i] = *reinterpret_cast<const half8_t*>(hi_lds[buf] + m * kLdsK + ko);
      al[i] = *reinterpret_cast<const half8_t*>(lo_lds[buf] + m * kLdsK + ko);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = wn * 128 + j * 32 + (lane & 31);
      b[j] = *reinterpret_cast<const half8_t*>(w_lds[buf] + n * kLdsK + ko);
    }
#pragma unroll
    for (int i = 0; i < kMT; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i], b[j], acc[i][j], 0, 0, 0);
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i], b[j], acc[i][j], 0, 0, 0);
      }
  };

  // prologue: steps 0 and 1 in flight, step 0 decoded and staged into buffer 0.
  // Every fetch is issued unconditionally (past the last step it reloads the
  // last one): a load a branch may skip leaves the compiler unsure of the
  // loads in flight, and it then waits for more of them than a step needs.
  const int last = steps - 1;
  fetch(0, 0);
  fetch(1, min(1, last));
#pragma unroll
  for (int i = 0; i < kTasks; ++i) decode_task(0, 0, i);
  stage(0, 0);
  fetch(0, min(2, last));
  __syncthreads();
  // step s: the MFMAs of buffer s & 1, interleaved with the decode and staging
  // of step s + 1 (register slot (s + 1) & 1) into the other buffer, then the
  // fetch of step s + 3 into the slot just decoded.  Steps run in pairs so the
  // buffer and slot indices are constants (registers cannot be indexed).
  //   The body has no branch: steps is a multiple of 4 (kp of whole
  //   128-input blocks), and after the last step the decode and staging of
  //   the clamped step land in the buffer no MFMA reads again.  (A branch
  //   here leaves the compiler unsure of the loads in flight where the paths
  //   meet, and it then waits for the prefetch of the step after as well.)
  auto iteration = [&](int step, int buf) {
    const int nslot = buf ^ 1;
    mfma_chunk(buf, 0);
    decode_task(nslot, buf ^ 1, 0);
    mfma_chunk(buf, 1);
#pragma unroll
    for (int i = 1; i < kTasks; ++i) decode_task(nslot, buf ^ 1, i);
    stage(nslot, buf ^ 1);
    fetch(nslot, min(step + 3, last));
    __syncthreads();
  };
  for (int step = 0; step < steps; step += 2) {
    iteration(step, 0);
    iteration(step + 1, 1);
  }

  // epilogue, the output transform fused: lane l, register r of tile (i, j)
  // is row 8 (r / 4) + 4 (l / 32) + r % 4, column 32 j + l % 32 of the
  // wavefront's 128-column band, which is one H128 block.  Per row: unscale
  // (2^-e), H128 (butterfly distances 1..16 across the 32 lanes of the row's
  // half-wavefront, 32 and 64 across the four registers j, in that order, as
  // the standalone transform), times svh, rounded to the output dtype.
  const int64_t band = col0 + wn * 128;
#pragma unroll
  for (int i = 0; i < kMT; ++i) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t row = row0 + wm * 32 * kMT + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
      const int e = a.row_exp[row < a.rows ? row : a.rows - 1];
      float v[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = ldexpf(acc[i][j][r], -e);
      // partner +- v as partner + v * (+-1): one FMA, exact product
      auto lane_stage = [&](auto d_tag) {
        constexpr int d = decltype(d_tag)::value;
        const float sgn = (lane & d) != 0 ? -1.0f : 1.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float o = vq::xor_lanes<d>(v[j], lane);
          v[j] = __builtin_fmaf(v[j], sgn, o);
        }
      };
      lane_stage(std::integral_constant<int, 1>{});
      lane_stage(std::integral_constant<int, 2>{});
      lane_stage(std::integral_constant<int, 4>{});
      lane_stage(std::integral_constant<int, 8>{});
      lane_stage(std::integral_constant<int, 16>{});
      // distance 32 (registers j, j ^ 1), then 64 (j, j ^ 2) with the scale
      float w[4];
      w[0] = v[0] + v[1];
      w[1] = v[0] - v[1];
      w[2] = v[2] + v[3];
      w[3] = v[2] - v[3];
      v[0] = (w[0] + w[2]) * vq::kH128Scale;
      v[2] = (w[0] - w[2]) * vq::kH128Scale;
      v[1] = (w[1] + w[3]) * vq::kH128Scale;
      v[3] = (w[1] - w[3]) * vq::kH128Scale;
      if (row < a.rows) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int64_t col = band + j * 32 + (lane & 31);
          if (col < a.logical_out) {
            vq::store_act(a.out, a.out_dtype, row * a.logical_out + col, v[j] * vq::f16_to_f32(a.svh[col]));
          }
        }
      }
    }
  }
}

template <int kBitsX2, int kCodebook>
int launch_gemm(bool aligned, const PrefillArgs& a, hipStream_t stream) {
  const dim3 grid(unsigned((a.rows + kBM - 1) / kBM), unsigned((a.np + kBN - 1) / kBN));
  if (aligned) {
    hipLaunchKernelGGL((prefill_gemm<kBitsX2, kCodebook, true>), grid, dim3(kGemmThreads), 0, stream, a);
  } else {
    hipLaunchKernelGGL((prefill_gemm<kBitsX2, kCodebook, false>), grid, dim3(kGemmThreads), 0, stream, a);
  }
  return vq::check_launch("exl3 prefill_gemm");
}

}  // namespace

int launch_tile_gemm(int64_t bits_x2, int64_t codebook, bool moe, bool lo, const TileArgs& a, dim3 grid,
                     hipStream_t stream) {
  const int index = format_index(int(bits_x2), int(codebook));
  if (index < 0 || !known_format(bits_x2, codebook) || !tile_rate(bits_x2)) {
    return vq::fail("Unsupported EXL3 rate/codebook combination");
  }
  switch (index % kTileParts) {
#define VQ_PART(P) \
  case P: return tile_launch_part<P>(bits_x2, codebook, moe, lo, a, grid, stream);
    VQ_PART(0) VQ_PART(1) VQ_PART(2) VQ_PART(3)
#undef VQ_PART
  }
  return vq::fail("Unsupported EXL3 rate/codebook combination");
}

namespace {

// exl3_set_tile_precision / exl3_set_prefill_kernel
std::atomic<int> g_tile_fp16_only{0};
std::atomic<int> g_prefill_kernel{0};

}  // namespace

bool tile_fp16_only() { return g_tile_fp16_only.load() != 0; }

int prefill_linear(const void* x, int x_dtype, int64_t rows, const uint8_t* trellis,
                   int64_t tiles_k, int64_t tiles_n, const uint16_t* suh, const uint16_t* svh,
                   int bits_x2, int codebook, int64_t logical_in, int64_t logical_out, void* out,
                   int out_dtype, float* workspace, hipStream_t stream) {
  const int64_t kp = tiles_k * 16;
  const int64_t np = tiles_n * 16;
  if (rows > 65535 * int64_t(kTileRows)) return vq::fail("EXL3 linear has too many rows");
  _Float16* act = reinterpret_cast<_Float16*>(workspace);
  int* row_exp = reinterpret_cast<int*>(workspace + rows * kp);
  // the tile GEMM: a 16-byte aligned trellis (LDS-DMA), 32-bit buffer
  // offsets over the matrix and the activations; under
  // exl3_set_tile_precision(1) it reads the activations' high parts alone
  const uintptr_t base = reinterpret_cast<uintptr_t>(trellis);
  const int forced = g_prefill_kernel.load();
  const bool tile = forced != 1 && tile_rate(bits_x2) && (base & 15) == 0 &&
                    tiles_k * tiles_n * 16 * bits_x2 <= INT_MAX && rows * 4 * kp <= INT_MAX;
  const bool tile_lo = !tile_fp16_only();
  const bool lo = !tile || tile_lo;
  {
    // the register cache sized to the 4-block groups a wavefront forms
    const int64_t per_wave = ((kp / 128 + 3) / 4 + 3) / 4;
    const dim3 grid{unsigned(rows)};
    if (per_wave <= 1) {
      hipLaunchKernelGGL(prefill_input<1>, grid, dim3(256), 0, stream, x, x_dtype, logical_in, kp, suh, act, row_exp, lo);
    } else if (per_wave <= 2) {
      hipLaunchKernelGGL(prefill_input<2>, grid, dim3(256), 0, stream, x, x_dtype, logical_in, kp, suh, act, row_exp, lo);
    } else {
      hipLaunchKernelGGL(prefill_input<4>, grid, dim3(256), 0, stream, x, x_dtype, logical_in, kp, suh, act, row_exp, lo);
    }
  }
  if (int rc = vq::check_launch("exl3 prefill_input")) return rc;
  if (tile) {
    TileArgs t{};
    t.act = reinterpret_cast<const uint8_t*>(act);
    t.act_row_bytes = 4 * kp;
    t.act_rows = rows;
    t.row_exp = row_exp;
    t.exp_stride = 1;
    t.kp = kp;
    t.np = np;
    t.trellis = trellis;
    t.svh = svh;
    t.tiles_n = tiles_n;
    t.rows = rows;
    t.out = out;
    t.out_dtype = out_dtype;
    t.logical_out = logical_out;
    const dim3 grid(unsigned((np + kTileCols - 1) / kTileCols), unsigned((rows + kTileRows - 1) / kTileRows));
    return launch_tile_gemm(bits_x2, codebook, false, tile_lo, t, grid, stream);
  }
  PrefillArgs a{act, row_exp, trellis, svh, out, rows, kp, np, tiles_n, logical_out, out_dtype};
  const bool aligned = (base & 3) == 0;
  int rc = vq::kOk;
  bool done = false;
#define VQ_CASE(B, C)                                        \
  if (!done && bits_x2 == B && codebook == C) {               \
    rc = launch_gemm<B, C>(aligned, a, stream);               \
    done = true;                                              \
  }
  VQ_EXL3_FORMATS(VQ_CASE)
#undef VQ_CASE
  if (!done) return vq::fail("Unsupported EXL3 rate/codebook combination");
  return rc;
}

}  // namespace exl3

extern "C" int exl3_set_tile_precision(int fp16_only) {
  if (fp16_only != 0 && fp16_only != 1) return vq::fail("EXL3 tile precision must be 0 (high and low parts) or 1 (FP16)");
  exl3::g_tile_fp16_only.store(fp16_only);
  return vq::kOk;
}

extern "C" int exl3_set_prefill_kernel(int kernel) {
  if (kernel < 0 || kernel > 2) return vq::fail("EXL3 prefill kernel must be 0 (automatic), 1 or 2");
  exl3::g_prefill_kernel.store(kernel);
  return vq::kOk;
}
