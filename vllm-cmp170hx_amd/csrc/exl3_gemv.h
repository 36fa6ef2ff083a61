// EXL3 small-M GEMV kernels for gfx950: the inspection decode kernel and
// the fused small-M GEMV, as templates over the format (bits_x2, codebook).
// The templates are instantiated by exl3_gemv_part.hip, compiled once per
// part of the format list (each part a few formats, built in parallel);
// exl3_linear.hip holds the host side and reaches a format through
// gemv_launch_part<P>.
//
// Small-M path (rows <= 8 per launch), two kernels:
//  1. gemv_kernel: one workgroup = 4 wavefronts = 128 output columns (one
//     H128 block) x 128 inputs (one H128 block, 4 steps of 32).  Wavefront w
//     owns two tile columns (32 outputs) over the whole range.  It
//       a. loads its activations, then issues all of its trellis loads
//          (one coalesced dword per lane per tile row: every trellis byte
//          is fetched once, in whole cache lines),
//       b. wavefront w forms rows w, w + 4: t = H128(x * suh) of the block,
//          stored in LDS, in MFMA B-operand order, as FP16 high and low
//          parts at a per-row power-of-two scale,
//       c. gathers each decoding lane's ring words with ds_bpermute, decodes
//          16 trellis states per lane per step straight into MFMA A-operand
//          order and runs two v_mfma_f32_16x16x32_f16 per step,
//       d. writes one FP32 partial sum per (K split, row, column).
//  2. gemv_output (exl3_linear.hip): sums the K-split partials in split
//     order, applies the output H128 and svh, rounds to the output dtype.
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
#pragma once

#include <hip/hip_runtime.h>

#include <climits>

#include "common.h"
#include "exl3_codec.h"
#include "exl3_internal.h"

namespace exl3 {

using vq::kBF16;
using vq::kFP16;
using vq::kFP32;


constexpr int kThreads = 256;
constexpr int kMaxGemvRows = 8;
// Calls of up to this many rows run the small-M kernel in chunks of
// kMaxGemvRows (each chunk streams the matrix once); the prefill GEMM's
// 256-row tiles only pay off above it.
constexpr int kGemvChunkedRows = 32;

// Per-rate geometry of the small-M kernel.
//
// A wavefront's two tiles of one tile row (its "chunk") are 32 * bits_x2
// contiguous bytes.  Three ways to bring them in:
//  * kLoadLds (16-byte aligned trellis, the fast path): buffer_load_dwordx4
//    ... lds copies whole chunks straight into a per-wavefront LDS ring, one
//    kilobyte (kStepsPerLoad steps of two tile rows) per instruction, with
//    the tile row in the scalar offset.  Decoding lanes then read their ring
//    words with ds_read_b32 at immediate offsets.  No VGPR staging, so deep
//    prefetch costs no registers.
//  * kLoadDword (4-byte aligned): up to 4 bits per weight each lane loads
//    one dword of the chunk (coalesced) and decoding lanes gather their ring
//    words with ds_bpermute; wider rates load each lane's window words.
//  * kLoadHalf (2-byte aligned): as kLoadDword, two halfword loads a word.
constexpr int kLoadHalf = 0;
constexpr int kLoadDword = 1;
constexpr int kLoadLds = 2;

template <int kBitsX2>
struct Gemv {
  static constexpr bool kCoalesced = kBitsX2 <= 8;
  static constexpr int kWords = LaneLoad<kBitsX2>::kWords;
  // registers each lane loads per tile row (two tiles)
  static constexpr int kRaw = kCoalesced ? 1 : 2 * kWords;
  // steps of loads each wavefront keeps in flight
  static constexpr int kDepth = 32 / (2 * kRaw);
  // LDS stream: bytes of one chunk, lanes loading one chunk (16 bytes each),
  // steps (two tile rows) per 1 KB load, loads kept in flight
  static constexpr int kChunk = 32 * kBitsX2;
  static constexpr int kChunkLanes = kChunk / 16;
  static constexpr int kStepsPerLoad = kBitsX2 <= 4 ? 4 : (kBitsX2 <= 8 ? 2 : 1);
  static constexpr int kStepsInFlight = 8;
};

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
  const uint16_t* svh;
  const uint8_t* trellis;
  float* partial;        // [splits][rows][np]
  void* out;             // [rows][out_stride], this launch's first column
  uint32_t* counters;    // the arrival-counter pool (device address)
  int counter_base;      // fused finish: first arrival-counter slot, or -1
  int64_t logical_in;
  int64_t logical_out;   // valid output columns from this launch's first
  int64_t out_stride;    // elements between output rows
  int64_t tiles_n;       // tile columns of a whole trellis row (its stride)
  int64_t np;            // columns of this launch (128 per workgroup column)
  int x_dtype;
  int out_dtype;
  int rows;              // 1..8
  int splits;            // K splits (padded_in / 128)
};

// Arrival counters of the fused finish: the pool of exl3_internal.h, one
// slot per 128-column block of a launch.

// Four consecutive partial sums at byte offset `offset` of buffer `r`,
// written through to the device-coherent level (cache policy sc1, that of an
// agent-scope store), so a workgroup on another XCD reads them after the
// arrival counter says they are complete.  A builtin rather than inline
// assembly: the compiler must see the 16-byte store to keep the VALU off its
// data registers for the cycle after it issues.
__device__ __forceinline__ void store_agent_x4(__amdgpu_buffer_rsrc_t r, int offset, f32x4_t v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), r, offset, 0, kCachePolicySc1);
}

// A partial sum: agent-scope (bypassing caches that may hold another
// call's data) in the fused finish, plain in the separate output kernel.
template <bool kCoherent>
__device__ __forceinline__ float load_partial(const float* p) {
  if constexpr (kCoherent) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    return *p;
  }
}

// Row r of one 128-column output block (the separate output kernel): lane l
// sums columns l and l + 64 over the K splits (32 loads in flight), then
// H128, times svh, rounded to the output dtype.
template <bool kCoherent>
__device__ __forceinline__ void finish_row_block(const float* __restrict__ partial, int splits,
                                                 int rows, int64_t np, int64_t r, int64_t base,
                                                 const uint16_t* __restrict__ svh,
                                                 int64_t logical_out, int64_t out_stride, void* out,
                                                 int out_dtype, int lane) {
  const int64_t c0 = base + lane;
  const int64_t c1 = c0 + 64;
  const uint32_t scale0 = svh[c0];
  const uint32_t scale1 = svh[c1];
  const float* p = partial + r * np;
  const int64_t stride = int64_t(rows) * np;
  // even splits, then odd splits, each in order, then even + odd: the same
  // additions as the fused finish
  float e0 = 0.0f, e1 = 0.0f, o0 = 0.0f, o1 = 0.0f;
  for (int s = 0; s < splits; s += 16) {
    float a0[16], a1[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const bool in = s + u < splits;
      a0[u] = in ? load_partial<kCoherent>(p + int64_t(s + u) * stride + c0) : 0.0f;
      a1[u] = in ? load_partial<kCoherent>(p + int64_t(s + u) * stride + c1) : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < 16; u += 2) {
      if (s + u < splits) {
        e0 += a0[u];
        e1 += a1[u];
      }
      if (s + u + 1 < splits) {
        o0 += a0[u + 1];
        o1 += a1[u + 1];
      }
    }
  }
  float v0 = e0 + o0, v1 = e1 + o1;
  vq::h128_wave(v0, v1, lane);
  if (c0 < logical_out) vq::store_act(out, out_dtype, r * out_stride + c0, v0 * vq::f16_to_f32(uint16_t(scale0)));
  if (c1 < logical_out) vq::store_act(out, out_dtype, r * out_stride + c1, v1 * vq::f16_to_f32(uint16_t(scale1)));
}

// Fused finish of one 128-column block by the first 256 threads of the
// workgroup (the others only pass its barrier): each column is summed over
// the even splits and over the odd splits, each in split order (agent-scope
// loads), the two parity sums are added (even + odd) through LDS, then
// wavefront w applies H128 and svh to rows w, w + 4.
__device__ __forceinline__ void finish_block(const GemvArgs& a, float* red, int tid, int cblk) {
  const int col = tid & 127;
  const int part = vq::uniform(tid >> 7);   // the split's scalar offset
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t base = 128 * int64_t(cblk);
  // buffer over this column block's partials of every split (the split in
  // the scalar offset): one VGPR per load in flight
  const int stride_bytes = 4 * a.rows * int(a.np);
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      a.partial + base, 0, (a.splits - 1) * stride_bytes + 4 * ((a.rows - 1) * int(a.np) + 128), 0x00020000);
  if (a.splits <= 16 && tid < 256) {
    // thread = (4 columns, split parity, row group): one 16-byte load per
    // split of its parity (index clamped to a valid split, the extra terms
    // not added), all in flight together: one memory round trip per row of
    // its group (rows rg, rg + 4)
    const int cq = tid & 31;
    const int par = (tid >> 5) & 1;  // differs inside a wavefront: offsets in VGPRs
    for (int r = tid >> 6; r < a.rows; r += 4) {
      f32x4_t t[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int split_off = min(par + 2 * u, a.splits - 1) * stride_bytes;
        t[u] = __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                               rsrc, split_off + 4 * (r * int(a.np) + 4 * cq), 0, kCachePolicySc1));
      }
      // (float vectors throughout: this compiler's __builtin_bit_cast of a
      // vector element reads element 0 whatever the index)
      f32x4_t v = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        if (par + 2 * u < a.splits) v += t[u];
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) red[(par * a.rows + r) * 128 + 4 * cq + c] = v[c];
    }
  } else if (a.splits <= 32 && tid < 256) {
    // one round of 16 loads per row (the split index clamped to a valid one,
    // the extra terms not added), the next row's loads issued before this
    // row's sum: rows one memory round trip apart in the pipeline, not one
    // round trip each
    auto load_row = [&](int r, float (&t)[16]) {
      const int voff = 4 * (r * int(a.np) + col);
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int sp = min(part + 2 * u, a.splits - 1);
        t[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsrc, voff, sp * stride_bytes,
                                                                              kCachePolicySc1));
      }
    };
    auto sum_row = [&](int r, const float (&t)[16]) {
      float v = 0.0f;
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        if (part + 2 * u < a.splits) v += t[u];
      }
      red[(part * a.rows + r) * 128 + col] = v;
    };
    float ta[16], tb[16];
    load_row(0, ta);
    for (int r = 0; r < a.rows; r += 2) {
      load_row(min(r + 1, a.rows - 1), tb);
      sum_row(r, ta);
      if (r + 1 < a.rows) {
        load_row(min(r + 2, a.rows - 1), ta);
        sum_row(r + 1, tb);
      }
    }
  }
  for (int r = 0; a.splits > 32 && r < a.rows && tid < 256; ++r) {
    const int voff = 4 * (r * int(a.np) + col);
    float v = 0.0f;
    // 16 loads in flight (32 splits) per round, split order
    for (int s = part; s < a.splits; s += 32) {
      float t[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        t[u] = s + 2 * u < a.splits
                   ? __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                   rsrc, voff, (s + 2 * u) * stride_bytes, kCachePolicySc1))
                   : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        if (s + 2 * u < a.splits) v += t[u];
      }
    }
    red[(part * a.rows + r) * 128 + col] = v;
  }
  __syncthreads();
  // svh loaded before the first output store (a load waited for after a
  // store also waits for the store: loads and stores share one counter)
  const int64_t c0 = base + lane;
  const int64_t c1 = c0 + 64;
  const float svh0 = vq::f16_to_f32(a.svh[c0]);
  const float svh1 = vq::f16_to_f32(a.svh[c1]);
  for (int r = wave; r < a.rows && wave < 4; r += 4) {
    float v0 = red[r * 128 + lane] + red[(a.rows + r) * 128 + lane];
    float v1 = red[r * 128 + lane + 64] + red[(a.rows + r) * 128 + lane + 64];
    vq::h128_wave(v0, v1, lane);
    void* out = a.out;
    if (c0 < a.logical_out) vq::store_act(out, a.out_dtype, r * a.out_stride + c0, v0 * svh0);
    if (c1 < a.logical_out) vq::store_act(out, a.out_dtype, r * a.out_stride + c1, v1 * svh1);
  }
}

using vq::wait_lgkmcnt0;
using vq::wait_vmcnt;

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// One workgroup = kGroups groups of 4 wavefronts = 128 output columns (one
// H128 block) x kGroups * kBlocks 128-input blocks.  Group q takes the
// kBlocks blocks (4 steps of 32 inputs each) from q * kBlocks on; the host
// picks kGroups * kBlocks dividing the input blocks, so every workgroup's
// range is whole.  Wavefront w of a group owns the column pair
// 4 * blockIdx.x + w (two tile columns, 32 outputs) over the group's range
// and streams its trellis chunks (kLoad: see Gemv).  The groups' sums meet in
// LDS (in group order), so a workgroup writes one partial sum per column.
//
// The grid is (column block, K split): consecutive workgroups read adjacent
// kilobytes of the same tile rows (DRAM page locality).
//
// kRows (1, 2, 4 or 8) is the row count the kernel is built for; a call with
// fewer rows (a.rows) computes its last row in the padding rows, which are
// never stored.
template <int kBitsX2, int kCodebook, int kLoad, int kRows, int kBlocks, int kGroups>
__global__ __launch_bounds__(kThreads * kGroups) void gemv_kernel(GemvArgs a) {
  using G = Gemv<kBitsX2>;
  using R = Ring<kBitsX2>;
  constexpr bool kLds = kLoad == kLoadLds;
  constexpr bool kAligned = kLoad != kLoadHalf;
  constexpr int kSteps = 4 * kBlocks;
  constexpr int kDepth = G::kDepth < kSteps ? G::kDepth : kSteps;
  constexpr int kCols = 2 * kRows;                        // B columns: hi, lo per row
  constexpr int kActHalves = kSteps * 4 * kCols * 8;      // B operands of the range
  constexpr int kTasks = kBlocks * kRows;                 // (block, row) forming tasks
  constexpr int kFormTasks = (kTasks + 3) / 4;            // per wavefront
  // 8-row kernels over pairs of blocks form four tasks a wavefront at a
  // time, one per 16-lane row, eight inputs a lane (h128_rows: the same
  // additions in the same order as h128_wave, so the same operands): pass p
  // of wavefront w is block 2 p + w / 2, rows 4 (w & 1) .. + 3
  constexpr bool kRowForm = kRows == 8 && kGroups == 1 && kBlocks % 2 == 0;
  constexpr int kPasses = kRowForm ? kBlocks / 2 : 1;
  // LDS stream: loads of the range, loads in flight per wavefront
  constexpr int kP = G::kStepsPerLoad;
  constexpr int kLoads = kSteps / kP;
  constexpr int kRingWant = G::kStepsInFlight / kP < 4 ? G::kStepsInFlight / kP : 4;
  constexpr int kRingLoads = kLds ? (kRingWant < kLoads ? kRingWant : kLoads) : 1;
  // Rotated loading order of the 4-bit chunk (dword loads, see below).
  constexpr bool kRotate = kBitsX2 == 8 && !kLds;
  static_assert(kSteps % kP == 0, "whole loads per range");
  static_assert(kGroups == 1 || (kLds && kRingLoads >= 2), "groups meet in two ring slots");
  // activations in B-operand order, per group.  Reused by the fused finish
  // for its row sums.
  constexpr int kActAll = kGroups * kActHalves;
  __shared__ __attribute__((aligned(16))) _Float16 act[kActAll > 2 * 128 * kRows * 2 ? kActAll : 2 * 128 * kRows * 2];
  // per (block, row) maxima of the formed activations: a group scales its
  // rows by one power of two across its blocks, so the MFMA sums run over the
  // whole range and fold once
  __shared__ uint32_t block_max[kGroups][kBlocks][kRows];
  // LDS stream: kRingLoads slots of 1 KB (kP steps) per wavefront, one
  // array per slot: the compiler's wait for an LDS-DMA load before a read
  // of its data then names that load, not every load in flight.
  constexpr int kSlotWords = kLds ? 4 * kGroups * 256 : 4;
  __shared__ __attribute__((aligned(16))) uint32_t ring0[kSlotWords];
  __shared__ __attribute__((aligned(16))) uint32_t ring1[kRingLoads > 1 ? kSlotWords : 4];
  __shared__ __attribute__((aligned(16))) uint32_t ring2[kRingLoads > 2 ? kSlotWords : 4];
  __shared__ __attribute__((aligned(16))) uint32_t ring3[kRingLoads > 3 ? kSlotWords : 4];
  static_assert(kRingLoads <= 4, "four ring slots");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // in the workgroup
  const int grp = wave >> 2;
  const int wc = wave & 3;                                       // column pair in the block
  const int g = lane >> 4;
  const int m = lane & 15;
  const int L = 4 * (m & 7) + g;
  const int cblk = blockIdx.x;
  const int split = blockIdx.y;
  const int block0 = (split * kGroups + grp) * kBlocks;
  const int64_t k0 = int64_t(block0) * 128;

  // a. activation loads first (they must not queue behind the trellis).
  //    Forming task t = wave + 4f is (block t / kRows, row t % kRows); lane l
  //    holds elements l and l + 64 of the block.  Every load is
  //    unconditional, at a clamped (always valid) index, and the value is
  //    selected afterwards: loads under a branch would each wait for their
  //    data before the branch closes.
  //    Buffer loads: 32-bit offsets, and a load past the resource's end (an
  //    input at or past logical_in) returns zero, the reference's padding.
  //    A wavefront's forming tasks lie in one row of x (kRows divides by
  //    the four wavefronts' task stride, or a task's row is wc % kRows).
  const uint16_t* xs = static_cast<const uint16_t*>(a.x);
  const __amdgpu_buffer_rsrc_t suh_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(a.suh), 0, int(2 * a.logical_in), 0x00020000);
  //    8-row kernels whose input rows are whole 16-byte chunks (logical_in
  //    a multiple of 8, x and suh 16-byte aligned) take the row form: a
  //    lane's eight inputs, all below logical_in or all past it (zeros), in
  //    one 16-byte load each of x and suh.  (Eight 2-byte loads a lane, each
  //    spread over four rows, were slower than the per-task form, which the
  //    others keep.)
  const bool row_form = kRowForm && (a.logical_in & 7) == 0 &&
                        ((reinterpret_cast<uintptr_t>(a.x) | reinterpret_cast<uintptr_t>(a.suh)) & 15) == 0;
  uint32_t xv[kFormTasks][2], sv[kFormTasks][2];
  u32x4_t xq[kPasses], sq[kPasses];  // row form: a lane's eight inputs of each pass
  const int rl = lane & 15;          // row form: the lane's place in its 16-lane row
  if (row_form) {
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
      const int b = 2 * p + (wc >> 1);
      const int row = min(4 * (wc & 1) + (lane >> 4), a.rows - 1);
      const __amdgpu_buffer_rsrc_t x_rsrc = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<uint16_t*>(xs + int64_t(row) * a.logical_in), 0, int(2 * a.logical_in), 0x00020000);
      const int k_0 = int(k0) + 128 * b + 8 * rl;
      sq[p] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(suh_rsrc, 2 * k_0, 0, 0));
      xq[p] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(x_rsrc, 2 * k_0, 0, 0));
    }
  }
#pragma unroll
  for (int f = 0; f < kFormTasks && !row_form; ++f) {
    const int t = wc + 4 * f;
    const int b = min(t / kRows, kBlocks - 1);
    const int row = vq::uniform(min(t % kRows, a.rows - 1));
    const __amdgpu_buffer_rsrc_t x_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(xs + int64_t(row) * a.logical_in), 0, int(2 * a.logical_in), 0x00020000);
    const int k_0 = int(k0) + 128 * b + lane;
    sv[f][0] = __builtin_amdgcn_raw_buffer_load_b16(suh_rsrc, 2 * k_0, 0, 0);
    sv[f][1] = __builtin_amdgcn_raw_buffer_load_b16(suh_rsrc, 2 * k_0 + 128, 0, 0);
    xv[f][0] = __builtin_amdgcn_raw_buffer_load_b16(x_rsrc, 2 * k_0, 0, 0);
    xv[f][1] = __builtin_amdgcn_raw_buffer_load_b16(x_rsrc, 2 * k_0 + 128, 0, 0);
  }

  // b. the first trellis loads.  The wavefront's chunk of tile row 0 is the
  //    base of a buffer resource, the tile row a scalar offset.
  int off[G::kWords];
  lane_word_offsets<kBitsX2>(L, off);
  const int row_bytes = int(a.tiles_n) * R::kTileBytes;
  const uint8_t* chunk = a.trellis + 2 * (4 * int64_t(cblk) + wc) * R::kTileBytes +
                         8 * int64_t(block0) * row_bytes;
  const __amdgpu_buffer_rsrc_t trellis_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(chunk), 0, (8 * kBlocks - 1) * row_bytes + 2 * R::kTileBytes, 0x00020000);
  const int tile_off = (m >> 3) * R::kTileBytes;

  //    LDS stream: load i (steps kP*i ..) fills ring slot i % kRingLoads of
  //    this wavefront: lane l copies 16 bytes, part l % kChunkLanes of tile
  //    row l / kChunkLanes of the load (lanes past the load's rows copy part
  //    0 of its first row again, into the slot's unread tail).
  auto slot_of_load = [&](int i) -> uint32_t* {
    switch (i % kRingLoads) {
      case 0: return ring0 + wave * 256;
      case 1: return ring1 + wave * 256;
      case 2: return ring2 + wave * 256;
      default: return ring3 + wave * 256;
    }
  };
  const int dma_off = lane < 2 * kP * G::kChunkLanes
                          ? (lane / G::kChunkLanes) * row_bytes + 16 * (lane % G::kChunkLanes)
                          : 0;
  auto load_lds = [&](int i) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(trellis_rsrc, (lds_ptr_t)slot_of_load(i), 16, dma_off,
                                             i * 2 * kP * row_bytes, 0, 0);
  };

  //    Dword / halfword loads: raw[j][h] holds tile row 2j + h of this
  //    wavefront's two tiles (coalesced: one dword of the chunk; direct: this
  //    lane's window words, tile m >> 3).  4-bit chunks load rotated: lane l
  //    holds word ((l & 31) - 2t) & 31 of tile t = l >> 5, so the two words
  //    each decoding lane gathers below come, across each half-wavefront,
  //    from 32 distinct lanes mod 32 (no ds_bpermute bank conflict between
  //    the two tiles).
  const int raw_off = kRotate ? 4 * (32 * (lane >> 5) + (((lane & 31) - 2 * (lane >> 5)) & 31))
                              : (lane < 8 * kBitsX2 ? 4 * lane : 0);  // lanes past the chunk reload dword 0
  //    A ring of kDepth register slots: step j's loads land in slot j % kDepth
  //    (every index is a compile-time constant: the step loop is unrolled).
  uint32_t raw[kLds ? 1 : kDepth][2][G::kRaw];
  auto load_step = [&](int j) {
    const int slot = j % kDepth;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int row = (2 * j + h) * row_bytes;
      if constexpr (G::kCoalesced) {
        if constexpr (kAligned) {
          raw[slot][h][0] = __builtin_amdgcn_raw_buffer_load_b32(trellis_rsrc, raw_off, row, 0);
        } else {
          raw[slot][h][0] = tile_word<false>(chunk + row, raw_off);
        }
      } else {
#pragma unroll
        for (int i = 0; i < G::kWords; ++i) {
          if constexpr (kAligned) {
            raw[slot][h][i] = __builtin_amdgcn_raw_buffer_load_b32(trellis_rsrc, tile_off + off[i], row, 0);
          } else {
            raw[slot][h][i] = tile_word<false>(chunk + row + tile_off, off[i]);
          }
        }
      }
    }
  };
  // (the activation loads above are issued first)
  asm volatile("" ::: "memory");
  if constexpr (kLds) {
#pragma unroll
    for (int i = 0; i < kRingLoads; ++i) load_lds(i);
  } else {
#pragma unroll
    for (int j = 0; j < kDepth; ++j) load_step(j);
  }
  // dword loads: ds_bpermute byte addresses of the lanes holding this lane's
  // words; LDS stream: this lane's word addresses within a slot's tile row
  int src[G::kWords];
#pragma unroll
  for (int i = 0; i < G::kWords; ++i) {
    const int t = m >> 3;
    const int w = off[i] / 4;
    if constexpr (kLds) {
      src[i] = (tile_off + off[i]) / 4;
    } else {
      src[i] = kRotate ? 4 * (32 * t + ((w + 2 * t) & 31)) : 4 * (t * 4 * kBitsX2 + w);
    }
  }

  // c. forming: t = H128(x * suh) of a (block, row) and its maximum |t|,
  //    published in LDS; after the first barrier (in the stream loop) each
  //    row's t is split at the group's power-of-two scale of that row into
  //    FP16 high / low parts, written straight into B-operand order:
  //    act = [step][g][B column 2r + (0 hi | 1 lo)][8 halves].  The LDS
  //    stores bypass the compiler's LDS-DMA tracking (they never touch a
  //    ring slot), so they do not wait for the trellis loads in flight.
  float fv[kFormTasks][2];
  float fr[kPasses][8];
  if (row_form) {
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t xw = xq[p][j >> 1], sw = sq[p][j >> 1];
        fr[p][j] = u16_act(uint16_t(xw >> (16 * (j & 1))), a.x_dtype) * vq::f16_to_f32(uint16_t(sw >> (16 * (j & 1))));
      }
      vq::h128_rows(fr[p], rl);
      float mx = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) mx = fmaxf(mx, fabsf(fr[p][j]));
      mx = fmaxf(mx, vq::xor_lanes<1>(mx, lane));
      mx = fmaxf(mx, vq::xor_lanes<2>(mx, lane));
      mx = fmaxf(mx, vq::xor_lanes<4>(mx, lane));
      mx = fmaxf(mx, vq::xor_lanes<8>(mx, lane));
      if (rl == 0) {
        vq::lds_store_b32(vq::lds_address(&block_max[0][2 * p + (wc >> 1)][4 * (wc & 1) + (lane >> 4)]),
                          __builtin_bit_cast(uint32_t, mx));
      }
    }
  }
#pragma unroll
  for (int f = 0; f < kFormTasks && !row_form; ++f) {
    const int t = wc + 4 * f;
    fv[f][0] = fv[f][1] = 0.0f;
    if (t < kTasks) {
      float v0 = u16_act(uint16_t(xv[f][0]), a.x_dtype) * vq::f16_to_f32(uint16_t(sv[f][0]));
      float v1 = u16_act(uint16_t(xv[f][1]), a.x_dtype) * vq::f16_to_f32(uint16_t(sv[f][1]));
      vq::h128_wave(v0, v1, lane);
      const float mx = vq::wave_max(fmaxf(fabsf(v0), fabsf(v1)), lane);
      if (lane == 0) vq::lds_store_b32(vq::lds_address(&block_max[grp][t / kRows][t % kRows]),
                                        __builtin_bit_cast(uint32_t, mx));
      fv[f][0] = v0;
      fv[f][1] = v1;
    }
  }
  // scale exponent of row r of this group (maxima complete)
  auto row_exponent = [&](int r) {
    uint32_t mx = 0u;
#pragma unroll
    for (int b = 0; b < kBlocks; ++b) {
      // nonnegative floats order as their bit patterns
      const uint32_t v = vq::lds_load_b32(vq::lds_address(&block_max[grp][b][r]));
      mx = v > mx ? v : mx;
    }
    return scale_exponent(mx);
  };
  auto split_store = [&]() {
    auto slot_of = [&](int k) {
      const int step = k >> 5;
      const int w = k & 31;
      const int kk = w & 15;
      const int gg = (kk & 7) >> 1;
      const int slot = 4 * (w >> 4) + (kk & 1) + 2 * (kk >> 3);
      return ((step * 4 + gg) * kCols) * 8 + slot;
    };
    const uint32_t gact = vq::lds_address(act + grp * kActHalves);
    if (row_form) {
      // inputs 8 rl + 2 i, + 1 of a block: adjacent halves of group i of
      // step rl / 4, at slot 4 ((rl & 3) >> 1) + 2 (rl & 1): one dword each
      const int s0 = 4 * ((rl & 3) >> 1) + 2 * (rl & 1);
#pragma unroll
      for (int p = 0; p < kPasses; ++p) {
        const int b = 2 * p + (wc >> 1);
        const int r = 4 * (wc & 1) + (lane >> 4);
        const int e = row_exponent(r);
        const uint32_t base = gact + 2 * uint32_t(b * 4 * 4 * kCols * 8 + (2 * r) * 8);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float t0 = ldexpf(fr[p][2 * i], e);
          const float t1 = ldexpf(fr[p][2 * i + 1], e);
          const _Float16 hi0 = _Float16(t0), hi1 = _Float16(t1);
          const _Float16 lo0 = _Float16(t0 - float(hi0)), lo1 = _Float16(t1 - float(hi1));
          const uint32_t hw = uint32_t(__builtin_bit_cast(uint16_t, hi0)) |
                              (uint32_t(__builtin_bit_cast(uint16_t, hi1)) << 16);
          const uint32_t lw = uint32_t(__builtin_bit_cast(uint16_t, lo0)) |
                              (uint32_t(__builtin_bit_cast(uint16_t, lo1)) << 16);
          const uint32_t h = uint32_t(((rl >> 2) * 4 + i) * kCols * 8 + s0);
          vq::lds_store_b32(base + 2 * h, hw);
          vq::lds_store_b32(base + 2 * (h + 8), lw);
        }
      }
      return;
    }
    const int h0 = slot_of(lane);
    const int h1 = slot_of(lane + 64);
#pragma unroll
    for (int f = 0; f < kFormTasks; ++f) {
      const int t = wc + 4 * f;
      const int b = t / kRows;
      const int r = t % kRows;
      if (t < kTasks) {
        const int e = row_exponent(r);
        const float t0 = ldexpf(fv[f][0], e);
        const float t1 = ldexpf(fv[f][1], e);
        const _Float16 hi0 = _Float16(t0), hi1 = _Float16(t1);
        const _Float16 lo0 = _Float16(t0 - float(hi0)), lo1 = _Float16(t1 - float(hi1));
        const uint32_t base = gact + 2 * uint32_t(b * 4 * 4 * kCols * 8 + (2 * r) * 8);
        vq::lds_store_b16(base + 2 * h0, __builtin_bit_cast(uint16_t, hi0));
        vq::lds_store_b16(base + 2 * (h0 + 8), __builtin_bit_cast(uint16_t, lo0));
        vq::lds_store_b16(base + 2 * h1, __builtin_bit_cast(uint16_t, hi1));
        vq::lds_store_b16(base + 2 * (h1 + 8), __builtin_bit_cast(uint16_t, lo1));
      }
    }
  };

  // d. stream: decode step j while later steps are in flight.  The products
  //    of the whole range accumulate in acc1/acc2 (one scale per row), and
  //    are folded, unscaled, into tot1/tot2 at the end (high + low parts:
  //    B columns 2r, 2r + 1 sit in adjacent lanes).  Lanes m >= kCols read
  //    B column m % kCols again: their MFMA columns are never used.
  //    Gathered words of step j in slot j % 2 (step j + 1 is gathered while
  //    step j decodes); its ring slot is free once gathered.
  uint32_t wv[kLds ? 1 : 2][2][G::kWords];
  auto gather = [&](int j) {
    const int slot = j % kDepth;
#pragma unroll
    for (int i = 0; i < G::kWords; ++i) {
      if constexpr (G::kCoalesced) {
        wv[j % 2][0][i] = uint32_t(__builtin_amdgcn_ds_bpermute(src[i], int(raw[slot][0][0])));
        wv[j % 2][1][i] = uint32_t(__builtin_amdgcn_ds_bpermute(src[i], int(raw[slot][1][0])));
      } else {
        wv[j % 2][0][i] = raw[slot][0][i];
        wv[j % 2][1][i] = raw[slot][1][i];
      }
    }
  };
  const half8_t* bops = reinterpret_cast<const half8_t*>(act + grp * kActHalves) + g * kCols + (m % kCols);
  const int r_own = (m >> 1) < kRows ? (m >> 1) : 0;
  f32x4_t acc1 = {}, acc2 = {};
  float tot1[4], tot2[4];
  half8_t bop = {};
  if constexpr (!kLds) gather(0);
  //    LDS stream: the words of step j + 1 are read at the start of step j,
  //    so their latency hides behind step j's decode (a wavefront running
  //    alone on its SIMD would otherwise wait for every step's reads).
  //    Reading step s, the first step of load i = s / kP, needs load i
  //    landed.  The reads of step s > 0 are issued in step s - 1, before
  //    that step's refill, so the loads issued by then are 0 .. min(i - 2 +
  //    kRingLoads, kLoads - 1), and at most min(kRingLoads - 2, kLoads - 1 -
  //    i) of them may still be pending; before step 0, kRingLoads - 1.
  uint32_t nw0[G::kWords], nw1[G::kWords];
  auto read_words = [&](int s) {
    const int i = s / kP;
    if (s % kP == 0) {
      const int younger = s == 0 ? kRingLoads - 1
                                 : (kRingLoads - 2 < kLoads - 1 - i ? kRingLoads - 2 : kLoads - 1 - i);
      switch (younger) {
        case 0: wait_vmcnt<0>(); break;
        case 1: wait_vmcnt<1>(); break;
        case 2: wait_vmcnt<2>(); break;
        default: wait_vmcnt<3>(); break;
      }
    }
    const uint32_t* slot = slot_of_load(i) + (2 * (s % kP)) * (G::kChunk / 4);
#pragma unroll
    for (int q = 0; q < G::kWords; ++q) {
      nw0[q] = slot[src[q]];
      nw1[q] = slot[G::kChunk / 4 + src[q]];
    }
  };
  if constexpr (kLds) read_words(0);
#pragma unroll
  for (int j = 0; j < kSteps; ++j) {
    uint32_t w0[G::kWords], w1[G::kWords];
    if constexpr (kLds) {
#pragma unroll
      for (int q = 0; q < G::kWords; ++q) {
        w0[q] = nw0[q];
        w1[q] = nw1[q];
      }
      if (j + 1 < kSteps) read_words(j + 1);
      // this step's B operand, read ahead of the decode (step 0's are
      // written after it, below)
      if (j > 0 && m < kCols) {
        asm volatile("" ::: "memory");
        bop = bops[j * 4 * kCols];
      }
    } else {
      if (j + 1 < kSteps) gather(j + 1);
      if (j + kDepth < kSteps) load_step(j + kDepth);
#pragma unroll
      for (int q = 0; q < G::kWords; ++q) {
        w0[q] = wv[j % 2][0][q];
        w1[q] = wv[j % 2][1][q];
      }
    }
    uint32_t q0[4], q1[4];
    decode_words<kBitsX2, kCodebook>(L, w0, q0);
    decode_words<kBitsX2, kCodebook>(L, w1, q1);
    // the activation maxima, then the B operands, are complete once every
    // wavefront is past a barrier (the first decode overlaps the wait).  LDS
    // stream: bare s_barriers after this wavefront's LDS writes;
    // __syncthreads would also wait for every trellis load in flight.
    if (j == 0) {
      auto barrier = [&]() {
        if constexpr (kLds) {
          wait_lgkmcnt0();
          __builtin_amdgcn_s_barrier();
          asm volatile("" ::: "memory");
        } else {
          __syncthreads();
        }
      };
      if constexpr (kBlocks > 1) barrier();
      split_store();
      barrier();
    }
    const u32x4_t a1 = {q0[0], q0[1], q1[0], q1[1]};
    const u32x4_t a2 = {q0[2], q0[3], q1[2], q1[3]};
    // only the lanes of used B columns read (LDS bandwidth): the others keep
    // a stale operand, whose MFMA columns are never looked at
    if ((!kLds || j == 0) && m < kCols) {
      asm volatile("" ::: "memory");
      bop = bops[j * 4 * kCols];
    }
    acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, a1), bop, acc1, 0, 0, 0);
    acc2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, a2), bop, acc2, 0, 0, 0);
    // LDS stream: the slot's last step was read in the previous step (its
    // reads returned during this step's decode): refill it with load
    // i + kRingLoads
    if constexpr (kLds) {
      if (j % kP == kP - 1 && j / kP + kRingLoads < kLoads) {
        wait_lgkmcnt0();
        load_lds(j / kP + kRingLoads);
      }
    }
  }

  {
    const int e = row_exponent(r_own);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      tot1[i] = ldexpf(acc1[i] + vq::xor_lanes<1>(acc1[i], lane), -e);
      tot2[i] = ldexpf(acc2[i] + vq::xor_lanes<1>(acc2[i], lane), -e);
    }
  }

  // e. the partial sums of this K split: lane (g, 2r) holds rows 4g..4g+3 of
  //    both MFMAs.  Agent-scope stores are written through to the
  //    device-coherent level, so the fused finish (on any XCD) reads them
  //    without a cache writeback of this workgroup.
  //    Lane (g, 2r)'s four rows 4g..4g+3 are columns 4 (g & 1) + 16 (g >> 1)
  //    + 0..3 of this wavefront's 32 (tot1) and the same + 8 (tot2): two
  //    16-byte stores, whole runs rather than scattered words.
  //    The buffer starts at this workgroup's 128 columns of its split
  //    and ends with row a.rows - 1 of them.
  //    Groups 1.. first hand their sums to group 0 through this wavefront's
  //    own regions of ring slots 0 and 1 (its loads have all landed and been
  //    read); group 0 adds them in group order.
  if constexpr (kGroups > 1) {
    if (grp > 0) {
      wait_lgkmcnt0();
      *reinterpret_cast<f32x4_t*>(ring0 + wave * 256 + 4 * lane) = f32x4_t{tot1[0], tot1[1], tot1[2], tot1[3]};
      *reinterpret_cast<f32x4_t*>(ring1 + wave * 256 + 4 * lane) = f32x4_t{tot2[0], tot2[1], tot2[2], tot2[3]};
    }
    wait_lgkmcnt0();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (grp == 0) {
#pragma unroll
      for (int q = 1; q < kGroups; ++q) {
        const f32x4_t o1 = *reinterpret_cast<const f32x4_t*>(ring0 + (4 * q + wc) * 256 + 4 * lane);
        const f32x4_t o2 = *reinterpret_cast<const f32x4_t*>(ring1 + (4 * q + wc) * 256 + 4 * lane);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          tot1[i] += o1[i];
          tot2[i] += o2[i];
        }
      }
    }
  }
  float* dst = a.partial + int64_t(split) * a.rows * a.np + 128 * int64_t(cblk);
  const __amdgpu_buffer_rsrc_t part_rsrc =
      __builtin_amdgcn_make_buffer_rsrc(dst, 0, int(4 * ((a.rows - 1) * a.np + 128)), 0x00020000);
  if (grp == 0 && m < kCols && (m & 1) == 0 && (m >> 1) < a.rows) {
    const int col = 32 * wc + 4 * (g & 1) + 16 * (g >> 1);
    const int offset = 4 * (int((m >> 1) * a.np) + col);
    store_agent_x4(part_rsrc, offset, f32x4_t{tot1[0], tot1[1], tot1[2], tot1[3]});
    store_agent_x4(part_rsrc, offset + 32, f32x4_t{tot2[0], tot2[1], tot2[2], tot2[3]});
  }

  // f. fused finish: the last workgroup of this 128-column block to arrive
  //    sums every split's partials and writes the outputs.
  if (a.counter_base >= 0) {
    uint32_t* counter = a.counters + (a.counter_base + cblk) * kCounterStride;
    __shared__ int is_last;
    // every store of this wavefront has completed (vmcnt counts stores on
    // gfx9), then every wavefront of the workgroup is past that point
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
      const uint32_t arrived =
          __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      is_last = arrived == uint32_t(a.splits - 1);
    }
    __syncthreads();
    if (is_last) {
      finish_block(a, reinterpret_cast<float*>(act), tid, cblk);
      if (tid == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// ---- dispatch ----------------------------------------------------------------

// Steps (two tile rows) per LDS-stream load, as Gemv<kBitsX2>::kStepsPerLoad.
inline int steps_per_load(int64_t bits_x2) { return bits_x2 <= 4 ? 4 : (bits_x2 <= 8 ? 2 : 1); }

// A workgroup of kGroups groups needs two loads per group range (the groups
// meet in two ring slots).
inline bool can_group(int64_t bits_x2, int blocks) { return steps_per_load(bits_x2) < 4 * blocks; }

template <int kBitsX2, int kCodebook, int kLoad, int kBlocks, int kGroups>
int launch_gemv(const GemvArgs& a, dim3 grid, hipStream_t stream) {
  if constexpr (kGroups > 1 && !(Gemv<kBitsX2>::kStepsPerLoad < 4 * kBlocks)) {
    return vq::fail("EXL3 GEMV: grouped workgroups need two loads per group");
  } else {
    const dim3 block(kThreads * kGroups);
    if (a.rows <= 1) {
      hipLaunchKernelGGL((gemv_kernel<kBitsX2, kCodebook, kLoad, 1, kBlocks, kGroups>), grid, block, 0, stream, a);
    } else if (a.rows <= 2) {
      hipLaunchKernelGGL((gemv_kernel<kBitsX2, kCodebook, kLoad, 2, kBlocks, kGroups>), grid, block, 0, stream, a);
    } else if (a.rows <= 4) {
      hipLaunchKernelGGL((gemv_kernel<kBitsX2, kCodebook, kLoad, 4, kBlocks, kGroups>), grid, block, 0, stream, a);
    } else {
      hipLaunchKernelGGL((gemv_kernel<kBitsX2, kCodebook, kLoad, 8, kBlocks, kGroups>), grid, block, 0, stream, a);
    }
    return vq::check_launch("exl3 gemv_kernel");
  }
}

template <int kBitsX2, int kCodebook>
int launch_format(bool aligned, int load, const GemvArgs* gemv, int gemv_blocks, int gemv_groups, dim3 grid,
                  hipStream_t stream, const uint8_t* trellis, int64_t tiles_k, int64_t tiles_n,
                  uint16_t* decoded) {
  if (gemv) {
    const GemvArgs& a = *gemv;
    if (load == kLoadLds && gemv_groups == 4) {
      if (gemv_blocks == 1) return launch_gemv<kBitsX2, kCodebook, kLoadLds, 1, 4>(a, grid, stream);
      if (gemv_blocks == 2) return launch_gemv<kBitsX2, kCodebook, kLoadLds, 2, 4>(a, grid, stream);
      return launch_gemv<kBitsX2, kCodebook, kLoadLds, 4, 4>(a, grid, stream);
    }
    if (load == kLoadLds) {
      if (gemv_blocks == 1) return launch_gemv<kBitsX2, kCodebook, kLoadLds, 1, 1>(a, grid, stream);
      if (gemv_blocks == 2) return launch_gemv<kBitsX2, kCodebook, kLoadLds, 2, 1>(a, grid, stream);
      if (gemv_blocks == 4) return launch_gemv<kBitsX2, kCodebook, kLoadLds, 4, 1>(a, grid, stream);
      return launch_gemv<kBitsX2, kCodebook, kLoadLds, 8, 1>(a, grid, stream);
    }
    if (load == kLoadDword) {
      if (gemv_blocks == 1) return launch_gemv<kBitsX2, kCodebook, kLoadDword, 1, 1>(a, grid, stream);
      if (gemv_blocks == 2) return launch_gemv<kBitsX2, kCodebook, kLoadDword, 2, 1>(a, grid, stream);
      if (gemv_blocks == 4) return launch_gemv<kBitsX2, kCodebook, kLoadDword, 4, 1>(a, grid, stream);
      return launch_gemv<kBitsX2, kCodebook, kLoadDword, 8, 1>(a, grid, stream);
    }
    if (gemv_blocks == 1) return launch_gemv<kBitsX2, kCodebook, kLoadHalf, 1, 1>(a, grid, stream);
    if (gemv_blocks == 2) return launch_gemv<kBitsX2, kCodebook, kLoadHalf, 2, 1>(a, grid, stream);
    if (gemv_blocks == 4) return launch_gemv<kBitsX2, kCodebook, kLoadHalf, 4, 1>(a, grid, stream);
    return launch_gemv<kBitsX2, kCodebook, kLoadHalf, 8, 1>(a, grid, stream);
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

// Parts of the format list built as separate objects: format i of
// VQ_EXL3_FORMATS is instantiated by part i % kGemvParts.
constexpr int kGemvParts = 8;


// launch_format for the formats of part P (exl3_gemv_part.hip, built with
// VQ_GEMV_PART = P); a format of another part is refused.
template <int P>
int gemv_launch_part(int64_t bits_x2, int64_t codebook, bool aligned, int load, const GemvArgs* gemv,
                     int gemv_blocks, int gemv_groups, dim3 grid, hipStream_t stream,
                     const uint8_t* trellis, int64_t tiles_k, int64_t tiles_n, uint16_t* decoded);

}  // namespace exl3
