// EXL3 PLE rows for gfx950: decodes selected rows of a trellis-compressed
// embedding table (one FP16 scale word, then a little-endian ring of dim *
// bits bits) into BF16, with per-head bias and row-ownership masks.
// Reference: csrc/exl3/ple.cu:49-147 (ple_decode_kernel), :167-234 (host
// checks); format statement tests/models/qwen4_exp/test_exl3_ple_decode.py:
// 1-12.
//
// Channel c's 16-bit state takes bit m from ring bit ((c - m / bits) mod dim)
// * bits + m % bits: the low `bits` state bits are channel c's own ring
// chunk, the next `bits` the chunk of channel c - 1, and so on.  The chunks
// of channels c - chunks + 1 .. c lie side by side in the ring, at most 31
// bits, so a lane reads them as one window (three halfword loads) and lays
// them out in reverse chunk order; only the first chunks - 1 channels, whose
// chunks wrap to the ring's end, read them one at a time.  The value is the
// mul1 codebook in the PLE decoder's own arithmetic: the hash's byte sum in
// one v_sad_u8, the FP32 product of (1024 + byte sum) and the FP16 constant
// 0x1EEE, FP32 add of 0xC931, rounded to FP16; then an FP32 product with the
// row scale and an FP32 add of the head bias (each rounded, never
// contracted), rounded to BF16.
//
// One wavefront per row, four rows a workgroup (a bounded grid strides over
// the rows), no LDS and no barrier: the wavefront finds the row's head with
// a 64-way search, one ballot a round.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstdint>

#include "../../include/vllm_mi355x.h"
#include "common.h"

namespace ple {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;  // rows a workgroup decodes at once

// The head of row id: the last head starting at or before id (head offsets
// ascend), when id lies inside its vocabulary (gaps and table-padding rows
// read nothing); else -1.  The count of heads starting at or before id is
// found by a 64-way search: each round the wavefront probes 64 evenly spaced
// heads of the remaining range and one ballot keeps the stretch between the
// last probe at or before id and the next; a range of at most 64 heads is
// counted directly.
__device__ int64_t head_of(int64_t id, const int64_t* offsets, const int64_t* sizes, int64_t heads,
                           int lane) {
  int64_t lo = 0, hi = heads;  // the count lies in [lo, hi]
  while (hi - lo > 64) {
    const int64_t step = (hi - lo + 63) / 64;
    const int64_t probe = lo + lane * step;
    const int k = __builtin_popcountll(__ballot(probe < hi && offsets[probe] <= id));
    if (k == 0) {
      hi = lo;
    } else {
      hi = std::min(lo + k * step, hi);
      lo += (k - 1) * step + 1;
    }
  }
  const int64_t at_or_before =
      lo + __builtin_popcountll(__ballot(lo + lane < hi && offsets[lo + lane] <= id));
  if (at_or_before == 0) return -1;
  const int64_t head = at_or_before - 1;
  const int64_t start = offsets[head];
  const int64_t size = sizes[head];
  return start >= 0 && size > 0 && id >= start && id - start < size ? head : -1;
}

// Up to 32 ring bits from ring bit p on, little-endian (ring bit p lands in
// bit 0): halfwords p / 16 .. p / 16 + 2 (those inside the ring).
__device__ __forceinline__ uint32_t ring_bits(const uint16_t* ring, int64_t ring_words, int64_t p) {
  const int64_t w = p >> 4;
  uint64_t v = ring[w];
  if (w + 1 < ring_words) v |= uint64_t(ring[w + 1]) << 16;
  if (w + 2 < ring_words) v |= uint64_t(ring[w + 2]) << 32;
  return uint32_t(v >> (p & 15));
}

// The state of channel c (see the file comment).
__device__ __forceinline__ uint32_t channel_state(const uint16_t* ring, int64_t ring_words, int64_t dim,
                                                  int bits, int chunks, int64_t c) {
  const uint32_t mask = (1u << bits) - 1u;  // bits <= 16
  uint32_t state = 0;
  if (c >= chunks - 1) {
    // chunk q (channel c - q) sits chunks - 1 - q chunks above the window's base
    const uint32_t w = ring_bits(ring, ring_words, (c - chunks + 1) * bits);
    for (int q = 0; q < chunks; ++q) state |= ((w >> ((chunks - 1 - q) * bits)) & mask) << (q * bits);
  } else {
    for (int q = 0; q < chunks; ++q) {
      const int64_t from = c >= q ? c - q : dim - (q - c);
      state |= (ring_bits(ring, ring_words, from * bits) & mask) << (q * bits);
    }
  }
  return state & 0xffffu;
}

__device__ __forceinline__ float mul1_value(uint32_t state) {
  const uint32_t t = __builtin_amdgcn_sad_u8(state * 0x83DCD12Du, 0u, 0u);  // byte sum of the hash
  const float v = __fadd_rn(__fmul_rn(float(1024u + t), vq::f16_to_f32(0x1eee)), vq::f16_to_f32(0xc931));
  return float(_Float16(v));
}

__global__ __launch_bounds__(kThreads) void ple_decode_kernel(
    const uint16_t* __restrict__ packed, const int64_t* __restrict__ ids,
    const uint16_t* __restrict__ head_bias, const int64_t* __restrict__ offsets,
    const int64_t* __restrict__ sizes, int64_t rows, int64_t words, int64_t heads, int64_t dim,
    int64_t owner_lo, int64_t owner_hi, int bits, uint16_t* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int chunks = (16 + bits - 1) / bits;
  const int64_t stride = int64_t(gridDim.x) * kWaves;
  for (int64_t row = int64_t(blockIdx.x) * kWaves + (threadIdx.x >> 6); row < rows; row += stride) {
    const int64_t id = ids[row];
    const int64_t head =
        id >= 0 && id >= owner_lo && id < owner_hi ? head_of(id, offsets, sizes, heads, lane) : -1;
    uint16_t* dst = out + row * dim;
    if (head < 0) {
      for (int64_t c = lane; c < dim; c += 64) dst[c] = 0;  // BF16 zero: masked rows read nothing
      continue;
    }
    const float scale = vq::f16_to_f32(packed[row * words]);
    const uint16_t* ring = packed + row * words + 1;
    const uint16_t* bias = head_bias + head * dim;
    for (int64_t c = lane; c < dim; c += 64) {
      const float scaled = __fmul_rn(mul1_value(channel_state(ring, words - 1, dim, bits, chunks, c)), scale);
      dst[c] = vq::f32_to_bf16(__fadd_rn(scaled, vq::f16_to_f32(bias[c])));
    }
  }
}

}  // namespace
}  // namespace ple

extern "C" int exl3_ple_decode_out(const void* packed_rows, int64_t rows, int64_t words,
                                   const int64_t* global_ids, const void* head_bias, int64_t heads,
                                   const int64_t* head_offsets, const int64_t* head_vocab_sizes,
                                   int64_t dim, int64_t owner_lo, int64_t owner_hi, int64_t bits,
                                   void* out, void* stream) {
  using namespace vq;
  // the reference's checks and wording (csrc/exl3/ple.cu:176-216)
  if (bits < 1 || bits > 16) return fail("ple_decode_out: bits must be an integer in [1, 16]");
  if (!(owner_lo >= 0 && owner_hi >= owner_lo)) {
    return fail("ple_decode_out: owner range must satisfy 0 <= owner_lo <= owner_hi");
  }
  constexpr int64_t kMaxIndex = INT64_MAX;
  if (!(dim > 0 && dim <= (kMaxIndex - 256) / bits)) {
    return fail("ple_decode_out: dimension is empty or ring geometry overflows");
  }
  const int64_t ring_bits = dim * bits;
  if (ring_bits % 16 != 0) return fail("ple_decode_out: dim * bits must be divisible by 16");
  if (rows < 0 || rows > (kMaxIndex - 65535) / (1 + ring_bits / 16)) {
    return fail("ple_decode_out: packed row geometry overflows 64-bit indexing");
  }
  if (rows > kMaxIndex / dim || heads > kMaxIndex / dim) {
    return fail("ple_decode_out: output or bias geometry overflows 64-bit indexing");
  }
  if (words != 1 + ring_bits / 16) {
    return fail("ple_decode_out: packed_rows must be [R, 1 + dim*bits/16] and out must be [R, dim], "
                "with R = global_ids.numel()");
  }
  if (heads <= 0) {
    return fail("ple_decode_out: head_bias must be [heads, dim] and offsets/vocab sizes must be "
                "[heads], with heads > 0");
  }
  const void* inputs[5] = {packed_rows, global_ids, head_bias, head_offsets, head_vocab_sizes};
  const int64_t input_bytes[5] = {rows * words * 2, rows * 8, heads * dim * 2, heads * 8, heads * 8};
  for (int i = 0; i < 5; ++i) {
    if (overlaps(out, rows * dim * 2, inputs[i], input_bytes[i])) {
      return fail("unsupported operation: some elements of the input tensor and the written-to "
                  "tensor refer to a single memory location.");
    }
  }
  if (rows == 0) return kOk;
  const unsigned blocks = unsigned(std::min<int64_t>((rows + ple::kWaves - 1) / ple::kWaves, 65535));
  hipLaunchKernelGGL(ple::ple_decode_kernel, dim3(blocks), dim3(ple::kThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(packed_rows),
                     global_ids, static_cast<const uint16_t*>(head_bias), head_offsets,
                     head_vocab_sizes, rows, words, heads, dim, owner_lo, owner_hi, int(bits),
                     static_cast<uint16_t*>(out));
  return check_launch("exl3 ple_decode_kernel");
}
