// EXL3 PLE rows for gfx950: decodes selected rows of a trellis-compressed
// embedding table (one FP16 scale word, then a little-endian ring of dim *
// bits bits) into BF16, with per-head bias and row-ownership masks.
// Reference: csrc/exl3/ple.cu:49-147 (ple_decode_kernel), :167-234 (host
// checks); format statement tests/models/qwen4_exp/test_exl3_ple_decode.py:
// 1-12.
//
// Channel c's 16-bit state takes bit m from ring bit ((c - m / bits) mod dim)
// * bits + m % bits: the low `bits` state bits are channel c's own ring
// chunk, the next `bits` the chunk of channel c - 1, and so on.  So the state
// is the chunks of channels c, c - 1, c - 2, ... laid side by side from the
// low bit, each chunk read from the ring with one 32-bit window.  The value
// is the mul1 codebook in the PLE decoder's own arithmetic: FP32 product of
// (1024 + byte sum) and the FP16 constant 0x1EEE, FP32 add of 0xC931,
// rounded to FP16; then an FP32 product with the row scale and an FP32 add
// of the head bias (each rounded, never contracted), rounded to BF16.
//
// One workgroup per row (a bounded grid strides over the rows); the row's
// head and scale are found once, by the first thread.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstdint>

#include "../../include/vllm_mi355x.h"
#include "common.h"

namespace ple {
namespace {

constexpr int kThreads = 256;

// Last head starting at or before id, if id lies inside its vocabulary (gaps
// and table-padding rows read nothing): reference ple.cu:51-75.
__device__ int64_t head_of(int64_t id, const int64_t* offsets, const int64_t* sizes, int64_t heads) {
  int64_t lo = 0, hi = heads;
  while (lo < hi) {
    const int64_t mid = lo + (hi - lo) / 2;
    if (offsets[mid] <= id) lo = mid + 1; else hi = mid;
  }
  if (lo == 0) return -1;
  const int64_t head = lo - 1;
  const int64_t start = offsets[head];
  const int64_t size = sizes[head];
  return start >= 0 && size > 0 && id >= start && id - start < size ? head : -1;
}

// 32 ring bits starting at ring bit p, little-endian (ring bit p is bit 0):
// words w = p / 16 and w + 1 of the ring (the second only when inside it).
__device__ __forceinline__ uint32_t ring_window(const uint16_t* ring, int64_t words, int64_t p) {
  const int64_t w = p >> 4;
  const uint32_t lo = ring[w];
  const uint32_t hi = w + 1 < words ? ring[w + 1] : 0u;
  return ((hi << 16) | lo) >> (p & 15);
}

__device__ __forceinline__ float mul1_value(uint32_t state) {
  const uint32_t p = state * 0x83DCD12Du;
  const uint32_t t = (p & 255u) + ((p >> 8) & 255u) + ((p >> 16) & 255u) + (p >> 24);
  const float k_inv = vq::f16_to_f32(0x1eee);
  const float k_bias = vq::f16_to_f32(0xc931);
  const float v = __fadd_rn(__fmul_rn(float(1024u + t), k_inv), k_bias);
  return float(_Float16(v));
}

__global__ __launch_bounds__(kThreads) void ple_decode_kernel(
    const uint16_t* __restrict__ packed, const int64_t* __restrict__ ids,
    const uint16_t* __restrict__ head_bias, const int64_t* __restrict__ offsets,
    const int64_t* __restrict__ sizes, int64_t rows, int64_t words, int64_t heads, int64_t dim,
    int64_t owner_lo, int64_t owner_hi, int bits, uint16_t* __restrict__ out) {
  __shared__ int64_t row_head;
  __shared__ float row_scale;
  const int64_t ring_words = words - 1;
  const uint32_t mask = (1u << bits) - 1u;  // bits <= 16
  const int chunks = (16 + bits - 1) / bits;
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    if (threadIdx.x == 0) {
      const int64_t id = ids[row];
      int64_t head = -1;
      float scale = 0.0f;
      if (id >= 0 && id >= owner_lo && id < owner_hi) {
        head = head_of(id, offsets, sizes, heads);
        if (head >= 0) scale = vq::f16_to_f32(packed[row * words]);
      }
      row_head = head;
      row_scale = scale;
    }
    __syncthreads();
    const int64_t head = row_head;
    const float scale = row_scale;
    const uint16_t* ring = packed + row * words + 1;
    for (int64_t c = threadIdx.x; c < dim; c += kThreads) {
      uint16_t v = 0;  // BF16 zero: masked rows read nothing
      if (head >= 0) {
        uint32_t state = 0;
        for (int q = 0; q < chunks; ++q) {
          const int64_t j = c >= q ? c - q : dim - (q - c);
          state |= (ring_window(ring, ring_words, j * bits) & mask) << (q * bits);
        }
        const float scaled = __fmul_rn(mul1_value(state & 0xffffu), scale);
        const float biased = __fadd_rn(scaled, vq::f16_to_f32(head_bias[head * dim + c]));
        v = vq::f32_to_bf16(biased);
      }
      out[row * dim + c] = v;
    }
    // the next row's head must not replace this one under a slower thread
    __syncthreads();
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
  const unsigned blocks = unsigned(std::min<int64_t>(rows, 65535));
  hipLaunchKernelGGL(ple::ple_decode_kernel, dim3(blocks), dim3(ple::kThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(packed_rows),
                     global_ids, static_cast<const uint16_t*>(head_bias), head_offsets,
                     head_vocab_sizes, rows, words, heads, dim, owner_lo, owner_hi, int(bits),
                     static_cast<uint16_t*>(out));
  return check_launch("exl3 ple_decode_kernel");
}
