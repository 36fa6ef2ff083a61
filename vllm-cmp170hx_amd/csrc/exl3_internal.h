// Internal declarations shared by the EXL3 translation units (not part of
// the C-ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"
#include "exl3_codec.h"

namespace exl3 {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// Every (bits_x2, codebook) the format admits (reference: csrc/exl3/gemm.cu:
// 17-20, kernels/exl3/utils.py:283-285): even rates 1..8 bits for both
// codebooks, and 1.5 / 2.5 / 3.5 bits for mul1.
#ifndef VQ_EXL3_FORMATS
#define VQ_EXL3_FORMATS(X)                                                       \
  X(2, 1) X(4, 1) X(6, 1) X(8, 1) X(10, 1) X(12, 1) X(14, 1) X(16, 1)           \
  X(2, 2) X(3, 2) X(4, 2) X(5, 2) X(6, 2) X(7, 2) X(8, 2) X(10, 2) X(12, 2)    \
  X(14, 2) X(16, 2)
#endif

// Arrival counters of fused finishes (the split-K GEMV's, the Marlin w13
// SwiGLU's): a pool in static device memory (exl3_linear.hip; zero when the
// code object loads, and every launch returns the slots it used to zero).
// The host hands out ranges of kCounterSlots slots, one per (device, stream,
// graph capture): launches that may overlap (on other streams, or in graphs
// replayed on other streams) never share a slot, and launches in one range
// run one after another.
constexpr int kCounterRanges = 128;
constexpr int kCounterSlots = 1024;
// One counter per 128-byte line: atomics to one line serialize, so the units
// a launch counts must not share lines.
constexpr int kCounterStride = 32;

// Cache policy bits of a buffer access at the device-coherent level (sc1,
// that of an agent-scope access): what one XCD writes so, another XCD reads
// so after an arrival counter says it is complete.
constexpr int kCachePolicySc1 = 16;

// The pool's device address and the first slot of the range of `stream`'s
// current capture (or of its eager launches), or a null pool when `slots`
// exceeds kCounterSlots or no range is free (the caller then takes a path
// without counters).
struct CounterSlots {
  uint32_t* pool;
  int base;
};
CounterSlots counter_slots(hipStream_t stream, int64_t slots);

// Position of a format in VQ_EXL3_FORMATS (-1: not admitted); the kernels'
// instantiations are split over separately compiled parts by it.
constexpr int format_index(int bits_x2, int codebook) {
  int i = 0;
#define VQ_INDEX(B, C)                       \
  if (bits_x2 == B && codebook == C) return i; \
  ++i;
  VQ_EXL3_FORMATS(VQ_INDEX)
#undef VQ_INDEX
  return -1;
}

inline bool known_format(int64_t bits_x2, int64_t codebook) {
#define VQ_KNOWN(B, C) if (bits_x2 == B && codebook == C) return true;
  VQ_EXL3_FORMATS(VQ_KNOWN)
#undef VQ_KNOWN
  return false;
}

// Ring word at `byte_offset` of a tile (4-byte aligned trellis, or two
// halfword loads from a 2-byte aligned one).
template <bool kAligned>
__device__ __forceinline__ uint32_t tile_word(const uint8_t* tile, int byte_offset) {
  if constexpr (kAligned) {
    return *reinterpret_cast<const uint32_t*>(tile + byte_offset);
  } else {
    const uint16_t* h = reinterpret_cast<const uint16_t*>(tile + byte_offset);
    return uint32_t(h[0]) | (uint32_t(h[1]) << 16);
  }
}

// Power-of-two exponent e so that max * 2^e lies in [2^14, 2^15): an FP16
// high part then stays below 2^15 and the low part keeps ~11 more bits.
__device__ __forceinline__ int scale_exponent(uint32_t max_bits) {
  const int biased = int((max_bits >> 23) & 0xff);
  if (max_bits == 0u) return 0;
  const int e = 14 - (biased - 127);
  return e > 127 ? 127 : (e < -126 ? -126 : e);
}

__device__ __forceinline__ float u16_act(uint16_t v, int dtype) {
  return dtype == vq::kBF16 ? vq::bf16_to_f32(v) : vq::f16_to_f32(v);
}

// Activation precision of the many-row tile GEMM (exl3_set_tile_precision,
// exl3_gemm.hip): false (the default) = FP16 high and low parts, true = the
// high part alone.
bool tile_fp16_only();

// Large-M (prefill) dense linear, rows > 32 (exl3_gemm.hip).  Arguments as
// exl3_linear_out's, validated by it; workspace holds rows * padded_in
// floats (the FP16 high and low activation halves) plus one int32 row
// exponent per row.
int prefill_linear(const void* x, int x_dtype, int64_t rows, const uint8_t* trellis,
                   int64_t tiles_k, int64_t tiles_n, const uint16_t* suh, const uint16_t* svh,
                   int bits_x2, int codebook, int64_t logical_in, int64_t logical_out, void* out,
                   int out_dtype, float* workspace, hipStream_t stream);

// The finish of exl3_linear_out: out = RN(H128(sum of `splits` partial rows)
// * svh) for every (row, 128-column block) (exl3_linear.hip).
int launch_output(const float* partial, int splits, int rows, int64_t np, const uint16_t* svh,
                  int64_t logical_out, int64_t out_stride, void* out, int out_dtype,
                  hipStream_t stream);

}  // namespace exl3
