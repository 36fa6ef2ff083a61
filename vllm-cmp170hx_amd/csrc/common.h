// Shared host/device definitions of the quantized-matmul library: status
// codes, dtype codes, the thread-local error text behind the C-ABI, and the
// small device helpers every kernel uses.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

namespace vq {

// C-ABI status codes (see include/vllm_mi355x.h).
enum Status : int { kOk = 0, kInvalidArgument = 1, kHipFailure = 2 };
// Activation / output element types (see include/vllm_mi355x.h).
enum Dtype : int { kBF16 = 0, kFP16 = 1, kFP32 = 2 };

// Records the message returned by vllm_mi355x_last_error() for this thread.
int fail(const std::string& message);
int check_launch(const char* what);

inline int64_t dtype_bytes(int dtype) { return dtype == kFP32 ? 4 : 2; }

// Half-open byte ranges [a, a+na) and [b, b+nb) share memory.
inline bool overlaps(const void* a, int64_t na, const void* b, int64_t nb) {
  if (!a || !b || na <= 0 || nb <= 0) return false;
  const uintptr_t pa = reinterpret_cast<uintptr_t>(a);
  const uintptr_t pb = reinterpret_cast<uintptr_t>(b);
  return pa < pb + static_cast<uintptr_t>(nb) && pb < pa + static_cast<uintptr_t>(na);
}

// ---- device helpers ---------------------------------------------------------

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __builtin_bit_cast(float, uint32_t(b) << 16);
}
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  const uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40u);
  return uint16_t((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}
__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return float(__builtin_bit_cast(_Float16, h));
}

__device__ __forceinline__ float load_act(const void* p, int dtype, int64_t i) {
  if (dtype == kBF16) return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
  if (dtype == kFP16) return f16_to_f32(static_cast<const uint16_t*>(p)[i]);
  return static_cast<const float*>(p)[i];
}
__device__ __forceinline__ void store_act(void* p, int dtype, int64_t i, float v) {
  if (dtype == kBF16) {
    static_cast<uint16_t*>(p)[i] = f32_to_bf16(v);
  } else if (dtype == kFP16) {
    static_cast<_Float16*>(p)[i] = _Float16(v);
  } else {
    static_cast<float*>(p)[i] = v;
  }
}

constexpr float kH128Scale = 0.08838834764831845f;

// H128 of one 128-value block held by a wavefront: lane l holds elements l
// (v0) and l + 64 (v1).  Butterfly distances 1, 2, ..., 64 in increasing
// order; the lower element becomes lo + hi and the upper one lo - hi (FP32
// round to nearest), then both are scaled by 1/sqrt(128).  The same
// operations in the same order as the reference (reference.cu:107-122,
// codec.cuh:186-209), so the transform is bit-identical to it.
__device__ __forceinline__ void h128_wave(float& v0, float& v1, int lane) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const float o0 = __shfl_xor(v0, d);
    const float o1 = __shfl_xor(v1, d);
    const bool upper = (lane & d) != 0;
    v0 = upper ? o0 - v0 : v0 + o0;
    v1 = upper ? o1 - v1 : v1 + o1;
  }
  const float lo = v0 + v1;
  const float hi = v0 - v1;
  v0 = lo * kH128Scale;
  v1 = hi * kH128Scale;
}

}  // namespace vq
