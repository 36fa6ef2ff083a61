// Shared host/device definitions of the quantized-matmul library: status
// codes, dtype codes, the thread-local error text behind the C-ABI, and the
// small device helpers every kernel uses.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>
#include <type_traits>

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

// Elements i .. i + 7 of an activation-dtype array, of which the first
// `valid` exist: 16-byte stores when all eight exist and the address allows
// them, else one store per element (the same roundings either way).
__device__ __forceinline__ void store8_act(void* p, int dtype, int64_t i, const float (&v)[8], int64_t valid) {
  if (dtype == kFP32) {
    float* q = static_cast<float*>(p) + i;
    if (valid >= 8 && (reinterpret_cast<uintptr_t>(q) & 15) == 0) {
      typedef float f4_t __attribute__((ext_vector_type(4)));
      *reinterpret_cast<f4_t*>(q) = f4_t{v[0], v[1], v[2], v[3]};
      *reinterpret_cast<f4_t*>(q + 4) = f4_t{v[4], v[5], v[6], v[7]};
      return;
    }
  } else {
    uint16_t* q = static_cast<uint16_t*>(p) + i;
    if (valid >= 8 && (reinterpret_cast<uintptr_t>(q) & 15) == 0) {
      typedef uint32_t u4_t __attribute__((ext_vector_type(4)));
      uint32_t w[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint16_t h0 = dtype == kBF16 ? f32_to_bf16(v[2 * k]) : __builtin_bit_cast(uint16_t, _Float16(v[2 * k]));
        const uint16_t h1 =
            dtype == kBF16 ? f32_to_bf16(v[2 * k + 1]) : __builtin_bit_cast(uint16_t, _Float16(v[2 * k + 1]));
        w[k] = uint32_t(h0) | (uint32_t(h1) << 16);
      }
      *reinterpret_cast<u4_t*>(q) = u4_t{w[0], w[1], w[2], w[3]};
      return;
    }
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    if (k < valid) store_act(p, dtype, i + k, v[k]);
  }
}

constexpr float kH128Scale = 0.08838834764831845f;

// v from lane (lane ^ d) of the wavefront, for d = 1, 2, ..., 32, without
// the address arithmetic of a generic shuffle: DPP quad permutes (d = 1, 2),
// a row shift left / right split by DPP bank mask (d = 4), a row rotate
// (d = 8), ds_swizzle's xor mode within 32 lanes (d = 16) and one
// ds_bpermute (d = 32).  Every lane must be active.
template <int d>
__device__ __forceinline__ float xor_lanes(float v, int lane) {
  const int x = __builtin_bit_cast(int, v);
  int r;
  if constexpr (d == 1) {
    r = __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false);          // quad_perm [1,0,3,2]
  } else if constexpr (d == 2) {
    r = __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false);          // quad_perm [2,3,0,1]
  } else if constexpr (d == 4) {
    r = __builtin_amdgcn_update_dpp(x, x, 0x104, 0xF, 0x5, false);   // row_shl:4, lanes 0-3, 8-11
    r = __builtin_amdgcn_update_dpp(r, x, 0x114, 0xF, 0xA, false);   // row_shr:4, lanes 4-7, 12-15
  } else if constexpr (d == 8) {
    r = __builtin_amdgcn_mov_dpp(x, 0x128, 0xF, 0xF, false);         // row_ror:8
  } else if constexpr (d == 16) {
    r = __builtin_amdgcn_ds_swizzle(x, 0x401F);                      // and 0x1f, xor 0x10
  } else {
    static_assert(d == 32, "xor distance");
    r = __builtin_amdgcn_ds_bpermute((lane ^ 32) << 2, x);
  }
  return __builtin_bit_cast(float, r);
}

// A wavefront-uniform value the compiler cannot prove uniform (read through a
// pointer into memory the kernel also writes, so with a vector load, or
// derived from threadIdx.x / 64) moved to a scalar register: buffer
// resources and scalar offsets built from it then need no per-lane loop.
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ int64_t uniform(int64_t v) {
  const uint64_t u = static_cast<uint64_t>(v);
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(u)));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(u >> 32)));
  return static_cast<int64_t>(uint64_t(lo) | (uint64_t(hi) << 32));
}

// Max over the wavefront (every lane gets it).
__device__ __forceinline__ float wave_max(float v, int lane) {
  v = fmaxf(v, xor_lanes<32>(v, lane));
  v = fmaxf(v, xor_lanes<16>(v, lane));
  v = fmaxf(v, xor_lanes<8>(v, lane));
  v = fmaxf(v, xor_lanes<4>(v, lane));
  v = fmaxf(v, xor_lanes<2>(v, lane));
  v = fmaxf(v, xor_lanes<1>(v, lane));
  return v;
}

// H128 of one 128-value block held by a wavefront: lane l holds elements l
// (v0) and l + 64 (v1).  Butterfly distances 1, 2, ..., 64 in increasing
// order; the lower element becomes lo + hi and the upper one lo - hi (FP32
// round to nearest), then both are scaled by 1/sqrt(128).  The same
// operations in the same order as the reference (reference.cu:107-122,
// codec.cuh:186-209), so the transform is bit-identical to it.  (A lane's
// partner +- v is one FMA, partner + v * (+-1): the product is exact, so it
// rounds as the sum does.)
template <int d>
__device__ __forceinline__ void h128_stage(float& v0, float& v1, int lane) {
  const float o0 = xor_lanes<d>(v0, lane);
  const float o1 = xor_lanes<d>(v1, lane);
  const float sgn = (lane & d) != 0 ? -1.0f : 1.0f;
  v0 = __builtin_fmaf(v0, sgn, o0);
  v1 = __builtin_fmaf(v1, sgn, o1);
}

__device__ __forceinline__ void h128_wave(float& v0, float& v1, int lane) {
  h128_stage<1>(v0, v1, lane);
  h128_stage<2>(v0, v1, lane);
  h128_stage<4>(v0, v1, lane);
  h128_stage<8>(v0, v1, lane);
  h128_stage<16>(v0, v1, lane);
  h128_stage<32>(v0, v1, lane);
  const float lo = v0 + v1;
  const float hi = v0 - v1;
  v0 = lo * kH128Scale;
  v1 = hi * kH128Scale;
}

// H128 of four 128-value blocks held as 16-lane rows: lane (q, l), q =
// lane >> 4, l = lane & 15, holds elements 8 l .. 8 l + 7 of row q's block
// in v[0..7].  The butterfly distances 1, 2, 4 pair elements of one lane, 8,
// 16, 32, 64 the lanes l ^ 1, 2, 4, 8 of the row (DPP): every element gets
// the same additions, in the same order of distances, as h128_wave (lower
// lo + hi, upper lo - hi, FP32 round to nearest), then the scale.  Every
// lane must be active.
__device__ __forceinline__ void h128_rows(float (&v)[8], int l) {
  // every sum rounded on its own: no product of the caller fused into the
  // first additions
#pragma clang fp contract(off)
#pragma unroll
  for (int d = 1; d < 8; d <<= 1) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if ((j & d) == 0) {
        const float lo = v[j], hi = v[j | d];
        v[j] = lo + hi;
        v[j | d] = lo - hi;
      }
    }
  }
  // partner +- v as partner + v * (+-1) in one FMA (exact product)
  auto cross = [&](auto dist) {
    constexpr int d = decltype(dist)::value;
    const float sgn = (l & d) != 0 ? -1.0f : 1.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float o = xor_lanes<d>(v[j], l);
      v[j] = __builtin_fmaf(v[j], sgn, o);
    }
  };
  cross(std::integral_constant<int, 1>{});
  cross(std::integral_constant<int, 2>{});
  cross(std::integral_constant<int, 4>{});
  cross(std::integral_constant<int, 8>{});
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] *= kH128Scale;
}

// s_waitcnt with only vmcnt <= n (the other counters unconstrained), and a
// compiler barrier: LDS reads of data an LDS-DMA load wrote must not move
// above it.
template <int n>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(n >= 0 && n < 64, "vmcnt is six bits");
  __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8));
  asm volatile("" ::: "memory");
}

// s_waitcnt lgkmcnt(0) only: every LDS read issued so far has returned.
__device__ __forceinline__ void wait_lgkmcnt0() {
  __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));
  asm volatile("" ::: "memory");
}

// LDS accesses outside the compiler's tracking of LDS-DMA loads (buffer
// loads into LDS, counted by vmcnt): the compiler waits for every such load
// in flight before an LDS access it cannot prove disjoint from them.  The
// caller guarantees the address is not the destination of a DMA load in
// flight, and orders the access itself (lgkmcnt waits before a barrier).
__device__ __forceinline__ uint32_t lds_address(const void* p) {
  return uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void*)p));
}

__device__ __forceinline__ void lds_store_b16(uint32_t address, uint32_t v) {
  asm volatile("ds_write_b16 %0, %1" ::"v"(address), "v"(v) : "memory");
}

__device__ __forceinline__ void lds_store_b32(uint32_t address, uint32_t v) {
  asm volatile("ds_write_b32 %0, %1" ::"v"(address), "v"(v) : "memory");
}

// Read and wait for it.
__device__ __forceinline__ uint32_t lds_load_b32(uint32_t address) {
  uint32_t v;
  asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(address) : "memory");
  return v;
}

}  // namespace vq
