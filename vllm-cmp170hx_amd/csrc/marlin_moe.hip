// Marlin-format int4 (uint4b8, group 128) fused MoE for gfx950: the grouped
// expert GEMM, the SwiGLU activation, the deterministic token alignment and
// the slot-order top-k sum behind the reference's _ampere_marlin_C operators
// (csrc/ampere_marlin/decode_orig.cu, prefill_tiles.cu) and the upstream
// moe_align_block_size / moe_sum they are called with.
//
// Weights stay in vLLM's Marlin packing (decode_orig.cu:10-19): int32
// [E][K/16][2N], where each 16 (k) x 64 (n) tile of a k16 row is 32 x 16
// bytes, one 16-byte fragment per NVIDIA lane (c = l % 4, g = l / 4) holding
// four 16 x 16 blocks' nibbles for k {2c, 2c+1, 2c+8, 2c+9} and n {g, g+8}.
//
// gfx950 mapping (one wavefront = one 64-column tile):
//  * a step is 32 k (two k16 rows); lane l = 16 q + r loads, coalesced, the
//    16-byte fragment of NVIDIA lane 4 (r % 8) + q from k16 row r / 8 of the
//    pair, so the wavefront reads 1 KB of contiguous weights per step;
//  * lanes r and r + 8 swap words over DPP (row_ror:8) and each keeps, by
//    one v_perm_b32 per word, the bytes of its own output column: lane r then
//    holds 8 nibbles = one v_mfma_f32_16x16x32_{f16,bf16} A operand (row
//    r = column 16 j + r of the tile, k 2q, 2q+1, 2q+8, 2q+9 and the same + 16);
//  * dequant w = RN_act((q - 8) * s) exactly as the reference rounds it
//    (decode_orig.cu:56-67): FP16 by the 0x6400 magic (exact q - 8) and one
//    packed multiply; BF16 by an exact FP32 FMA and v_cvt_pk_bf16_f32;
//  * the tokens of an aligned block (up to 64, in 16-token sub-blocks) are the
//    MFMA's N dimension: activations are staged in LDS in the same k order,
//    so one ds_read_b128 gives a lane its B operand; sub-blocks with no
//    routed token are skipped;
//  * a workgroup is (aligned block, 1 or 4 tiles, k-split); with one tile its
//    four wavefronts split K and sum through LDS in a fixed order.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cmath>
#include <type_traits>

#include "../../include/vllm_mi355x.h"
#include "common.h"
#include "exl3_internal.h"

namespace marlin {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;
constexpr int kMaxBlock = 64;  // tokens per aligned block (upstream block sizes 8..64)

// kPartialAct (marlin_moe_w13_act only): kPartial, then the SwiGLU of each
// (block, 64 gate columns) by the last of its 2 ksplit wavefronts to arrive.
// kTopkSum (marlin_moe_w2_sum only, identity routing): kTopk, then the sum
// over a token's routed slots of each 64 columns by the last of its slots'
// wavefronts to arrive.
enum Mode : int { kPartial = 0, kStore = 1, kTopk = 2, kSwiglu = 3, kPartialAct = 4, kTopkSum = 5 };

struct GemmArgs {
  const uint16_t* a;      // activations, row r at a + r * a_stride
  int64_t a_stride;
  uint32_t a_bytes;       // bytes of a addressable by the kernel
  const u32x4_t* w;       // [E][K/16][N/2] 16-byte fragments
  const uint16_t* s;      // [E][K/128][N] group scales (permuted columns)
  const int32_t* sorted;  // [blocks * bs] routed slot ids, sentinel >= n_slots
  const int32_t* eids;    // [blocks] expert of each block, -1 = none
  const int32_t* ntpp;    // [1] padded routed rows
  const float* topk_w;    // [n_slots] router weights (kTopk)
  float* part;            // kPartial: [ksplit][n_slots][N]
  uint16_t* out;          // kStore / kTopk: row slot at out + slot * out_stride
  int64_t out_stride;
  int top_k, n_slots, K, N, bs, experts, groups_per_split;
  float limit;            // kSwiglu / kPartialAct: SwiGLU clamp (+inf: none)
  uint32_t* counters;     // kPartialAct: this launch's arrival counters, one per (block, gate tile);
                          // kTopkSum: one per (token, tile)
  uint16_t* sum_out;      // kTopkSum: [n_slots / sum_topk][N] slot sums
  int sum_topk;           // kTopkSum: slots per token (a holds one row per slot)
};

// Raw buffer resource over [base, base + bytes): 32-bit offsets, and loads
// past the end return zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, int(bytes), 0x00020000);
}
__device__ __forceinline__ u32x4_t load16(__amdgpu_buffer_rsrc_t r, uint32_t voffset, uint32_t soffset) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, int(voffset), int(soffset), 0));
}

// ---- dequant ---------------------------------------------------------------------

// One word of 8 nibbles (bytes [A.x, B.x, A.y, B.y] of the two k16 rows A and
// B, x / y the nibble pairs of k {2q, 2q+8} / {2q+1, 2q+9}) -> four packed
// pairs, k order (2q, 2q+1) (2q+8, 2q+9) (16+2q, 17+2q) (24+2q, 25+2q).
// FP16: a nibble in mantissa bits 0-3 under 0x6400 is 1024 + q exactly, so
// minus 1032 is q - 8; in bits 4-7 it is 1024 + 16 q, and * 1/16 - 72 is
// q - 8 (one exact FMA); times (s, s) then rounds once.
// (x & mask) | magic as one v_and_or_b32: gfx9's VOP3 takes no 32-bit
// literal, so the compiler would otherwise split it; the constants live in
// VGPRs, set once per kernel.
struct NibbleMasks {
  uint32_t lo, hi, magic;  // 0x000f000f, 0x00f000f0, 0x64006400
};
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t mask, uint32_t magic) {
  uint32_t r;
  asm volatile("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "v"(mask), "v"(magic));
  return r;
}

__device__ __forceinline__ void dequant_f16(uint32_t c, uint32_t s2, const NibbleMasks& k,
                                            uint32_t (&o)[4]) {
  const half2_t s = __builtin_bit_cast(half2_t, s2);
  const half2_t b1032 = {_Float16(1032.0f), _Float16(1032.0f)};
  const half2_t r16 = {_Float16(0.0625f), _Float16(0.0625f)};
  const half2_t m72 = {_Float16(-72.0f), _Float16(-72.0f)};
  const uint32_t c8 = c >> 8;
  const half2_t p0 = __builtin_bit_cast(half2_t, and_or(c, k.lo, k.magic));
  const half2_t p1 = __builtin_bit_cast(half2_t, and_or(c, k.hi, k.magic));
  const half2_t p2 = __builtin_bit_cast(half2_t, and_or(c8, k.lo, k.magic));
  const half2_t p3 = __builtin_bit_cast(half2_t, and_or(c8, k.hi, k.magic));
  o[0] = __builtin_bit_cast(uint32_t, (p0 - b1032) * s);
  o[1] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(p1, r16, m72) * s);
  o[2] = __builtin_bit_cast(uint32_t, (p2 - b1032) * s);
  o[3] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(p3, r16, m72) * s);
}

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  const bf16x2_t v = {__bf16(lo), __bf16(hi)};  // v_cvt_pk_bf16_f32, round to nearest even
  return __builtin_bit_cast(uint32_t, v);
}

// BF16: (q - 8) * s is exact in FP32 (4 x 8 significant bits), so
// fma(q, s, -8 s) is that product and the conversion rounds once.
__device__ __forceinline__ void dequant_bf16(uint32_t c, float s, float ns8, uint32_t (&o)[4]) {
  const uint32_t lo = c & 0x0f0f0f0fu;         // [2q, 16+2q, 2q+1, 17+2q]
  const uint32_t hi = (c >> 4) & 0x0f0f0f0fu;  // [2q+8, 24+2q, 2q+9, 25+2q]
  auto two = [&](uint32_t w, int b0, int b1) {
    const float x0 = __builtin_fmaf(float((w >> (8 * b0)) & 0xffu), s, ns8);
    const float x1 = __builtin_fmaf(float((w >> (8 * b1)) & 0xffu), s, ns8);
    return pack_bf16(x0, x1);
  };
  o[0] = two(lo, 0, 2);
  o[1] = two(hi, 0, 2);
  o[2] = two(lo, 1, 3);
  o[3] = two(hi, 1, 3);
}

// Byte offset, inside an expert's matrix, of this lane's 16-byte fragment
// (NVIDIA lane 4 (r % 8) + q of k16 row r / 8) in step 0 of tile `tile`;
// a step (two k16 rows) adds N * 16 bytes.
__device__ __forceinline__ uint32_t fragment_offset(int N, int tile, int lane) {
  const int q = lane >> 4, r = lane & 15;
  return uint32_t(((r >> 3) * (N >> 1) + tile * 32 + 4 * (r & 7) + q) * 16);
}

// Swap with lane r ^ 8 of the 16-lane row and keep this lane's column's bytes.
__device__ __forceinline__ uint32_t combine(uint32_t own, int lane) {
  const uint32_t other = uint32_t(__builtin_amdgcn_update_dpp(0, int(own), 0x128, 0xf, 0xf, false));
  // r < 8: own = row A, half 0 (bytes 0, 2); r >= 8: own = row B, half 1 (bytes 1, 3)
  return __builtin_amdgcn_perm(other, own, (lane & 8) ? 0x03070105u : 0x06020400u);
}

template <bool kBF16>
struct Scales {
  uint32_t pair[4];  // FP16: (s_j, s_j)
  float s[4], ns8[4];  // BF16: s_j, -8 s_j
  __device__ __forceinline__ void set(u32x4_t v, int lane) {
    const bool high = (lane & 8) != 0;  // column g + 8: the odd stored position
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (kBF16) {
        s[j] = __builtin_bit_cast(float, high ? (v[j] & 0xffff0000u) : (v[j] << 16));
        ns8[j] = -8.0f * s[j];
      } else {
        pair[j] = __builtin_amdgcn_perm(v[j], v[j], high ? 0x03020302u : 0x01000100u);
      }
    }
  }
  __device__ __forceinline__ u32x4_t operand(uint32_t c, int j, const NibbleMasks& k) const {
    uint32_t o[4];
    if constexpr (kBF16) {
      dequant_bf16(c, s[j], ns8[j], o);
    } else {
      dequant_f16(c, pair[j], k, o);
    }
    return u32x4_t{o[0], o[1], o[2], o[3]};
  }
};

template <bool kBF16>
__device__ __forceinline__ f32x4_t mfma(u32x4_t a, u32x4_t b, f32x4_t c) {
  if constexpr (kBF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, a),
                                                  __builtin_bit_cast(half8_t, b), c, 0, 0, 0);
  }
}

template <bool kBF16>
__device__ __forceinline__ float round_act(float v) {
  if constexpr (kBF16) {
    return vq::bf16_to_f32(vq::f32_to_bf16(v));
  } else {
    return float(_Float16(v));
  }
}

template <bool kBF16>
__device__ __forceinline__ uint16_t to_act(float v) {
  if constexpr (kBF16) {
    return vq::f32_to_bf16(v);
  } else {
    return __builtin_bit_cast(uint16_t, _Float16(v));
  }
}

template <bool kBF16>
__device__ __forceinline__ float act_f32(uint16_t v) {
  return kBF16 ? vq::bf16_to_f32(v) : vq::f16_to_f32(v);
}

// h = RN(RN(SiLU(min(G, L))) * clamp(U, -L, L)), G and U the activation-dtype
// roundings of the gate and up sums (decode_orig.cu:272-305).
template <bool kBF16>
__device__ __forceinline__ uint16_t swiglu(float gs, float us, float limit) {
  const float gv = fminf(round_act<kBF16>(gs), limit);
  const float uv = fmaxf(fminf(round_act<kBF16>(us), limit), -limit);
  const float sl = round_act<kBF16>(gv / (1.0f + expf(-gv)));
  return to_act<kBF16>(sl * uv);
}

using exl3::kCachePolicySc1;
using exl3::kCounterStride;

// ---- grouped GEMM -----------------------------------------------------------------

// kTilesWG: 64-column tiles per workgroup (1: its four wavefronts split K;
// 4: one tile per wavefront, all of K); kSub: 16-token sub-blocks (block
// size <= 16 kSub).  Each wavefront streams whole 128-k groups (4 steps and
// their scales) through a 3-slot register ring, two groups ahead.
template <bool kBF16, int kTilesWG, int kSub, int kMode>
__global__ __launch_bounds__(kThreads, 2) void marlin_gemm(GemmArgs g) {
  constexpr int kWavesK = 4 / kTilesWG;
  constexpr int kRounds = 1;                         // groups per wavefront per chunk
  constexpr int kChunkGroups = kWavesK * kRounds;   // 128-k groups per LDS chunk
  constexpr int kChunkSteps = 4 * kChunkGroups;
  constexpr int kTok = 16 * kSub;
  constexpr int kStepBytes = 4 * kTok * 16;          // [q][token][8 halves]
  constexpr int kChunkBytes = kChunkSteps * kStepBytes;
  constexpr int kStage = kChunkSteps * kTok * 4 / kThreads;  // 16-byte loads per thread
  constexpr int kStageStride = kThreads / (4 * kTok);        // steps between a thread's loads
  static_assert(kStage >= 1 && kChunkSteps * kTok * 4 % kThreads == 0, "staging split");
  constexpr int kRedBytes = (kWavesK - 1) * 64 * 4 * kSub * 16 * kTilesWG;
  constexpr int kLds = 2 * kChunkBytes > kRedBytes ? 2 * kChunkBytes : kRedBytes;
  __shared__ __attribute__((aligned(16))) uint8_t lds[kLds];
  __shared__ int s_slot[kMaxBlock];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wk = wave % kWavesK;
  const int wt = wave / kWavesK;
  const int tile = int(blockIdx.x) * kTilesWG + wt;
  const bool tile_ok = tile < (g.N >> 6);
  const int b = blockIdx.y;
  const int ks = blockIdx.z;
  if (g.sorted && int64_t(b) * g.bs >= int64_t(g.ntpp[0])) return;
  // (a vector load: the kernel writes memory the compiler cannot tell apart)
  const int e = vq::uniform(g.eids[b]);
  if (e < 0 || e >= g.experts) {
    if constexpr (kMode == kTopkSum) {
      // a token none of whose slots is routed has no arriving wavefront to
      // write its sum: the block of its first slot writes the zero sum
      const int topk = g.sum_topk;
      const int t = b / topk;
      if (b != t * topk || !tile_ok || wk != 0) return;
      const int32_t* tok_ids = g.eids + int64_t(t) * topk;
      for (int k = 0; k < topk; ++k) {
        const int id = tok_ids[k];
        if (id >= 0 && id < g.experts) return;
      }
      g.sum_out[int64_t(t) * g.N + 64 * tile + lane] = to_act<kBF16>(0.0f);
    }
    return;
  }
  if (tid < kMaxBlock) {
    int slot = -1;
    if (!g.sorted) {
      slot = tid == 0 ? b : -1;  // identity routing: block b is slot b alone
    } else if (tid < g.bs) {
      const int sid = g.sorted[int64_t(b) * g.bs + tid];
      if (sid >= 0 && sid < g.n_slots) slot = sid;
    }
    s_slot[tid] = slot;
  }
  __syncthreads();
  const uint64_t valid = __ballot(s_slot[lane] >= 0);
  if (valid == 0) return;
  const int nvalid = 64 - __builtin_clzll(valid);
  const int nsub = (nvalid + 15) >> 4;  // sub-blocks holding a routed token

  const int gps = g.groups_per_split;
  const int g0 = ks * gps;
  const int nch = (gps + kChunkGroups - 1) / kChunkGroups;
  const int groups_total = g.K >> 7;
  const __amdgpu_buffer_rsrc_t wbuf =
      buffer(g.w + int64_t(e) * (g.K >> 4) * (g.N >> 1), uint32_t(g.K >> 4) * uint32_t(g.N >> 1) * 16u);
  const __amdgpu_buffer_rsrc_t sbuf =
      buffer(g.s + int64_t(e) * groups_total * g.N, uint32_t(groups_total) * uint32_t(g.N) * 2u);
  const __amdgpu_buffer_rsrc_t abuf_g = buffer(g.a, g.a_bytes);
  const uint32_t wstep = uint32_t(g.N) * 16u;  // bytes per step
  uint32_t woff[4];
#pragma unroll
  for (int st = 0; st < 4; ++st) woff[st] = fragment_offset(g.N, tile, lane) + st * wstep;
  const uint32_t soff = uint32_t(tile * 64 + 8 * (lane & 7)) * 2u;

  // activation staging: thread = (16-byte segment, token, first step)
  const int seg = tid & 3;
  const int tok = (tid >> 2) % kTok;
  const int st0 = tid / (4 * kTok);
  const int tslot = s_slot[tok];
  const uint32_t aoff = tslot >= 0
      ? uint32_t((int64_t(tslot / g.top_k) * g.a_stride + 8 * seg + 32 * st0) * 2)
      : 0x80000000u;  // past the buffer: loads return zero
  uint8_t* lds_stage = lds + st0 * kStepBytes + tok * 16 + 4 * seg;
  u32x4_t stage_regs[kStage];
  auto stage_load = [&](int c) {
    const uint32_t kbase = uint32_t(g0 + c * kChunkGroups) * 256u;  // bytes of 128 k
#pragma unroll
    for (int u = 0; u < kStage; ++u) {
      stage_regs[u] = load16(abuf_g, aoff + uint32_t(u * kStageStride * 64), kbase);
    }
  };
  auto stage_store = [&](int buf) {
#pragma unroll
    for (int u = 0; u < kStage; ++u) {
      uint8_t* base = lds_stage + buf * kChunkBytes + u * kStageStride * kStepBytes;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        *reinterpret_cast<uint32_t*>(base + d * kTok * 16) = stage_regs[u][d];
      }
    }
  };

  // this wavefront's groups: i -> chunk i / kRounds, round i % kRounds
  auto group_of = [&](int i) { return g0 + (i / kRounds) * kChunkGroups + (i % kRounds) * kWavesK + wk; };
  const int my_groups = nch * kRounds;
  u32x4_t ring_w[3][4];
  u32x4_t ring_s[3];
  auto load_group = [&](int slot, int i) {
    const int grp = group_of(i);
    if (tile_ok && grp < g0 + gps) {
      const uint32_t gbase = uint32_t(grp) * 4u * wstep;
#pragma unroll
      for (int st = 0; st < 4; ++st) ring_w[slot][st] = load16(wbuf, woff[st], gbase);
      ring_s[slot] = load16(sbuf, soff, uint32_t(grp) * uint32_t(g.N) * 2u);
    }
  };

  load_group(0, 0);
  if (my_groups > 1) load_group(1, 1);
  stage_load(0);
  stage_store(0);
  if (nch > 1) stage_load(1);
  __syncthreads();

  const int q = lane >> 4;
  const int col = lane & 15;
  NibbleMasks masks;
  masks.lo = 0x000f000fu;
  masks.hi = 0x00f000f0u;
  masks.magic = 0x64006400u;

  // The main loop and epilogue for the first kNs sub-blocks (those holding a
  // routed token), specialized once per workgroup.
  auto run = [&](auto ns_tag) {
    constexpr int kNs = decltype(ns_tag)::value;
    f32x4_t acc[4][kNs];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int sb = 0; sb < kNs; ++sb) acc[j][sb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

    // group i of this wavefront from ring slot kSlot (static, so the ring
    // stays in registers); the last group of a chunk refills the other LDS
    // buffer
    auto body = [&](int i, auto slot_tag) {
      constexpr int kSlot = decltype(slot_tag)::value;
      const int c = i / kRounds;
      const int r = i % kRounds;
      const int grp = group_of(i);
      if (i + 2 < my_groups) load_group((kSlot + 2) % 3, i + 2);
      if (tile_ok && grp < g0 + gps) {
        const uint8_t* abuf = lds + (c & 1) * kChunkBytes;
        Scales<kBF16> sc;
        sc.set(ring_s[kSlot], lane);
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          const u32x4_t v = ring_w[kSlot][st];
          const int stepc = (r * kWavesK + wk) * 4 + st;
          u32x4_t bop[kNs];
#pragma unroll
          for (int sb = 0; sb < kNs; ++sb) {
            bop[sb] = *reinterpret_cast<const u32x4_t*>(abuf + stepc * kStepBytes +
                                                        (q * kTok + 16 * sb + col) * 16);
          }
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const u32x4_t a = sc.operand(combine(v[j], lane), j, masks);
#pragma unroll
            for (int sb = 0; sb < kNs; ++sb) acc[j][sb] = mfma<kBF16>(a, bop[sb], acc[j][sb]);
          }
        }
      }
      if (r == kRounds - 1) {
        if (c + 1 < nch) stage_store((c + 1) & 1);
        if (c + 2 < nch) stage_load(c + 2);
        __syncthreads();
      }
    };
    for (int i = 0; i < my_groups; i += 3) {
      body(i, std::integral_constant<int, 0>{});
      if (i + 1 < my_groups) body(i + 1, std::integral_constant<int, 1>{});
      if (i + 2 < my_groups) body(i + 2, std::integral_constant<int, 2>{});
    }

    // split-K inside the workgroup: wavefronts 1.. of a tile hand their sums
    // to wavefront 0 of it, which adds them in order 1, 2, 3
    if constexpr (kWavesK > 1) {
      float* red = reinterpret_cast<float*>(lds);
      auto red_at = [&](int from, int j, int sb) {
        return red + ((((wt * (kWavesK - 1) + from - 1) * 4 + j) * kSub + sb) * 64 + lane) * 4;
      };
      if (wk > 0) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int sb = 0; sb < kNs; ++sb) *reinterpret_cast<f32x4_t*>(red_at(wk, j, sb)) = acc[j][sb];
      }
      __syncthreads();
      if (wk > 0) return;
#pragma unroll
      for (int from = 1; from < kWavesK; ++from)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int sb = 0; sb < kNs; ++sb) acc[j][sb] += *reinterpret_cast<const f32x4_t*>(red_at(from, j, sb));
    }
    if (!tile_ok) return;

    // the router weights before the first store (loads and stores share one
    // in-order counter: a load waited for after a store waits for it too)
    float wts[kNs];
#pragma unroll
    for (int sb = 0; sb < kNs; ++sb) {
      const int slot = s_slot[16 * sb + col];
      wts[sb] = (kMode == kTopk || kMode == kTopkSum) && slot >= 0 ? round_act<kBF16>(g.topk_w[slot]) : 0.0f;
    }
    // kPartialAct: the partials of every K split; kTopkSum: the slot rows
    // (each fewer than 2^31 bytes)
    const __amdgpu_buffer_rsrc_t part_buf = buffer(g.part, uint32_t(gridDim.z) * uint32_t(g.n_slots) * uint32_t(g.N) * 4u);
    const __amdgpu_buffer_rsrc_t out_buf = buffer(g.out, uint32_t(g.n_slots) * uint32_t(g.out_stride) * 2u);
    // C fragment: lane holds columns 16 j + 4 q .. +3 of token 16 sb + col
#pragma unroll
    for (int sb = 0; sb < kNs; ++sb) {
      const int slot = s_slot[16 * sb + col];
      if (slot < 0) continue;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t n = int64_t(tile) * 64 + 16 * j + 4 * q;
        const f32x4_t v = acc[j][sb];
        if constexpr (kMode == kPartial) {
          *reinterpret_cast<f32x4_t*>(g.part + (int64_t(ks) * g.n_slots + slot) * g.N + n) = v;
        } else if constexpr (kMode == kPartialAct) {
          // through to the device-coherent level: the finishing wavefront
          // may run on another XCD
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), part_buf,
                                                 int(4 * ((int64_t(ks) * g.n_slots + slot) * g.N + n)), 0,
                                                 kCachePolicySc1);
        } else {
          float x[4] = {v[0], v[1], v[2], v[3]};
          if constexpr (kMode == kTopk || kMode == kTopkSum) {
            const float w = wts[sb];
#pragma unroll
            for (int u = 0; u < 4; ++u) x[u] = round_act<kBF16>(x[u]) * w;  // exact product
          }
          const u32x2_t packed = {uint32_t(to_act<kBF16>(x[0])) | (uint32_t(to_act<kBF16>(x[1])) << 16),
                                  uint32_t(to_act<kBF16>(x[2])) | (uint32_t(to_act<kBF16>(x[3])) << 16)};
          if constexpr (kMode == kTopkSum) {
            // through to the device-coherent level, as kPartialAct's partials
            __builtin_amdgcn_raw_buffer_store_b64(packed, out_buf, int(2 * (int64_t(slot) * g.out_stride + n)), 0,
                                                  kCachePolicySc1);
          } else {
            *reinterpret_cast<u32x2_t*>(g.out + int64_t(slot) * g.out_stride + n) = packed;
          }
        }
      }
    }
    if constexpr (kMode == kTopkSum) {
      // identity routing: block b is slot b of token b / sum_topk.  One arrival
      // per wavefront once its stores have completed; the last of the
      // token's routed slots (ids in [0, experts)) forms moe_sum_kernel's
      // FP32 slot-order sum of this tile's 64 columns
      __builtin_amdgcn_s_waitcnt(0);
      const int topk = g.sum_topk;
      const int t = b / topk;
      // the token's routed slots as bits (topk <= 64)
      const int32_t* tok_ids = g.eids + int64_t(t) * topk;
      uint64_t routed = 0;
      for (int k = 0; k < topk; ++k) {
        const int id = tok_ids[k];
        if (id >= 0 && id < g.experts) routed |= uint64_t(1) << k;
      }
      const uint32_t expected = uint32_t(__builtin_popcountll(routed));
      uint32_t* counter = g.counters + (int64_t(t) * (g.N >> 6) + tile) * kCounterStride;
      uint32_t arrived = 0;
      if (lane == 0) arrived = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      arrived = __builtin_amdgcn_readfirstlane(arrived);
      if (arrived != expected - 1u) return;
      const int n = 64 * tile + lane;
      float acc = 0.0f;
      // eight slots' loads in flight per round, summed in slot order
      for (int k0 = 0; k0 < topk; k0 += 8) {
        bool use[8];
        uint16_t v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          use[u] = k0 + u < topk && ((routed >> (k0 + u)) & 1) != 0;
          const int row = t * topk + min(k0 + u, topk - 1);
          v[u] = __builtin_amdgcn_raw_buffer_load_b16(out_buf, 2 * (row * int(g.out_stride) + n), 0, kCachePolicySc1);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          if (use[u]) acc += act_f32<kBF16>(v[u]);
        }
      }
      g.sum_out[int64_t(t) * g.N + n] = to_act<kBF16>(acc);
      if (lane == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if constexpr (kMode == kPartialAct) {
      // one arrival per wavefront once its stores have completed (vmcnt
      // counts stores); tiles t and t + Nh / 64 (gate and up) of every K
      // split share the counter of (block b, gate tile)
      __builtin_amdgcn_s_waitcnt(0);
      const int gate_tiles = g.N >> 7;
      const int tg = tile < gate_tiles ? tile : tile - gate_tiles;
      uint32_t* counter = g.counters + (int64_t(b) * gate_tiles + tg) * kCounterStride;
      uint32_t arrived = 0;
      if (lane == 0) arrived = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      arrived = __builtin_amdgcn_readfirstlane(arrived);
      if (arrived != 2u * gridDim.z - 1u) return;
      // the last: marlin_act_kernel's sums and rounding for columns 64 tg +
      // lane of the block's slots, the partials read at the coherent level
      const int nh = g.N >> 1;
      const int n = 64 * tg + lane;
      const int plane = 4 * g.n_slots * g.N;
      for (int i = 0; i < g.bs; ++i) {
        const int slot = s_slot[i];
        if (slot < 0) continue;
        const int off = 4 * (slot * g.N + n);
        const int splits = int(gridDim.z);
        float gs = 0.0f, us = 0.0f;
        // eight splits' loads in flight per round (indices past the last
        // split clamped, their terms not added), summed in split order
        for (int k0 = 0; k0 < splits; k0 += 8) {
          float gp[8], up[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const int k = min(k0 + u, splits - 1);
            gp[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(part_buf, off, k * plane, kCachePolicySc1));
            up[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(part_buf, off + 4 * nh, k * plane,
                                                                                   kCachePolicySc1));
          }
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            if (k0 + u < splits) {
              gs += gp[u];
              us += up[u];
            }
          }
        }
        g.out[int64_t(slot) * g.out_stride + n] = swiglu<kBF16>(gs, us, g.limit);
      }
      if (lane == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  };
  if constexpr (kSub == 1) {
    run(std::integral_constant<int, 1>{});
  } else if constexpr (kSub == 2) {
    if (nsub == 1) run(std::integral_constant<int, 1>{});
    else run(std::integral_constant<int, 2>{});
  } else {
    if (nsub == 1) run(std::integral_constant<int, 1>{});
    else if (nsub == 2) run(std::integral_constant<int, 2>{});
    else if (nsub == 3) run(std::integral_constant<int, 3>{});
    else run(std::integral_constant<int, 4>{});
  }
}


// ---- grouped GEMM on k-permuted activations (the fused path) -------------------

// Position, inside its 32-k step, of activation k in the permuted layout the
// direct GEMM reads: element 8 q + 2 s + t of a step holds k = 8 s + 2 q + t,
// so lane (q, token) finds its whole B operand (k {2q, 2q+1, 2q+8, 2q+9,
// 16+2q, 17+2q, 24+2q, 25+2q}, the A operand's order) in 16 contiguous bytes.
__host__ __device__ __forceinline__ int permuted_k(int k) {
  const int w = k & 31;
  return (k & ~31) + 8 * ((w >> 1) & 3) + 2 * (w >> 3) + (w & 1);
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// As marlin_gemm, but:
//  * each wavefront owns direct_tiles 64-column tiles over the workgroup's
//    whole K range (with two, every B operand it loads feeds both tiles'
//    MFMAs);
//  * weights stream through a per-wavefront LDS ring of direct_slots
//    half-groups (64 k of its tiles, buffer_load_dwordx4 ... lds: no VGPR
//    staging);
//  * each lane loads its B operands straight from k-permuted activations
//    (one 16-byte load per step and 16-token sub-block, one group ahead), so
//    there is no activation staging and no workgroup barrier in the loop;
//  * kSwiglu: wavefronts 0, 1 take gate tiles and wavefronts 2, 3 the
//    matching up tiles (N / 128 further on): the up sums meet the gate sums
//    in LDS and h = RN(RN(SiLU(min(G, L))) * clamp(U, -L, L)) is written in
//    the permuted layout (the w2 GEMM's input), G / U the activation-dtype
//    roundings of the FP32 sums (marlin_act_kernel's arithmetic).
// The MFMA sequence per tile is marlin_gemm's, so the sums are bitwise the
// same.
// Tiles per wavefront and ring slots (half-groups) per wavefront by mode.
// kSwiglu: one tile per wavefront (a workgroup = two gate tiles and their
// up tiles), so the GPU holds every workgroup of a 256-token w13 at once
// and its VALU dequant spreads over more wavefronts; three half-groups
// ahead.  The other modes: two tiles per wavefront (each B operand feeds
// both) for blocks of more than 16 tokens, one tile for blocks of up to 16
// (the few-token forwards, whose few routed blocks then give twice the
// wavefronts streaming weights); one half-group ahead.
template <int kMode, int kSub>
struct DirectShape {
  static constexpr int kTiles = kMode == kSwiglu || kSub == 1 ? 1 : 2;
  static constexpr int kSlots = 2;
  // kSwiglu: the B operands go through LDS too (all four wavefronts read the
  // same rows): two group slots
  static constexpr bool kLdsB = kMode == kSwiglu;
};
inline int direct_tiles(int mode, int sub) { return mode == kSwiglu || sub == 1 ? 1 : 2; }
// The kernel's per-tile arrays have this fixed size (loops run to the mode's
// tile count): arrays whose size depends on the template arguments, captured
// by the kernel's lambdas, make the host compilation drop the kernel's launch
// stub.
constexpr int kMaxDirectTiles = 2;
template <bool kBF16, int kSub, int kMode>
__global__ __launch_bounds__(kThreads, kSub <= 2 ? 3 : 2) void marlin_gemm_direct(GemmArgs g) {
  constexpr int kDirectTiles = DirectShape<kMode, kSub>::kTiles;
  constexpr int kSlots = DirectShape<kMode, kSub>::kSlots;
  // ring slot = [wavefront][tile][step of the half-group][64 lanes] x 16 bytes
  constexpr int kSlotVecs = 4 * kDirectTiles * 2 * 64;
  __shared__ __attribute__((aligned(16))) u32x4_t ring0[kSlotVecs];
  __shared__ __attribute__((aligned(16))) u32x4_t ring1[kSlotVecs];
  __shared__ __attribute__((aligned(16))) u32x4_t ring2[kSlots > 2 ? kSlotVecs : 4];
  __shared__ __attribute__((aligned(16))) u32x4_t ring3[kSlots > 2 ? kSlotVecs : 4];
  // B slot = [row / 4][row % 4][16-byte chunk ^ (row % 16)] of 16 bytes: one
  // group (128 k) of the block's rows (the chunk swizzle keeps the 16 rows a
  // B-operand read touches on distinct banks), then per wavefront 256 bytes:
  // its tile's group scales (128 bytes) and zeros
  constexpr bool kLdsB = DirectShape<kMode, kSub>::kLdsB;
  constexpr int kBRowVecs = kSub * 16 * 16;
  constexpr int kBVecs = kLdsB ? kBRowVecs + 4 * 16 : 4;
  __shared__ __attribute__((aligned(16))) u32x4_t bring0[kBVecs];
  __shared__ __attribute__((aligned(16))) u32x4_t bring1[kBVecs];
  __shared__ int s_slot[kMaxBlock];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q = lane >> 4;
  const int col = lane & 15;
  int tiles[kMaxDirectTiles];
  bool tile_ok[kMaxDirectTiles];
#pragma unroll
  for (int x = 0; x < kDirectTiles; ++x) {
    if constexpr (kMode == kSwiglu) {
      const int gate_tiles = g.N >> 7;
      const int gt = 2 * kDirectTiles * int(blockIdx.x) + kDirectTiles * (wave & 1) + x;  // gate tile
      tiles[x] = wave < 2 ? gt : gate_tiles + gt;
      tile_ok[x] = gt < gate_tiles;
    } else {
      tiles[x] = 4 * kDirectTiles * int(blockIdx.x) + kDirectTiles * wave + x;
      tile_ok[x] = tiles[x] < (g.N >> 6);
    }
  }
  const int b = blockIdx.y;
  const int ks = blockIdx.z;
  if (g.sorted && int64_t(b) * g.bs >= int64_t(g.ntpp[0])) return;
  // (a vector load: the kernel writes memory the compiler cannot tell apart)
  const int e = vq::uniform(g.eids[b]);
  if (e < 0 || e >= g.experts) return;
  if (tid < kMaxBlock) {
    int slot = -1;
    if (!g.sorted) {
      slot = tid == 0 ? b : -1;  // identity routing: block b is slot b alone
    } else if (tid < g.bs) {
      const int sid = g.sorted[int64_t(b) * g.bs + tid];
      if (sid >= 0 && sid < g.n_slots) slot = sid;
    }
    s_slot[tid] = slot;
  }
  __syncthreads();
  const uint64_t valid = __ballot(s_slot[lane] >= 0);
  if (valid == 0) return;
  const int nvalid = 64 - __builtin_clzll(valid);
  const int nsub = (nvalid + 15) >> 4;

  const int gps = g.groups_per_split;
  const int g0 = ks * gps;
  const int groups_total = g.K >> 7;
  const uint32_t wstep = uint32_t(g.N) * 16u;
  // Buffers over this split's groups only: the loop below issues every load
  // unconditionally (a load that a branch may skip makes the compiler's
  // count of loads in flight unknown, and it then waits for all of them),
  // and the loads of the group after the last fall past the end and return
  // zeros without touching memory.
  const __amdgpu_buffer_rsrc_t wbuf =
      buffer(g.w + (int64_t(e) * (g.K >> 4) + int64_t(g0) * 8) * (g.N >> 1), uint32_t(gps) * 4u * wstep);
  const __amdgpu_buffer_rsrc_t sbuf =
      buffer(g.s + (int64_t(e) * groups_total + g0) * g.N, uint32_t(gps) * uint32_t(g.N) * 2u);
  const __amdgpu_buffer_rsrc_t abuf = buffer(g.a, g.a_bytes);
  // a missing tile streams tile 0 and stores nothing
  uint32_t woff[kMaxDirectTiles], soff[kMaxDirectTiles];
#pragma unroll
  for (int x = 0; x < kDirectTiles; ++x) {
    const int t = tile_ok[x] ? tiles[x] : 0;
    woff[x] = fragment_offset(g.N, t, lane);
    soff[x] = uint32_t(t * 64 + 8 * (lane & 7)) * 2u;
  }
  uint32_t boff[kSub];
#pragma unroll
  for (int sb = 0; sb < kSub; ++sb) {
    const int slot = s_slot[16 * sb + col];
    boff[sb] = slot >= 0 ? uint32_t((int64_t(slot / g.top_k) * g.a_stride + 8 * q) * 2) : 0x80000000u;
  }

  auto slot_base = [&](int k) -> u32x4_t* {
    return (k == 0 ? ring0 : (k == 1 ? ring1 : (k == 2 ? ring2 : ring3))) + wave * (kDirectTiles * 2 * 64);
  };
  // half-group (group i of the split, steps 2 half, 2 half + 1) of both
  // tiles into ring slot k
  auto load_half = [&](int k, int i, int half) {
#pragma unroll
    for (int x = 0; x < kDirectTiles; ++x) {
#pragma unroll
      for (int sl = 0; sl < 2; ++sl) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(wbuf, (lds_ptr_t)(slot_base(k) + (2 * x + sl) * 64), 16,
                                                 woff[x], int(uint32_t(4 * i + 2 * half + sl) * wstep), 0, 0);
      }
    }
  };
  u32x4_t s_next[kMaxDirectTiles];
  auto load_scales = [&](int i) {
#pragma unroll
    for (int x = 0; x < kDirectTiles; ++x) s_next[x] = load16(sbuf, soff[x], uint32_t(i) * uint32_t(g.N) * 2u);
  };

  NibbleMasks masks;
  masks.lo = 0x000f000fu;
  masks.hi = 0x00f000f0u;
  masks.magic = 0x64006400u;

  auto run = [&](auto ns_tag) {
    constexpr int kNs = decltype(ns_tag)::value;
    f32x4_t acc[kMaxDirectTiles][4][kNs];
#pragma unroll
    for (int x = 0; x < kDirectTiles; ++x)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int sb = 0; sb < kNs; ++sb) acc[x][j][sb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (kLdsB) {
      // The block's B operands of group i go to B slot i % 2 in 4 kNs
      // loads of four rows (1 KB) each, kNs per wavefront: lane l fetches row
      // 4d + l / 16, chunk (l % 16) ^ (row % 16).  Group i starts with this
      // wavefront's own B loads of group i complete, then a workgroup
      // barrier: every wavefront's loads of group i have landed and every
      // wavefront is done with group i - 1, whose B slot group i + 1 reuses.
      uint32_t brow[kNs];
#pragma unroll
      for (int j = 0; j < kNs; ++j) {
        const int row = 4 * (wave * kNs + j) + (lane >> 4);
        const int slot = s_slot[row];
        const int chunk = (lane & 15) ^ (row & 15);
        brow[j] = slot >= 0 ? uint32_t((int64_t(slot / g.top_k) * g.a_stride + 8 * chunk) * 2) : 0x80000000u;
      }
      // the scales go through LDS as well (dword loads, lanes 0-31; the others
      // fall past the buffer): a VGPR load here would be the loop's only one,
      // and the compiler, which does not count the LDS loads issued after it,
      // would wait for every load in flight before its first use
      const uint32_t sdw = lane < 32 ? uint32_t(tile_ok[0] ? tiles[0] : 0) * 128u + 4u * uint32_t(lane) : 0x80000000u;
      auto load_bgroup = [&](int k, int i) {
        u32x4_t* slot = k == 0 ? bring0 : bring1;
#pragma unroll
        for (int j = 0; j < kNs; ++j) {
          __builtin_amdgcn_raw_ptr_buffer_load_lds(abuf, (lds_ptr_t)(slot + (wave * kNs + j) * 64), 16, brow[j],
                                                   int(uint32_t(g0 + i) * 256u), 0, 0);
        }
        __builtin_amdgcn_raw_ptr_buffer_load_lds(sbuf, (lds_ptr_t)(slot + kBRowVecs + wave * 16), 4, sdw,
                                                 int(uint32_t(i) * uint32_t(g.N) * 2u), 0, 0);
      };
      // this lane's B operand of step st, sub-block sb in a B slot
      auto bread = [&](int k, int st, int sb) {
        const int row = 16 * sb + col;
        const int chunk = 4 * st + q;
        return (k == 0 ? bring0 : bring1)[(row >> 2) * 64 + (row & 3) * 16 + (chunk ^ (row & 15))];
      };
      // per group i: [wait own B(i), barrier] [B(i + 1)] [weights of half 1,
      // scales of i + 1] steps 0, 1 [weights of i + 1's half 0] steps 2, 3
      load_bgroup(0, 0);
      load_half(0, 0, 0);
      for (int i0 = 0; i0 < gps; i0 += 2) {
#pragma unroll
        for (int gi = 0; gi < 2; ++gi) {
          const int i = i0 + gi;
          const bool live = i < gps;
          // only the two weight loads of this group's half 0 in flight: B(i)
          // and the scales of i have landed
          vq::wait_vmcnt<2>();
          __builtin_amdgcn_s_barrier();
          asm volatile("" ::: "memory");
          Scales<kBF16> sc;
          sc.set((gi == 0 ? bring0 : bring1)[kBRowVecs + wave * 16 + (lane & 7)], lane);
          load_bgroup(gi ^ 1, i + 1);
#pragma unroll
          for (int half = 0; half < 2; ++half) {
            if (half == 0) {
              load_half(1, i, 1);
            } else {
              load_half(0, i + 1, 0);
            }
            asm volatile("" ::: "memory");
            if (live) {
#pragma unroll
              for (int sl = 0; sl < 2; ++sl) {
                const int st = 2 * half + sl;
                u32x4_t bop[kNs];
#pragma unroll
                for (int sb = 0; sb < kNs; ++sb) bop[sb] = bread(gi, st, sb);
                const u32x4_t v = slot_base(half)[sl * 64 + lane];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                  const u32x4_t a = sc.operand(combine(v[j], lane), j, masks);
#pragma unroll
                  for (int sb = 0; sb < kNs; ++sb) acc[0][j][sb] = mfma<kBF16>(a, bop[sb], acc[0][j][sb]);
                }
              }
            }
          }
        }
      }
    } else {
    // B operands of the current group's steps; step st of the next group is
    // loaded into breg[st] as soon as step st of this one has been read
    u32x4_t breg[4][kNs];
    // (a B offset past the split's last group reads the next k, or past
    // the buffer: zeros; either way unused)
    auto load_b = [&](int st, int i) {
#pragma unroll
      for (int sb = 0; sb < kNs; ++sb) breg[st][sb] = load16(abuf, boff[sb], uint32_t((g0 + i) * 128 + 32 * st) * 2u);
    };
    // Issue order matters too: vmcnt retires loads in order, so a wait for
    // a B operand also waits for every load issued before it.  Half-group h
    // (ring slot h % kSlots) starts by issuing the weights of half-group
    // h + kSlots - 1 into the slot read in half-group h - 1 (and, at a group's
    // start, the next group's scales); then per step the MFMAs and the B
    // operands of the same step of the next group (into the registers just
    // read: no copies).  Every wait then names data that is due, and each
    // weight load has kSlots - 1 half-groups to land.  The loop runs whole
    // rounds of kSlots / 2 groups; a group past the split (odd gps) only
    // issues its loads, which fall past the buffers.
    auto half_group = [&](int i, int half) { load_half((2 * i + half) % kSlots, i, half); };
#pragma unroll
    for (int h = 0; h < kSlots - 1; ++h) {
      half_group(h / 2, h % 2);
      if (h == 0) {
        load_scales(0);
#pragma unroll
        for (int st = 0; st < 4; ++st) load_b(st, 0);
      }
    }

    for (int i0 = 0; i0 < gps; i0 += kSlots / 2) {
#pragma unroll
      for (int gi = 0; gi < kSlots / 2; ++gi) {
        const int i = i0 + gi;
        const bool live = i < gps;
        Scales<kBF16> sc[kMaxDirectTiles];
#pragma unroll
        for (int x = 0; x < kDirectTiles; ++x) sc[x].set(s_next[x], lane);
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          const int h = 2 * gi + half;  // slot
          const int ahead = 2 * i + half + kSlots - 1;
          half_group(ahead / 2, ahead % 2);
          if (half == 0) load_scales(i + 1);
          asm volatile("" ::: "memory");
#pragma unroll
          for (int sl = 0; sl < 2; ++sl) {
            const int st = 2 * half + sl;
            if (live) {
#pragma unroll
              for (int x = 0; x < kDirectTiles; ++x) {
                const u32x4_t v = slot_base(h)[(2 * x + sl) * 64 + lane];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                  const u32x4_t a = sc[x].operand(combine(v[j], lane), j, masks);
#pragma unroll
                  for (int sb = 0; sb < kNs; ++sb) acc[x][j][sb] = mfma<kBF16>(a, breg[st][sb], acc[x][j][sb]);
                }
              }
            }
            load_b(st, i + 1);
            asm volatile("" ::: "memory");
          }
        }
      }
    }

    }  // kLdsB

    if constexpr (kMode == kSwiglu) {
      // up wavefronts 2, 3 hand their sums to gate wavefronts 0, 1 through
      // ring slots 0, 1 (every wavefront's ring reads are done, and its loads
      // past the split have landed), two 16-token sub-blocks per round
      u32x4_t* xbase = wave == 2 || wave == 0 ? ring0 : ring1;
      auto xch = [&](int x, int j, int sbl) {
        return reinterpret_cast<f32x4_t*>(xbase) + ((x * 4 + j) * 2 + sbl) * 64 + lane;
      };
#pragma unroll
      for (int r0 = 0; r0 < kNs; r0 += 2) {
        __syncthreads();
        if (wave >= 2) {
#pragma unroll
          for (int x = 0; x < kDirectTiles; ++x)
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
              for (int sbl = 0; sbl < 2; ++sbl)
                if (r0 + sbl < kNs) *xch(x, j, sbl) = acc[x][j][r0 + sbl];
        }
        __syncthreads();
        if (wave < 2) {
#pragma unroll
          for (int x = 0; x < kDirectTiles; ++x) {
            if (!tile_ok[x]) continue;
#pragma unroll
            for (int sbl = 0; sbl < 2; ++sbl) {
              const int sb = r0 + sbl;
              if (sb >= kNs) continue;
              const int slot = s_slot[16 * sb + col];
              if (slot < 0) continue;
#pragma unroll
              for (int j = 0; j < 4; ++j) {
                const f32x4_t u = *xch(x, j, sbl);
                const f32x4_t gsum = acc[x][j][sb];
                uint16_t hv[4];
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                  const float gv = fminf(round_act<kBF16>(gsum[c]), g.limit);
                  const float uv = fmaxf(fminf(round_act<kBF16>(u[c]), g.limit), -g.limit);
                  const float sl = round_act<kBF16>(gv / (1.0f + expf(-gv)));
                  hv[c] = to_act<kBF16>(sl * uv);
                }
                // columns n .. n + 3 (n = 4q mod 8 inside their 32-k step): two
                // adjacent pairs in the permuted layout
                const int n = tiles[x] * 64 + 16 * j + 4 * q;
                uint16_t* row = g.out + int64_t(slot) * g.out_stride;
                *reinterpret_cast<uint32_t*>(row + permuted_k(n)) = uint32_t(hv[0]) | (uint32_t(hv[1]) << 16);
                *reinterpret_cast<uint32_t*>(row + permuted_k(n + 2)) = uint32_t(hv[2]) | (uint32_t(hv[3]) << 16);
              }
            }
          }
        }
      }
      return;
    }
    // the router weights before the first store (loads and stores share one
    // in-order counter: a load waited for after a store waits for it too)
    float wts[kNs];
#pragma unroll
    for (int sb = 0; sb < kNs; ++sb) {
      const int slot = s_slot[16 * sb + col];
      wts[sb] = kMode == kTopk && slot >= 0 ? round_act<kBF16>(g.topk_w[slot]) : 0.0f;
    }
#pragma unroll
    for (int x = 0; x < kDirectTiles; ++x) {
      if (!tile_ok[x]) continue;
#pragma unroll
      for (int sb = 0; sb < kNs; ++sb) {
        const int slot = s_slot[16 * sb + col];
        if (slot < 0) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int64_t n = int64_t(tiles[x]) * 64 + 16 * j + 4 * q;
          const f32x4_t v = acc[x][j][sb];
          if constexpr (kMode == kPartial) {
            *reinterpret_cast<f32x4_t*>(g.part + (int64_t(ks) * g.n_slots + slot) * g.N + n) = v;
          } else {
            float y[4] = {v[0], v[1], v[2], v[3]};
            if constexpr (kMode == kTopk) {
              const float w = wts[sb];
#pragma unroll
              for (int u = 0; u < 4; ++u) y[u] = round_act<kBF16>(y[u]) * w;  // exact product
            }
            const u32x2_t packed = {uint32_t(to_act<kBF16>(y[0])) | (uint32_t(to_act<kBF16>(y[1])) << 16),
                                    uint32_t(to_act<kBF16>(y[2])) | (uint32_t(to_act<kBF16>(y[3])) << 16)};
            *reinterpret_cast<u32x2_t*>(g.out + int64_t(slot) * g.out_stride + n) = packed;
          }
        }
      }
    }
  };
  if constexpr (kSub == 1) {
    run(std::integral_constant<int, 1>{});
  } else if constexpr (kSub == 2) {
    if (nsub == 1) run(std::integral_constant<int, 1>{});
    else run(std::integral_constant<int, 2>{});
  } else {
    if (nsub <= 2) run(std::integral_constant<int, 2>{});
    else run(std::integral_constant<int, 4>{});
  }
}

// out[r][permuted_k(k)] = a[r][k]: rows of `cols` elements (cols % 32 == 0).
__global__ __launch_bounds__(kThreads) void marlin_permute_kernel(const uint16_t* a, int64_t a_stride,
                                                                 int64_t rows, int cols, uint16_t* out,
                                                                 int64_t out_stride) {
  // one thread per (row, 32-k step, pair of halves)
  const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  const int64_t pairs = int64_t(cols) / 2;
  if (i >= rows * pairs) return;
  const int64_t r = i / pairs;
  const int k = int(i - r * pairs) * 2;
  const uint32_t v = *reinterpret_cast<const uint32_t*>(a + r * a_stride + k);
  *reinterpret_cast<uint32_t*>(out + r * out_stride + permuted_k(k)) = v;
}

// ---- dequant of one matrix (the GEMM's own operand path, for exact checks) ----

// W [K][N] in the activation dtype: one wavefront per (step, tile), the same
// fragment load, lane exchange and dequant as marlin_gemm, each operand
// element written at its (k, n).
template <bool kBF16>
__global__ __launch_bounds__(kThreads) void marlin_dequant_kernel(const u32x4_t* w, const uint16_t* s,
                                                                  int K, int N, uint16_t* out) {
  const int lane = threadIdx.x & 63;
  const int64_t item = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int tiles = N >> 6;
  if (item >= int64_t(K >> 5) * tiles) return;
  const int step = int(item / tiles);
  const int tile = int(item % tiles);
  Scales<kBF16> sc;
  sc.set(*reinterpret_cast<const u32x4_t*>(s + int64_t(step >> 2) * N + tile * 64 + 8 * (lane & 7)),
         lane);
  const u32x4_t v = *reinterpret_cast<const u32x4_t*>(
      reinterpret_cast<const uint8_t*>(w) + fragment_offset(N, tile, lane) + int64_t(step) * N * 16);
  const NibbleMasks masks{0x000f000fu, 0x00f000f0u, 0x64006400u};
  const int q = lane >> 4, r = lane & 15;
  const int kofs[8] = {2 * q, 2 * q + 1, 2 * q + 8, 2 * q + 9, 16 + 2 * q, 17 + 2 * q, 24 + 2 * q, 25 + 2 * q};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const u32x4_t a = sc.operand(combine(v[j], lane), j, masks);
    const int64_t n = int64_t(tile) * 64 + 16 * j + r;
#pragma unroll
    for (int h = 0; h < 8; ++h) {
      const uint32_t word = a[h >> 1];
      out[(int64_t(step) * 32 + kofs[h]) * N + n] = uint16_t((h & 1) ? word >> 16 : word & 0xffffu);
    }
  }
}

// ---- activation (decode_orig.cu:272-305) -----------------------------------------

// h[slot][n] = RN(RN(SiLU(min(G, L))) * clamp(U, -L, L)), G and U the
// activation-dtype roundings of the k-split FP32 sums in ks order; slots
// whose routed id is negative are skipped.
template <bool kBF16>
__global__ __launch_bounds__(kThreads) void marlin_act_kernel(const float* part, const int32_t* ids,
                                                              int ksplit, int n_slots, int nh,
                                                              float limit, uint16_t* h) {
  const int slot = blockIdx.y;
  const int n = int(blockIdx.x) * kThreads + threadIdx.x;
  if (n >= nh || ids[slot] < 0) return;
  const int64_t plane = int64_t(n_slots) * 2 * nh;
  const float* p = part + int64_t(slot) * 2 * nh + n;
  float gs = 0.0f, us = 0.0f;
  for (int k = 0; k < ksplit; ++k) {
    gs += p[k * plane];
    us += p[k * plane + nh];
  }
  h[int64_t(slot) * nh + n] = swiglu<kBF16>(gs, us, limit);
}

// ---- top-k sum (kernels/moe/routing.py:579-600) -------------------------------------

// out[t][c] = RN(sum over slots k = 0..topk-1 in order of in[t][k][c]) in FP32;
// with ids, a slot whose id is outside [0, experts) adds nothing.

// kVec columns per thread (8 with 16-byte loads when hidden % 8 == 0, else 1).
// With `shared` (the shared expert's output, element strides sh0 / sh1; sh1
// == 1 when kVec == 8): out[t][c] = RN(f32(RN(sum)) + f32(shared[t][c])), the
// routed sum rounded as moe_sum stores it, then one rounded add
// (vllm_sm80/kernels/moe/sum.py:18-56).
template <bool kBF16, int kVec>
__global__ __launch_bounds__(kThreads) void moe_sum_kernel(const uint16_t* in, int topk, int64_t hidden,
                                                           const int32_t* ids, int experts,
                                                           const uint16_t* shared, int64_t sh0,
                                                           int64_t sh1, uint16_t* out) {
  const int64_t t = blockIdx.y;
  const int64_t c = (int64_t(blockIdx.x) * kThreads + threadIdx.x) * kVec;
  if (c >= hidden) return;
  float acc[kVec];
#pragma unroll
  for (int u = 0; u < kVec; ++u) acc[u] = 0.0f;
  // eight slots at a time: their ids, then their rows' loads all in flight,
  // then the sums in slot order
  constexpr int kBatch = 8;
  for (int k0 = 0; k0 < topk; k0 += kBatch) {
    bool use[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int k = k0 + i;
      bool ok = k < topk;
      if (ok && ids) {
        const int id = ids[t * topk + k];
        ok = id >= 0 && id < experts;
      }
      use[i] = ok;
    }
    if constexpr (kVec == 8) {
      u32x4_t v[kBatch];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        v[i] = use[i] ? *reinterpret_cast<const u32x4_t*>(in + (t * topk + k0 + i) * hidden + c)
                      : u32x4_t{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        if (!use[i]) continue;
#pragma unroll
        for (int u = 0; u < 8; ++u) acc[u] += act_f32<kBF16>(uint16_t(v[i][u >> 1] >> (16 * (u & 1))));
      }
    } else {
      uint16_t v[kBatch];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) v[i] = use[i] ? in[(t * topk + k0 + i) * hidden + c] : uint16_t(0);
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        if (use[i]) acc[0] += act_f32<kBF16>(v[i]);
      }
    }
  }
  if (shared) {
    float sh[kVec];
    if constexpr (kVec == 8) {
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(shared + t * sh0 + c);
#pragma unroll
      for (int u = 0; u < 8; ++u) sh[u] = act_f32<kBF16>(uint16_t(v[u >> 1] >> (16 * (u & 1))));
    } else {
      sh[0] = act_f32<kBF16>(shared[t * sh0 + c * sh1]);
    }
#pragma unroll
    for (int u = 0; u < kVec; ++u) acc[u] = act_f32<kBF16>(to_act<kBF16>(acc[u])) + sh[u];
  }
  if constexpr (kVec == 8) {
    u32x4_t o;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      o[u] = uint32_t(to_act<kBF16>(acc[2 * u])) | (uint32_t(to_act<kBF16>(acc[2 * u + 1])) << 16);
    }
    *reinterpret_cast<u32x4_t*>(out + t * hidden + c) = o;
  } else {
    out[t * hidden + c] = to_act<kBF16>(acc[0]);
  }
}

// ---- deterministic alignment (tests/kernels/moe_align_reference.py) -------------------

constexpr int kAlignThreads = 1024;

__device__ __forceinline__ int routed_expert(const int32_t* ids, const int32_t* expert_map, int64_t i,
                                             int experts) {
  int e = ids[i];
  if (e < 0 || e >= experts) return -1;
  if (expert_map) {
    e = expert_map[e];
    if (e < 0 || e >= experts) return -1;
  }
  return e;
}

// Inclusive prefix sum over the 1024 threads of the workgroup: within each
// wavefront by shuffles, then across the 16 wavefront totals.
__device__ __forceinline__ int block_inclusive_scan(int v, int* wave_tot) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int o = __shfl_up(v, d);
    if (lane >= d) v += o;
  }
  if (lane == 63) wave_tot[wave] = v;
  __syncthreads();
  int before = 0;
  for (int w = 0; w < wave; ++w) before += wave_tot[w];
  __syncthreads();
  return v + before;
}

// Rounds of 1024 rows in ascending flat order: each wavefront ranks its rows
// per expert with ballots, and a row's rank within its expert counts the
// expert's rows of earlier rounds and earlier wavefronts (cursor[] starts at
// zero; wcnt[16][experts] when wave_counts, else the 16 wavefronts take turns
// at the cursors).  place(i, e, rank) for every routed row: the rank is its
// position in the stable (flat index) order of its expert's rows.
template <typename Place>
__device__ __forceinline__ void rank_rows(const int32_t* ids, int64_t numel, int experts,
                                          const int32_t* expert_map, int* count, int* wcnt,
                                          int wave_counts, Place&& place) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int id_bits = experts > 1 ? 32 - __builtin_clz(unsigned(experts - 1)) : 1;
  for (int64_t base = 0; base < numel; base += kAlignThreads) {
    const int64_t i = base + tid;
    const int e = i < numel ? routed_expert(ids, expert_map, i, experts) : -1;
    // lanes of this wavefront routed to the same expert: one ballot per bit
    // of the expert id (no data exchange between lanes)
    uint64_t same = __ballot(e >= 0);
    for (int bit = 0; bit < id_bits; ++bit) {
      const bool set = (e >> bit) & 1;
      const uint64_t m = __ballot(set);
      same &= set ? m : ~m;
    }
    const int rank = __builtin_popcountll(same & ((uint64_t(1) << lane) - 1));
    const int n_same = __builtin_popcountll(same);
    const bool leader = e >= 0 && rank == 0;
    int dest = -1;  // rank within the expert
    if (wave_counts) {
      if (leader) wcnt[wave * experts + e] = n_same;
      __syncthreads();
      if (e >= 0) {
        int before = count[e];
        for (int w = 0; w < wave; ++w) before += wcnt[w * experts + e];
        dest = before + rank;
      }
      __syncthreads();
      for (int x = tid; x < experts; x += kAlignThreads) {
        int add = 0;
        for (int w = 0; w < kAlignThreads / 64; ++w) {
          add += wcnt[w * experts + x];
          wcnt[w * experts + x] = 0;
        }
        count[x] += add;
      }
      __syncthreads();
    } else {
      for (int turn = 0; turn < kAlignThreads / 64; ++turn) {
        if (wave == turn && e >= 0) {
          const int cursor = count[e];
          dest = cursor + rank;
          if (leader) count[e] = cursor + n_same;
        }
        __syncthreads();
      }
    }
    if (dest >= 0) place(i, e, dest);
  }
}

// Rows a thread holds in registers on the one-pass alignment.
constexpr int kAlignChunks = 8;

// The alignment of up to kAlignChunks x 1024 rows and 1024 experts in one
// pass (align mode 2): every row's expert loaded at once (row c * 1024 +
// tid in register c), each wavefront's rows ranked per expert with ballots
// and counted per (round c, wavefront, expert) in LDS; one thread per
// expert turns its counts into exclusive prefixes in (round, wavefront)
// order, its total and padded size; one scan gives the padded starts.  A
// row then lands at start + prefix + rank: ascending flat order inside each
// expert, as the rounds below produce.  Five barriers, one round of loads.
__device__ __forceinline__ void align_block_onepass(
    const int32_t* ids, int64_t numel, int experts, int bs, const int32_t* expert_map,
    int32_t* sorted, int64_t sorted_size, int32_t* eids, int64_t blocks, int32_t* ntpp) {
  extern __shared__ int align_shared[];
  int* start = align_shared;       // experts: padded exclusive starts
  int* count = start + experts;    // experts: routed rows
  int* wcnt = count + experts;     // [rounds][16][experts]: counts, then prefixes
  __shared__ int wave_tot[kAlignThreads / 64];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int rounds = int((numel + kAlignThreads - 1) / kAlignThreads);
  int e[kAlignChunks];
#pragma unroll
  for (int c = 0; c < kAlignChunks; ++c) {
    const int64_t i = int64_t(c) * kAlignThreads + tid;
    e[c] = c < rounds && i < numel ? routed_expert(ids, expert_map, i, experts) : -1;
  }
  for (int x = tid; x < rounds * 16 * experts; x += kAlignThreads) wcnt[x] = 0;
  __syncthreads();
  const int id_bits = experts > 1 ? 32 - __builtin_clz(unsigned(experts - 1)) : 1;
  int rank[kAlignChunks];
#pragma unroll
  for (int c = 0; c < kAlignChunks; ++c) {
    rank[c] = 0;
    if (c < rounds) {
      // lanes of this wavefront routed to the same expert: one ballot per
      // bit of the expert id
      uint64_t same = __ballot(e[c] >= 0);
      for (int bit = 0; bit < id_bits; ++bit) {
        const bool set = (e[c] >> bit) & 1;
        const uint64_t m = __ballot(set);
        same &= set ? m : ~m;
      }
      rank[c] = __builtin_popcountll(same & ((uint64_t(1) << lane) - 1));
      if (e[c] >= 0 && rank[c] == 0) wcnt[(c * 16 + wave) * experts + e[c]] = __builtin_popcountll(same);
    }
  }
  __syncthreads();
  int run = 0;  // this thread's expert's padded size
  if (tid < experts) {
    // a round's 16 counts read together, then written back as prefixes (a
    // read after the previous entry's write would wait for it: one LDS round
    // trip per entry)
    int acc = 0;
    for (int c = 0; c < rounds; ++c) {
      int t[16];
#pragma unroll
      for (int w = 0; w < 16; ++w) t[w] = wcnt[(c * 16 + w) * experts + tid];
#pragma unroll
      for (int w = 0; w < 16; ++w) {
        wcnt[(c * 16 + w) * experts + tid] = acc;
        acc += t[w];
      }
    }
    count[tid] = acc;
    run = (acc + bs - 1) / bs * bs;
  }
  const int incl = block_inclusive_scan(run, wave_tot);
  if (tid < experts) start[tid] = incl - run;
  if (tid == kAlignThreads - 1) wave_tot[0] = incl;  // the padded total
  __syncthreads();
  const int total = wave_tot[0];
  if (tid == 0) ntpp[0] = total;
#pragma unroll
  for (int c = 0; c < kAlignChunks; ++c) {
    if (c < rounds && e[c] >= 0) {
      const int64_t dest = int64_t(start[e[c]]) + wcnt[(c * 16 + wave) * experts + e[c]] + rank[c];
      if (dest < sorted_size) sorted[dest] = c * kAlignThreads + tid;
    }
  }
  // the sentinel in each expert's padding and past the padded total
  if (tid < experts) {
    const int64_t p1 = min(int64_t(start[tid]) + (count[tid] + bs - 1) / bs * bs, sorted_size);
    for (int64_t p = int64_t(start[tid]) + count[tid]; p < p1; ++p) sorted[p] = int32_t(numel);
  }
  for (int64_t p = total + tid; p < sorted_size; p += kAlignThreads) sorted[p] = int32_t(numel);
  // each expert's blocks name it (an expert of no rows owns none); blocks
  // past the padded total name -1
  if (tid < experts) {
    const int b1 = min(int64_t(start[tid] + run) / bs, blocks);
    for (int b = start[tid] / bs; b < b1; ++b) eids[b] = tid;
  }
  for (int64_t b = total / bs + tid; b < blocks; b += kAlignThreads) eids[b] = -1;
}

// One workgroup: counts, padded exclusive scan, expert per block, then the
// routed rows placed in ascending flat order inside each expert: rounds of
// 1024 rows; each wavefront ranks its rows per expert with ballots, and a row
// lands after its expert's rows of earlier rounds and earlier wavefronts
// (per-wavefront counts in LDS when 16 x experts fit, else the 16 wavefronts
// take turns at the per-expert cursors).  Mode 2: align_block_onepass.
__device__ __forceinline__ void align_block(
    const int32_t* ids, int64_t numel, int experts, int bs, const int32_t* expert_map,
    int32_t* sorted, int64_t sorted_size, int32_t* eids, int64_t blocks, int32_t* ntpp,
    int wave_counts) {
  if (wave_counts == 2) {
    align_block_onepass(ids, numel, experts, bs, expert_map, sorted, sorted_size, eids, blocks, ntpp);
    return;
  }
  extern __shared__ int align_shared[];
  int* count = align_shared;          // experts: counts, then cursors
  int* start = count + experts;       // experts: padded exclusive starts
  int* wcnt = start + experts;        // [16][experts] when wave_counts
  __shared__ int wave_tot[kAlignThreads / 64];
  const int tid = threadIdx.x;
  for (int e = tid; e < experts; e += kAlignThreads) count[e] = 0;
  if (wave_counts) {
    for (int i = tid; i < 16 * experts; i += kAlignThreads) wcnt[i] = 0;
  }
  __syncthreads();
  for (int64_t i = tid; i < numel; i += kAlignThreads) {
    const int e = routed_expert(ids, expert_map, i, experts);
    if (e >= 0) atomicAdd(&count[e], 1);
  }
  __syncthreads();
  const int per = (experts + kAlignThreads - 1) / kAlignThreads;
  const int e0 = min(experts, tid * per);
  const int e1 = min(experts, e0 + per);
  int run = 0;
  for (int e = e0; e < e1; ++e) run += (count[e] + bs - 1) / bs * bs;
  const int incl = block_inclusive_scan(run, wave_tot);
  int at = incl - run;
  for (int e = e0; e < e1; ++e) {
    start[e] = at;
    at += (count[e] + bs - 1) / bs * bs;
    count[e] = 0;
  }
  if (tid == kAlignThreads - 1) wave_tot[0] = incl;  // the padded total
  __syncthreads();
  const int total = wave_tot[0];
  if (tid == 0) ntpp[0] = total;
  for (int64_t b = tid; b < blocks; b += kAlignThreads) {
    int owner = -1;
    if (b < total / bs) {
      // last expert whose first block is at or before b
      int lo = 0, hi = experts;
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (start[mid] / bs <= b) lo = mid; else hi = mid;
      }
      owner = lo;
    }
    eids[b] = owner;
  }
  for (int64_t i = tid; i < sorted_size; i += kAlignThreads) sorted[i] = int32_t(numel);
  __syncthreads();
  rank_rows(ids, numel, experts, expert_map, count, wcnt, wave_counts, [&](int64_t i, int e, int rank) {
    const int64_t dest = int64_t(start[e]) + rank;
    if (dest < sorted_size) sorted[dest] = int32_t(i);
  });
}

__global__ __launch_bounds__(kAlignThreads) void moe_align_kernel(
    const int32_t* ids, int64_t numel, int experts, int bs, const int32_t* expert_map,
    int32_t* sorted, int64_t sorted_size, int32_t* eids, int64_t blocks, int32_t* ntpp,
    int wave_counts) {
  align_block(ids, numel, experts, bs, expert_map, sorted, sorted_size, eids, blocks, ntpp, wave_counts);
}

// ---- router: logits, top-k, alignment (vllm_sm80/kernels/moe/route.py) ------------------

typedef short bf16raw8_t __attribute__((ext_vector_type(8)));

// logits[m][e] = sum_k x[m][k] W[e][k] in FP32 (bf16 or fp16 products are
// exact in FP32).  Workgroup = 16 kEB experts x 16 kRB rows: its four
// wavefronts take a quarter of K each on v_mfma_f32_16x16x32 (A = 16 rows x
// 32 k, B = 32 k x 16 experts, every lane 8 consecutive k of its row /
// expert), each 16 x 16 block of the tile its own accumulator, and the
// quarters are added in wavefront order.  Every logit is then the same
// sequence of operations whatever the tile and M, so the logits are
// bitwise reproducible and independent of M; larger tiles (large M) read
// the router matrix and the rows fewer times.  Rows past M and experts past
// E read a valid row and are not stored.
template <bool kBF16, int kRB, int kEB>
__global__ __launch_bounds__(256) void route_logits_kernel(const uint16_t* x, int64_t x_stride,
                                                           const uint16_t* w, int64_t M, int64_t K,
                                                           int64_t E, float* logits) {
  __shared__ f32x4_t red[3][kRB * kEB][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t e0 = int64_t(blockIdx.x) * 16 * kEB;
  const int64_t m0 = int64_t(blockIdx.y) * 16 * kRB;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int64_t kq = K / 4;
  const uint16_t* xa[kRB];
  const uint16_t* wb[kEB];
#pragma unroll
  for (int i = 0; i < kRB; ++i) xa[i] = x + min(m0 + 16 * i + r, M - 1) * x_stride + wave * kq + 8 * g;
#pragma unroll
  for (int j = 0; j < kEB; ++j) wb[j] = w + min(e0 + 16 * j + r, E - 1) * K + wave * kq + 8 * g;
  f32x4_t acc[kRB][kEB];
#pragma unroll
  for (int i = 0; i < kRB; ++i)
#pragma unroll
    for (int j = 0; j < kEB; ++j) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  // the next step's fragments are loaded before this step's products
  u32x4_t a[kRB], b[kEB];
#pragma unroll
  for (int i = 0; i < kRB; ++i) a[i] = *reinterpret_cast<const u32x4_t*>(xa[i]);
#pragma unroll
  for (int j = 0; j < kEB; ++j) b[j] = *reinterpret_cast<const u32x4_t*>(wb[j]);
  for (int64_t k = 0; k < kq; k += 32) {
    const int64_t kn = k + 32 < kq ? k + 32 : k;  // the last step reloads its own
    u32x4_t an[kRB], bn[kEB];
#pragma unroll
    for (int i = 0; i < kRB; ++i) an[i] = *reinterpret_cast<const u32x4_t*>(xa[i] + kn);
#pragma unroll
    for (int j = 0; j < kEB; ++j) bn[j] = *reinterpret_cast<const u32x4_t*>(wb[j] + kn);
#pragma unroll
    for (int i = 0; i < kRB; ++i)
#pragma unroll
      for (int j = 0; j < kEB; ++j) acc[i][j] = mfma<kBF16>(b[j], a[i], acc[i][j]);  // C[e][m]
#pragma unroll
    for (int i = 0; i < kRB; ++i) a[i] = an[i];
#pragma unroll
    for (int j = 0; j < kEB; ++j) b[j] = bn[j];
  }
  if (wave > 0) {
#pragma unroll
    for (int i = 0; i < kRB; ++i)
#pragma unroll
      for (int j = 0; j < kEB; ++j) red[wave - 1][i * kEB + j][lane] = acc[i][j];
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int i = 0; i < kRB; ++i) {
#pragma unroll
      for (int j = 0; j < kEB; ++j) {
        f32x4_t v = acc[i][j];
#pragma unroll
        for (int q = 0; q < 3; ++q) {
          const f32x4_t o = red[q][i * kEB + j][lane];
#pragma unroll
          for (int c = 0; c < 4; ++c) v[c] += o[c];
        }
        // lane holds experts 4 g .. 4 g + 3 of row r of block (i, j)
        const int64_t m = m0 + 16 * i + r;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int64_t e = e0 + 16 * j + 4 * g + c;
          if (m < M && e < E) logits[m * E + e] = v[c];
        }
      }
    }
  }
}

constexpr int64_t kLogitsTile32Rows = 256;
constexpr int64_t kLogitsTile64Rows = 1024;

// An FP32 key as a signed integer of the same order.
__device__ __forceinline__ int32_t monotone(float v) {
  const int32_t b = __builtin_bit_cast(int32_t, v);
  return b ^ ((b >> 31) & 0x7fffffff);
}

constexpr int kRouteMaxExperts = 1024;

// 64-bit maximum over the wavefront, in scalar registers: within each
// 16-lane row by DPP (quad swaps, then the half-row and row mirrors), then
// over the four rows' maxima.  Every lane must be active.
__device__ __forceinline__ int64_t wave_max_i64(int64_t v) {
  auto step = [&](auto ctrl) {
    constexpr int c = decltype(ctrl)::value;
    const uint64_t u = uint64_t(v);
    const uint32_t lo = uint32_t(__builtin_amdgcn_mov_dpp(int(uint32_t(u)), c, 0xF, 0xF, false));
    const uint32_t hi = uint32_t(__builtin_amdgcn_mov_dpp(int(uint32_t(u >> 32)), c, 0xF, 0xF, false));
    const int64_t o = int64_t((uint64_t(hi) << 32) | lo);
    v = o > v ? o : v;
  };
  step(std::integral_constant<int, 0xB1>{});   // quad_perm [1,0,3,2]
  step(std::integral_constant<int, 0x4E>{});   // quad_perm [2,3,0,1]
  step(std::integral_constant<int, 0x141>{});  // row_half_mirror
  step(std::integral_constant<int, 0x140>{});  // row_mirror
  int64_t best = INT64_MIN;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const uint64_t u = uint64_t(v);
    const uint32_t lo = uint32_t(__builtin_amdgcn_readlane(int(uint32_t(u)), 16 * r));
    const uint32_t hi = uint32_t(__builtin_amdgcn_readlane(int(uint32_t(u >> 32)), 16 * r));
    const int64_t o = int64_t((uint64_t(hi) << 32) | lo);
    best = o > best ? o : best;
  }
  return best;
}

// One wavefront a row (four rows a workgroup, the grid looping over more),
// kPer experts a lane (expert lane + 64 j): scores of every expert
// (sigmoid: 0.5 tanh(0.5 l) + 0.5, the key adding the bias; softmax:
// exp(l - max) / sum, the key the probability), top-k by the packed
// (monotone(key) << 32 | E - 1 - e) maximum (the lower expert wins an exact
// tie), weights = the selected scores, renormalized (/ (sum + 1e-20)) if
// asked, times `scale`; padding rows (is_padding != 0) route to -1.  The
// block alignment of the ids follows as a launch of its own.
template <int kPer>
__global__ __launch_bounds__(256) void route_select_kernel(const float* logits, const float* bias,
                                                           int64_t M, int E, int topk, int sigmoid,
                                                           int renorm, float scale,
                                                           const uint8_t* is_padding, float* topk_w,
                                                           int32_t* topk_ids) {
  const int lane = threadIdx.x & 63;
  const int64_t stride = int64_t(gridDim.x) * 4;
  for (int64_t m = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6); m < M; m += stride) {
    const float* lrow = logits + m * E;
    float score[kPer];
    int64_t packed[kPer];
    float mx = -INFINITY;
    if (!sigmoid) {
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        const int e = lane + 64 * j;
        if (e < E) mx = fmaxf(mx, lrow[e]);
      }
      mx = vq::wave_max(mx, lane);
    }
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int e = lane + 64 * j;
      score[j] = 0.0f;
      if (e < E) score[j] = sigmoid ? 0.5f * tanhf(0.5f * lrow[e]) + 0.5f : expf(lrow[e] - mx);
      sum += score[j];
    }
    if (!sigmoid) {
      // the softmax denominator: a fixed-order sum (per lane in expert
      // order, then the butterfly, whose partners add the same two values)
#pragma unroll
      for (int d = 32; d >= 1; d >>= 1) sum += __shfl_xor(sum, d);
#pragma unroll
      for (int j = 0; j < kPer; ++j) score[j] = score[j] / sum;
    }
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int e = lane + 64 * j;
      const float key = sigmoid ? score[j] + bias[e < E ? e : 0] : score[j];
      packed[j] = e < E ? (int64_t(monotone(key)) << 32) | int64_t(E - 1 - e) : INT64_MIN;
    }
    float sel_w = 0.0f;
    int sel_e = -1;
    float total = 0.0f;
    for (int k = 0; k < topk; ++k) {
      int64_t best = INT64_MIN;
#pragma unroll
      for (int j = 0; j < kPer; ++j) best = packed[j] > best ? packed[j] : best;
      best = wave_max_i64(best);  // uniform
      const int e = E - 1 - int(best & 0xffffffff);
      float v_own = 0.0f;
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        if (j == e / 64) v_own = score[j];
        if (packed[j] == best) packed[j] = INT64_MIN;
      }
      const float chosen = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v_own), e % 64));
      total += chosen;
      if (lane == k) {
        sel_w = chosen;
        sel_e = e;
      }
    }
    if (lane < topk) {
      float wgt = renorm ? sel_w / (total + 1e-20f) : sel_w;
      wgt *= scale;
      const bool pad = is_padding != nullptr && is_padding[m] != 0;
      topk_w[m * topk + lane] = wgt;
      topk_ids[m * topk + lane] = pad ? -1 : sel_e;
    }
  }
}

// ---- split-cover alignment (marlin_moe/split_align.py:173-224's layout) ----------------

// Block sizes of the split lists, largest first.
constexpr int kSplitSizes[4] = {64, 48, 32, 16};

struct SplitLists {
  int32_t* sorted[4];   // list k: sorted row ids (sentinel numel on padding)
  int32_t* eids[4];     // list k: expert of each block (-1 past the list)
  int64_t sorted_numel[4];
  int64_t eids_numel[4];
  int32_t* ntpp;        // [4]: rows (padded) of each list
};

// One workgroup.  An expert with r routed rows is covered by cover[r][k]
// blocks of size kSplitSizes[k] (the cheapest cover, a table built on the
// host); its rows, in stable flat order, fill list 0's blocks, then list 1's,
// and so on, so only its last block holds padding.  Lists are laid out
// expert after expert (exclusive scans over experts per list).
__global__ __launch_bounds__(kAlignThreads) void moe_split_align_kernel(
    const int32_t* ids, int64_t numel, int experts, const int32_t* expert_map, const int32_t* cover,
    SplitLists out, int wave_counts) {
  extern __shared__ int align_shared[];
  int* count = align_shared;            // experts: counts, then cursors
  int* off = count + experts;           // [4][experts]: list offsets (rows)
  int* lo = off + 4 * experts;          // [4][experts]: first rank of each list
  int* wcnt = lo + 4 * experts;         // [16][experts] when wave_counts
  __shared__ int wave_tot[kAlignThreads / 64];
  __shared__ int totals[4];
  const int tid = threadIdx.x;
  for (int e = tid; e < experts; e += kAlignThreads) count[e] = 0;
  if (wave_counts) {
    for (int i = tid; i < 16 * experts; i += kAlignThreads) wcnt[i] = 0;
  }
  __syncthreads();
  for (int64_t i = tid; i < numel; i += kAlignThreads) {
    const int e = routed_expert(ids, expert_map, i, experts);
    if (e >= 0) atomicAdd(&count[e], 1);
  }
  __syncthreads();
  const int per = (experts + kAlignThreads - 1) / kAlignThreads;
  const int e0 = min(experts, tid * per);
  const int e1 = min(experts, e0 + per);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    int run = 0;
    for (int e = e0; e < e1; ++e) run += cover[count[e] * 4 + k] * kSplitSizes[k];
    const int incl = block_inclusive_scan(run, wave_tot);
    int at = incl - run;
    for (int e = e0; e < e1; ++e) {
      off[k * experts + e] = at;
      at += cover[count[e] * 4 + k] * kSplitSizes[k];
    }
    if (tid == kAlignThreads - 1) totals[k] = incl;
    __syncthreads();
  }
  for (int e = e0; e < e1; ++e) {
    int at = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      lo[k * experts + e] = at;
      at += cover[count[e] * 4 + k] * kSplitSizes[k];
    }
    count[e] = 0;  // cursor
  }
  if (tid < 4) out.ntpp[tid] = totals[tid];
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int bs = kSplitSizes[k];
    const int total = totals[k];
    for (int64_t b = tid; b < out.eids_numel[k]; b += kAlignThreads) {
      int owner = -1;
      if (b < total / bs) {
        int lo_e = 0, hi_e = experts;  // last expert whose first block is at or before b
        while (hi_e - lo_e > 1) {
          const int mid = (lo_e + hi_e) >> 1;
          if (off[k * experts + mid] / bs <= b) lo_e = mid; else hi_e = mid;
        }
        owner = lo_e;
      }
      out.eids[k][b] = owner;
    }
    for (int64_t i = tid; i < total; i += kAlignThreads) out.sorted[k][i] = int32_t(numel);
  }
  __syncthreads();
  rank_rows(ids, numel, experts, expert_map, count, wcnt, wave_counts, [&](int64_t i, int e, int rank) {
    int k = 3;
    while (k > 0 && rank < lo[k * experts + e]) --k;
    out.sorted[k][off[k * experts + e] + rank - lo[k * experts + e]] = int32_t(i);
  });
}

// The alignment (workgroup 0) and the activations' k permutation (the other
// workgroups) in one launch: the two are independent, and the permutation
// hides under the single-workgroup alignment.  Permutation thread = (row,
// 32-k step, q): the 16 bytes at permuted positions 8q .. 8q + 7, i.e.
// k = 8s + 2q + t for s = 0..3, t = 0, 1 (four 4-byte loads, one store).
__global__ __launch_bounds__(kAlignThreads) void moe_align_permute_kernel(
    const int32_t* ids, int64_t numel, int experts, int bs, const int32_t* expert_map,
    int32_t* sorted, int64_t sorted_size, int32_t* eids, int64_t blocks, int32_t* ntpp,
    int wave_counts, const uint16_t* a, int64_t a_stride, int64_t rows, int cols, uint16_t* out,
    int64_t out_stride) {
  if (blockIdx.x == 0) {
    align_block(ids, numel, experts, bs, expert_map, sorted, sorted_size, eids, blocks, ntpp, wave_counts);
    return;
  }
  const int64_t i = int64_t(blockIdx.x - 1) * kAlignThreads + threadIdx.x;
  const int64_t per_row = int64_t(cols) / 8;
  if (i >= rows * per_row) return;
  const int64_t r = i / per_row;
  const int c = int(i - r * per_row);  // 8-half chunk of the row: step c / 4, q = c % 4
  const int base = (c >> 2) * 32 + 2 * (c & 3);
  const uint16_t* src = a + r * a_stride + base;
  u32x4_t v;
#pragma unroll
  for (int s4 = 0; s4 < 4; ++s4) v[s4] = *reinterpret_cast<const uint32_t*>(src + 8 * s4);
  *reinterpret_cast<u32x4_t*>(out + r * out_stride + 8 * int64_t(c)) = v;
}

// ---- host ----------------------------------------------------------------------------

template <bool kBF16, int kTilesWG, int kSub>
int launch_gemm(const GemmArgs& g, int mode, int blocks, int ksplit, hipStream_t s) {
  const dim3 grid(unsigned((g.N / 64 + kTilesWG - 1) / kTilesWG), unsigned(blocks), unsigned(ksplit));
  switch (mode) {
    case kPartial: hipLaunchKernelGGL((marlin_gemm<kBF16, kTilesWG, kSub, kPartial>), grid, dim3(kThreads), 0, s, g); break;
    case kStore: hipLaunchKernelGGL((marlin_gemm<kBF16, kTilesWG, kSub, kStore>), grid, dim3(kThreads), 0, s, g); break;
    case kPartialAct: hipLaunchKernelGGL((marlin_gemm<kBF16, kTilesWG, kSub, kPartialAct>), grid, dim3(kThreads), 0, s, g); break;
    case kTopkSum: hipLaunchKernelGGL((marlin_gemm<kBF16, kTilesWG, kSub, kTopkSum>), grid, dim3(kThreads), 0, s, g); break;
    default: hipLaunchKernelGGL((marlin_gemm<kBF16, kTilesWG, kSub, kTopk>), grid, dim3(kThreads), 0, s, g); break;
  }
  return vq::check_launch("marlin_gemm");
}

template <bool kBF16, int kSub>
int launch_direct(const GemmArgs& g, int mode, int blocks, int ksplit, hipStream_t s) {
  // 4 direct_tiles(mode, kSub) tiles per workgroup (kSwiglu: half of them
  // gate tiles, half the matching up tiles)
  const int per = 4 * direct_tiles(mode, kSub);
  const unsigned gx = unsigned((g.N / 64 + per - 1) / per);
  const dim3 grid(gx, unsigned(blocks), unsigned(ksplit));
  switch (mode) {
    case kPartial: hipLaunchKernelGGL((marlin_gemm_direct<kBF16, kSub, kPartial>), grid, dim3(kThreads), 0, s, g); break;
    case kStore: hipLaunchKernelGGL((marlin_gemm_direct<kBF16, kSub, kStore>), grid, dim3(kThreads), 0, s, g); break;
    case kTopk: hipLaunchKernelGGL((marlin_gemm_direct<kBF16, kSub, kTopk>), grid, dim3(kThreads), 0, s, g); break;
    default: hipLaunchKernelGGL((marlin_gemm_direct<kBF16, kSub, kSwiglu>), grid, dim3(kThreads), 0, s, g); break;
  }
  return vq::check_launch("marlin_gemm_direct");
}

template <bool kBF16>
int dispatch_direct(const GemmArgs& g, int mode, int blocks, int ksplit, hipStream_t s) {
  if (g.bs <= 16) return launch_direct<kBF16, 1>(g, mode, blocks, ksplit, s);
  if (g.bs <= 32) return launch_direct<kBF16, 2>(g, mode, blocks, ksplit, s);
  return launch_direct<kBF16, 4>(g, mode, blocks, ksplit, s);
}

// One 64-column tile per workgroup with its four wavefronts splitting K (few
// blocks: many workgroups), or four tiles per workgroup sharing the staged
// activations (enough blocks to fill the GPU: a quarter of the activation
// traffic).  16-token sub-blocks: up to 2 for blocks of <= 32 tokens, 4 above.
template <bool kBF16>
int dispatch_gemm(const GemmArgs& g, int mode, int blocks, int ksplit, int wide, hipStream_t s) {
  if (g.bs <= 16) {
    return wide ? launch_gemm<kBF16, 4, 1>(g, mode, blocks, ksplit, s)
                : launch_gemm<kBF16, 1, 1>(g, mode, blocks, ksplit, s);
  }
  if (g.bs <= 32) {
    return wide ? launch_gemm<kBF16, 4, 2>(g, mode, blocks, ksplit, s)
                : launch_gemm<kBF16, 1, 2>(g, mode, blocks, ksplit, s);
  }
  return launch_gemm<kBF16, 4, 4>(g, mode, blocks, ksplit, s);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Four tiles per workgroup once that still gives ~2 workgroups per CU (the
// routed blocks are at most min(blocks, n_slots / 2 + experts); the cheaper
// estimate of blocks routed by the slot count is used).
int wide_tiles(int64_t blocks, int64_t n_slots, int64_t block_size, int64_t experts, int64_t N,
               int64_t ksplit) {
  const int64_t routed_blocks = std::min<int64_t>(blocks, (n_slots + block_size - 1) / block_size + experts / 2);
  return routed_blocks * (N / 256) * ksplit >= 512 ? 1 : 0;
}

}  // namespace
}  // namespace marlin

namespace marlin {
namespace {

// Argument checks shared by the staged and the direct GEMM (the reference's
// checks where it has them), then the kernel arguments; `blocks` = the
// aligned blocks to launch (0: nothing to do).
int prepare_gemm(const void* a, int act_dtype, int64_t a_rows, int64_t a_stride, const int32_t* w,
                 const void* scales, int64_t experts, const int32_t* sorted, int64_t sorted_numel,
                 const int32_t* expert_ids, int64_t expert_ids_numel, const int32_t* ntpp,
                 const float* topk_w, int64_t top_k, int64_t n_slots, int64_t K, int64_t N,
                 int64_t block_size, int mode, int64_t ksplit, float limit, float* part,
                 int64_t part_numel, void* out, int64_t out_stride, int64_t out_rows, GemmArgs& g,
                 int64_t& blocks) {
  using namespace vq;
  if (act_dtype != kBF16 && act_dtype != kFP16) return fail("a: bf16 or fp16 activations");
  if (K <= 0 || N <= 0 || K % 128 != 0 || N % 64 != 0) return fail("K % 128, N % 64");
  if (K > INT_MAX / 2 || N > INT_MAX / 2) return fail("K and N must fit int32");
  if (block_size < 8 || block_size > kMaxBlock || block_size % 8 != 0) {
    return fail("moe block size must be a multiple of 8 up to 64");
  }
  if (top_k <= 0 || n_slots < 0 || n_slots > INT_MAX || experts <= 0 || experts > INT_MAX) {
    return fail("routing sizes out of range");
  }
  if (a_rows < 0 || a_stride < K || a_stride % 8 != 0) {
    return fail("a: unit inner stride, row stride a multiple of 8 and at least K");
  }
  if ((n_slots + top_k - 1) / top_k > a_rows) return fail("a has fewer rows than the routed slots need");
  if (a_rows * a_stride * 2 >= (int64_t(1) << 31) || K * N / 2 >= (int64_t(1) << 31)) {
    return fail("a and each expert's weights must stay below 2 GiB");
  }
  if (!aligned16(a) || !aligned16(w) || !aligned16(scales)) {
    return fail("a, w and s must be 16-byte aligned");
  }
  // every routed block holds at least one slot, and routed blocks come first;
  // without sorted ids (identity routing), block b is slot b and
  // expert_ids[b] its local expert
  if (!sorted) {
    if (expert_ids_numel < n_slots) return fail("identity routing: one expert id per slot");
    blocks = n_slots;
  } else {
    if (!ntpp) return fail("routing: num_tokens_post_pad required with sorted ids");
    blocks = std::min(std::min<int64_t>(sorted_numel / block_size, expert_ids_numel), n_slots);
  }
  if (blocks > 65535) return fail("too many aligned blocks");
  const int64_t groups = K / 128;
  if (ksplit <= 0 || groups % ksplit != 0 || ksplit > 65535) {
    return fail("ksplit must divide K / 128");
  }
  if (mode == kPartial || mode == kPartialAct) {
    if (!part || part_numel < ksplit * n_slots * N) return fail("w13 partial buffer");
    if (!aligned16(part)) return fail("w13 partial buffer must be 16-byte aligned");
    if (mode == kPartialAct) {
      if (N % 128 != 0) return fail("w13 SwiGLU: the gate and up halves must be whole 64-column tiles");
      if (ksplit * n_slots * N * 4 >= (int64_t(1) << 31)) return fail("w13 partials must stay below 2 GiB");
      if (!out || out_stride < N / 2 || out_rows < n_slots) return fail("h output too small");
      if (std::isnan(limit)) return fail("act: limit must not be NaN");
    }
  } else if (mode == kStore || mode == kTopk || mode == kTopkSum) {
    if (ksplit != 1) return fail("a stored output takes one k-slice");
    if (!out || out_stride < N || out_stride % 4 != 0 || out_rows < n_slots) return fail("output too small");
    if ((reinterpret_cast<uintptr_t>(out) & 7) != 0) return fail("output must be 8-byte aligned");
    if (mode != kStore && !topk_w) return fail("topk weights required");
    if (mode == kTopkSum) {
      if (sorted) return fail("w2 sum: identity routing only");
      if (n_slots * out_stride * 2 >= (int64_t(1) << 31)) return fail("w2 sum: slot rows must stay below 2 GiB");
    }
  } else if (mode == kSwiglu) {
    if (ksplit != 1) return fail("a stored output takes one k-slice");
    if (N % 256 != 0) return fail("SwiGLU: the gate and up halves must be whole 128-column pairs");
    if (!out || out_stride < N / 2 || out_stride % 32 != 0 || out_rows < n_slots) {
      return fail("h output too small (row stride a multiple of 32)");
    }
    if ((reinterpret_cast<uintptr_t>(out) & 7) != 0) return fail("output must be 8-byte aligned");
    if (std::isnan(limit)) return fail("act: limit must not be NaN");
  } else {
    return fail("unknown marlin_moe_gemm mode");
  }
  g = GemmArgs{};
  g.a = static_cast<const uint16_t*>(a);
  g.a_stride = a_stride;
  g.a_bytes = uint32_t(a_rows * a_stride * 2);
  g.w = reinterpret_cast<const u32x4_t*>(w);
  g.s = static_cast<const uint16_t*>(scales);
  g.sorted = sorted;
  g.eids = expert_ids;
  g.ntpp = ntpp;
  g.topk_w = topk_w;
  g.part = part;
  g.out = static_cast<uint16_t*>(out);
  g.out_stride = out_stride;
  g.top_k = int(top_k);
  g.n_slots = int(n_slots);
  g.K = int(K);
  g.N = int(N);
  g.bs = int(block_size);
  g.experts = int(experts);
  g.groups_per_split = int(groups / ksplit);
  g.limit = limit;
  if (n_slots == 0) blocks = 0;
  return kOk;
}

}  // namespace
}  // namespace marlin

extern "C" int marlin_moe_gemm(const void* a, int act_dtype, int64_t a_rows, int64_t a_stride,
                               const int32_t* w, const void* scales, int64_t experts,
                               const int32_t* sorted, int64_t sorted_numel, const int32_t* expert_ids,
                               int64_t expert_ids_numel, const int32_t* ntpp, const float* topk_w,
                               int64_t top_k, int64_t n_slots, int64_t K, int64_t N,
                               int64_t block_size, int mode, int64_t ksplit, float* part,
                               int64_t part_numel, void* out, int64_t out_stride, int64_t out_rows,
                               void* stream) {
  if (mode == marlin::kSwiglu || mode >= marlin::kPartialAct) return vq::fail("unknown marlin_moe_gemm mode");
  marlin::GemmArgs g;
  int64_t blocks = 0;
  if (int rc = marlin::prepare_gemm(a, act_dtype, a_rows, a_stride, w, scales, experts, sorted, sorted_numel,
                                    expert_ids, expert_ids_numel, ntpp, topk_w, top_k, n_slots, K, N,
                                    block_size, mode, ksplit, INFINITY, part, part_numel, out, out_stride,
                                    out_rows, g, blocks)) {
    return rc;
  }
  if (blocks == 0) return vq::kOk;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int wide = marlin::wide_tiles(blocks, n_slots, block_size, experts, N, ksplit);
  return act_dtype == vq::kBF16 ? marlin::dispatch_gemm<true>(g, mode, int(blocks), int(ksplit), wide, s)
                                : marlin::dispatch_gemm<false>(g, mode, int(blocks), int(ksplit), wide, s);
}

extern "C" int marlin_moe_w13_act(const void* a, int act_dtype, int64_t a_rows, int64_t a_stride,
                                  const int32_t* w, const void* scales, int64_t experts,
                                  const int32_t* sorted, int64_t sorted_numel, const int32_t* expert_ids,
                                  int64_t expert_ids_numel, const int32_t* ntpp, const int32_t* ids,
                                  int64_t top_k, int64_t n_slots, int64_t K, int64_t N, int64_t block_size,
                                  int64_t ksplit, float limit, float* part, int64_t part_numel, void* h,
                                  int64_t h_stride, int64_t h_rows, void* stream) {
  marlin::GemmArgs g;
  int64_t blocks = 0;
  if (!ids) return vq::fail("w13 SwiGLU: routed ids required");
  if (h_stride != N / 2) return vq::fail("w13 SwiGLU: h rows of N / 2 elements");
  if (int rc = marlin::prepare_gemm(a, act_dtype, a_rows, a_stride, w, scales, experts, sorted, sorted_numel,
                                    expert_ids, expert_ids_numel, ntpp, nullptr, top_k, n_slots, K, N,
                                    block_size, marlin::kPartialAct, ksplit, limit, part, part_numel, h,
                                    h_stride, h_rows, g, blocks)) {
    return rc;
  }
  if (blocks == 0) return vq::kOk;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int wide = marlin::wide_tiles(blocks, n_slots, block_size, experts, N, ksplit);
  // one arrival counter per (block, 64 gate columns)
  const exl3::CounterSlots slots = exl3::counter_slots(s, blocks * (N / 128));
  if (slots.pool) {
    g.counters = slots.pool + int64_t(slots.base) * marlin::kCounterStride;
    return act_dtype == vq::kBF16
        ? marlin::dispatch_gemm<true>(g, marlin::kPartialAct, int(blocks), int(ksplit), wide, s)
        : marlin::dispatch_gemm<false>(g, marlin::kPartialAct, int(blocks), int(ksplit), wide, s);
  }
  // no counter slots free: the partials, then the separate SwiGLU launch
  const int rc = act_dtype == vq::kBF16
      ? marlin::dispatch_gemm<true>(g, marlin::kPartial, int(blocks), int(ksplit), wide, s)
      : marlin::dispatch_gemm<false>(g, marlin::kPartial, int(blocks), int(ksplit), wide, s);
  if (rc) return rc;
  return marlin_moe_act(part, ids, ksplit, n_slots, N / 2, limit, h, act_dtype, stream);
}

namespace marlin {
namespace {
int launch_moe_sum(const void* in, int act_dtype, int64_t tokens, int64_t topk, int64_t hidden,
                   const int32_t* ids, int64_t experts, const void* shared, int64_t sh0, int64_t sh1,
                   void* out, void* stream, const char* what);
}  // namespace
}  // namespace marlin

extern "C" int marlin_moe_w2_sum(const void* a, int act_dtype, int64_t a_rows, int64_t a_stride,
                                 const int32_t* w, const void* scales, int64_t experts,
                                 const int32_t* expert_ids, int64_t expert_ids_numel, const float* topk_w,
                                 int64_t top_k, int64_t n_slots, int64_t K, int64_t N, int64_t block_size,
                                 void* out, int64_t out_stride, int64_t out_rows, void* sum_out,
                                 void* stream) {
  marlin::GemmArgs g;
  int64_t blocks = 0;
  if (!sum_out || (reinterpret_cast<uintptr_t>(sum_out) & 1) != 0) return vq::fail("w2 sum: 2-byte aligned sums");
  if (out_stride != N) return vq::fail("w2 sum: slot rows of N elements");
  if (top_k <= 0 || top_k > INT_MAX || n_slots % top_k != 0) return vq::fail("w2 sum: whole tokens of top_k slots");
  // a holds one row per slot (the GEMM's own top_k is 1)
  if (int rc = marlin::prepare_gemm(a, act_dtype, a_rows, a_stride, w, scales, experts, nullptr, 0, expert_ids,
                                    expert_ids_numel, nullptr, topk_w, 1, n_slots, K, N, block_size,
                                    marlin::kTopkSum, 1, INFINITY, nullptr, 0, out, out_stride, out_rows, g,
                                    blocks)) {
    return rc;
  }
  if (blocks == 0) return vq::kOk;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int wide = marlin::wide_tiles(blocks, n_slots, block_size, experts, N, 1);
  const int64_t tokens = n_slots / top_k;
  g.sum_out = static_cast<uint16_t*>(sum_out);
  g.sum_topk = int(top_k);
  // one arrival counter per (token, 64 columns)
  const exl3::CounterSlots slots =
      top_k <= 64 ? exl3::counter_slots(s, tokens * (N / 64)) : exl3::CounterSlots{nullptr, -1};
  if (slots.pool) {
    g.counters = slots.pool + int64_t(slots.base) * marlin::kCounterStride;
    return act_dtype == vq::kBF16 ? marlin::dispatch_gemm<true>(g, marlin::kTopkSum, int(blocks), 1, wide, s)
                                  : marlin::dispatch_gemm<false>(g, marlin::kTopkSum, int(blocks), 1, wide, s);
  }
  // no counter slots free: the slot rows, then the separate sum
  const int rc = act_dtype == vq::kBF16 ? marlin::dispatch_gemm<true>(g, marlin::kTopk, int(blocks), 1, wide, s)
                                        : marlin::dispatch_gemm<false>(g, marlin::kTopk, int(blocks), 1, wide, s);
  if (rc) return rc;
  return marlin::launch_moe_sum(out, act_dtype, tokens, top_k, N, expert_ids, experts, nullptr, 0, 0, sum_out,
                                stream, "marlin_moe_w2_sum");
}

extern "C" int marlin_moe_gemm_direct(const void* a_perm, int act_dtype, int64_t a_rows, int64_t a_stride,
                                      const int32_t* w, const void* scales, int64_t experts,
                                      const int32_t* sorted, int64_t sorted_numel,
                                      const int32_t* expert_ids, int64_t expert_ids_numel,
                                      const int32_t* ntpp, const float* topk_w, int64_t top_k,
                                      int64_t n_slots, int64_t K, int64_t N, int64_t block_size, int mode,
                                      int64_t ksplit, float limit, float* part, int64_t part_numel,
                                      void* out, int64_t out_stride, int64_t out_rows, void* stream) {
  if (mode >= marlin::kPartialAct) return vq::fail("unknown marlin_moe_gemm_direct mode");
  marlin::GemmArgs g;
  int64_t blocks = 0;
  if (int rc = marlin::prepare_gemm(a_perm, act_dtype, a_rows, a_stride, w, scales, experts, sorted,
                                    sorted_numel, expert_ids, expert_ids_numel, ntpp, topk_w, top_k, n_slots,
                                    K, N, block_size, mode, ksplit, limit, part, part_numel, out, out_stride,
                                    out_rows, g, blocks)) {
    return rc;
  }
  if (blocks == 0) return vq::kOk;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  return act_dtype == vq::kBF16 ? marlin::dispatch_direct<true>(g, mode, int(blocks), int(ksplit), s)
                                : marlin::dispatch_direct<false>(g, mode, int(blocks), int(ksplit), s);
}

extern "C" int marlin_permute_act(const void* a, int act_dtype, int64_t rows, int64_t cols, int64_t a_stride,
                                  void* out, int64_t out_stride, void* stream) {
  using namespace vq;
  if (act_dtype != kBF16 && act_dtype != kFP16) return fail("a: bf16 or fp16 activations");
  if (rows < 0 || cols <= 0 || cols % 32 != 0 || cols > INT_MAX) return fail("permute: cols % 32");
  if (a_stride < cols || out_stride < cols || a_stride % 2 != 0 || out_stride % 2 != 0) {
    return fail("permute: even row strides of at least cols");
  }
  if ((reinterpret_cast<uintptr_t>(a) & 3) != 0 || (reinterpret_cast<uintptr_t>(out) & 3) != 0) {
    return fail("permute: 4-byte aligned rows");
  }
  if (rows == 0) return kOk;
  const int64_t pairs = rows * (cols / 2);
  hipLaunchKernelGGL(marlin::marlin_permute_kernel, dim3(unsigned((pairs + marlin::kThreads - 1) / marlin::kThreads)),
                     dim3(marlin::kThreads), 0, static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(a),
                     a_stride, rows, int(cols), static_cast<uint16_t*>(out), out_stride);
  return check_launch("marlin_permute");
}

extern "C" int marlin_moe_act(const float* part, const int32_t* ids, int64_t ksplit, int64_t n_slots,
                              int64_t nh, float limit, void* h, int act_dtype, void* stream) {
  using namespace vq;
  if (act_dtype != kBF16 && act_dtype != kFP16) return fail("h: bf16 or fp16");
  if (ksplit <= 0 || nh <= 0 || n_slots < 0 || n_slots > 65535 || nh > INT_MAX / 2) {
    return fail("act: ksplit > 0, 0 < Nh, n_slots <= 65535");
  }
  if (std::isnan(limit)) return fail("act: limit must not be NaN");
  if (n_slots == 0) return kOk;
  const dim3 grid(unsigned((nh + marlin::kThreads - 1) / marlin::kThreads), unsigned(n_slots));
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (act_dtype == kBF16) {
    hipLaunchKernelGGL(marlin::marlin_act_kernel<true>, grid, dim3(marlin::kThreads), 0, s, part, ids,
                       int(ksplit), int(n_slots), int(nh), limit, static_cast<uint16_t*>(h));
  } else {
    hipLaunchKernelGGL(marlin::marlin_act_kernel<false>, grid, dim3(marlin::kThreads), 0, s, part, ids,
                       int(ksplit), int(n_slots), int(nh), limit, static_cast<uint16_t*>(h));
  }
  return check_launch("marlin_act");
}

extern "C" int marlin_dequant(const int32_t* w, const void* scales, int act_dtype, int64_t K, int64_t N,
                              void* out, void* stream) {
  using namespace vq;
  if (act_dtype != kBF16 && act_dtype != kFP16) return fail("bf16 or fp16 scales");
  if (K <= 0 || N <= 0 || K % 128 != 0 || N % 64 != 0) return fail("K % 128, N % 64");
  if (!marlin::aligned16(w) || !marlin::aligned16(scales)) return fail("w and s must be 16-byte aligned");
  const int64_t items = (K / 32) * (N / 64);
  if ((items + 3) / 4 > INT_MAX) return fail("matrix too large");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(unsigned((items + 3) / 4));
  const auto* wp = reinterpret_cast<const marlin::u32x4_t*>(w);
  const auto* sp = static_cast<const uint16_t*>(scales);
  if (act_dtype == kBF16) {
    hipLaunchKernelGGL(marlin::marlin_dequant_kernel<true>, grid, dim3(marlin::kThreads), 0, s, wp, sp,
                       int(K), int(N), static_cast<uint16_t*>(out));
  } else {
    hipLaunchKernelGGL(marlin::marlin_dequant_kernel<false>, grid, dim3(marlin::kThreads), 0, s, wp, sp,
                       int(K), int(N), static_cast<uint16_t*>(out));
  }
  return check_launch("marlin_dequant");
}

namespace marlin {
namespace {

int launch_moe_sum(const void* in, int act_dtype, int64_t tokens, int64_t topk, int64_t hidden,
                   const int32_t* ids, int64_t experts, const void* shared, int64_t sh0, int64_t sh1,
                   void* out, void* stream, const char* what) {
  using namespace vq;
  if (act_dtype != kBF16 && act_dtype != kFP16) return fail(std::string(what) + ": bf16 or fp16");
  if (tokens < 0 || tokens > 65535 || topk <= 0 || hidden <= 0 || experts < 0 || experts > INT_MAX ||
      topk > INT_MAX) {
    return fail(std::string(what) + ": sizes out of range");
  }
  if (tokens == 0) return kOk;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const auto* ip = static_cast<const uint16_t*>(in);
  const auto* sp = static_cast<const uint16_t*>(shared);
  auto* op = static_cast<uint16_t*>(out);
  const bool vec = hidden % 8 == 0 && aligned16(in) && aligned16(out) &&
                   (!shared || (sh1 == 1 && sh0 % 8 == 0 && aligned16(shared)));
  const int64_t per_block = int64_t(kThreads) * (vec ? 8 : 1);
  const dim3 grid(unsigned((hidden + per_block - 1) / per_block), unsigned(tokens));
#define VQ_SUM(B, V) hipLaunchKernelGGL((moe_sum_kernel<B, V>), grid, dim3(kThreads), 0, s, \
                                        ip, int(topk), hidden, ids, int(experts), sp, sh0, sh1, op)
  if (act_dtype == kBF16) {
    if (vec) VQ_SUM(true, 8); else VQ_SUM(true, 1);
  } else {
    if (vec) VQ_SUM(false, 8); else VQ_SUM(false, 1);
  }
#undef VQ_SUM
  return check_launch(what);
}

}  // namespace
}  // namespace marlin

extern "C" int moe_sum(const void* in, int act_dtype, int64_t tokens, int64_t topk, int64_t hidden,
                       const int32_t* ids, int64_t experts, void* out, void* stream) {
  return marlin::launch_moe_sum(in, act_dtype, tokens, topk, hidden, ids, experts, nullptr, 0, 0, out,
                                stream, "moe_sum");
}

extern "C" int moe_sum_add(const void* in, int act_dtype, int64_t tokens, int64_t topk, int64_t hidden,
                           const void* shared, int64_t shared_stride0, int64_t shared_stride1,
                           void* out, void* stream) {
  if (!shared) return vq::fail("moe_sum_add: shared is required");
  return marlin::launch_moe_sum(in, act_dtype, tokens, topk, hidden, nullptr, 0, shared, shared_stride0,
                                shared_stride1, out, stream, "moe_sum_add");
}

namespace marlin {
namespace {

// moe_align_block_size's argument checks; `lds` and `wave_counts` configure
// the alignment workgroup.
int align_checks(int64_t numel, int64_t num_experts, int64_t block_size, int64_t sorted_numel,
                 int64_t expert_ids_numel, int& wave_counts, size_t& lds) {
  using vq::fail;
  if (numel < 0 || numel > INT_MAX || block_size <= 0 || block_size > 1024) {
    return fail("align: numel and block size out of range");
  }
  if (num_experts <= 0 || num_experts > 8192) return fail("align: 1 <= num_experts <= 8192");
  const int64_t worst = numel + num_experts * (block_size - 1);
  if (worst > INT_MAX) return fail("align: padded total must fit int32");
  const int64_t need = numel < num_experts ? std::min(numel * block_size, worst) : worst;
  if (sorted_numel < need) return fail("align: sorted_token_ids is smaller than numel + E (bs - 1)");
  if (expert_ids_numel * block_size < need) return fail("align: expert_ids too small");
  // one pass (mode 2) over 1-8 rounds of rows when every row fits the
  // registers and the per-round counts fit 64 KB of LDS; else per-wavefront
  // counts when they fit, with the rest; else turns at the cursors
  const int64_t rounds = (numel + kAlignThreads - 1) / kAlignThreads;
  if (rounds >= 1 && rounds <= kAlignChunks && num_experts <= kAlignThreads &&
      (2 + 16 * rounds) * num_experts * int64_t(sizeof(int)) <= 65536) {
    wave_counts = 2;
    lds = size_t(2 + 16 * rounds) * size_t(num_experts) * sizeof(int);
    return vq::kOk;
  }
  wave_counts = num_experts <= 960 ? 1 : 0;
  lds = size_t(2 + (wave_counts ? 16 : 0)) * size_t(num_experts) * sizeof(int);
  return vq::kOk;
}

}  // namespace
}  // namespace marlin

extern "C" int moe_align_block_size(const int32_t* topk_ids, int64_t numel, int64_t num_experts,
                                    int64_t block_size, const int32_t* expert_map, int32_t* sorted,
                                    int64_t sorted_numel, int32_t* expert_ids, int64_t expert_ids_numel,
                                    int32_t* ntpp, void* stream) {
  using namespace vq;
  int wave_counts = 0;
  size_t lds = 0;
  if (int rc = marlin::align_checks(numel, num_experts, block_size, sorted_numel, expert_ids_numel,
                                    wave_counts, lds)) {
    return rc;
  }
  const hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(marlin::moe_align_kernel, dim3(1), dim3(marlin::kAlignThreads), lds, s, topk_ids,
                     numel, int(num_experts), int(block_size), expert_map, sorted, sorted_numel,
                     expert_ids, expert_ids_numel, ntpp, wave_counts);
  return check_launch("moe_align_block_size");
}

extern "C" int moe_split_align(const int32_t* topk_ids, int64_t numel, int64_t num_experts,
                               const int32_t* expert_map, const int32_t* cover, int64_t cover_rows,
                               int32_t* sorted64, int32_t* sorted48, int32_t* sorted32, int32_t* sorted16,
                               const int64_t* sorted_numel, int32_t* eids64, int32_t* eids48,
                               int32_t* eids32, int32_t* eids16, const int64_t* eids_numel,
                               int32_t* ntpp, void* stream) {
  using namespace vq;
  if (numel < 0 || numel > INT_MAX) return fail("split_align: numel out of range");
  if (num_experts <= 0 || num_experts > 8192) return fail("split_align: 1 <= num_experts <= 8192");
  if (cover_rows < numel) return fail("split_align buffers too small");
  if (9 * num_experts * int64_t(sizeof(int)) > 65536) return fail("split_align: at most 1820 experts");
  marlin::SplitLists lists{};
  int32_t* sorted[4] = {sorted64, sorted48, sorted32, sorted16};
  int32_t* eids[4] = {eids64, eids48, eids32, eids16};
  for (int k = 0; k < 4; ++k) {
    const int64_t bs = marlin::kSplitSizes[k];
    // the reference's buffers: numel + bs E rows, (numel + bs E) / bs + 1 blocks
    if (sorted_numel[k] < numel + bs * num_experts || eids_numel[k] < (numel + bs * num_experts) / bs) {
      return fail("split_align buffers too small");
    }
    if (numel + bs * num_experts > INT_MAX) return fail("split_align: padded total must fit int32");
    lists.sorted[k] = sorted[k];
    lists.eids[k] = eids[k];
    lists.sorted_numel[k] = sorted_numel[k];
    lists.eids_numel[k] = eids_numel[k];
  }
  lists.ntpp = ntpp;
  const int wave_counts = num_experts <= 640 ? 1 : 0;
  const size_t lds = size_t(9 + (wave_counts ? 16 : 0)) * size_t(num_experts) * sizeof(int);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(marlin::moe_split_align_kernel, dim3(1), dim3(marlin::kAlignThreads), lds, s, topk_ids,
                     numel, int(num_experts), expert_map, cover, lists, wave_counts);
  return check_launch("moe_split_align");
}

extern "C" int moe_route(const void* x, int x_dtype, int64_t M, int64_t K, int64_t x_stride,
                         const void* weight, const float* bias, int64_t num_experts, int64_t topk,
                         int scoring, int renormalize, float scale, int64_t block_size,
                         const uint8_t* is_padding, float* logits, float* topk_weights,
                         int32_t* topk_ids, int32_t* sorted, int64_t sorted_numel,
                         int32_t* expert_ids, int64_t expert_ids_numel, int32_t* ntpp,
                         void* stream) {
  using namespace vq;
  if (x_dtype != kBF16 && x_dtype != kFP16) return fail("moe_route: bf16 or fp16 x and weight");
  if (M <= 0 || M > (int64_t(1) << 24)) return fail("moe_route: 1 <= M <= 2^24 rows");
  if (K <= 0 || K % 128 != 0 || K > (int64_t(1) << 24)) return fail("moe_route: K % 128 == 0");
  if (x_stride < K || x_stride % 8 != 0) return fail("moe_route: x rows 16-byte aligned, stride >= K");
  if ((reinterpret_cast<uintptr_t>(x) & 15) != 0 || (reinterpret_cast<uintptr_t>(weight) & 15) != 0) {
    return fail("moe_route: 16-byte aligned x and weight");
  }
  if (num_experts <= 0 || num_experts > marlin::kRouteMaxExperts) return fail("moe_route: 1 <= E <= 1024");
  if (topk <= 0 || topk > num_experts || topk > 64) return fail("moe_route: 1 <= topk <= min(E, 64)");
  if (scoring != 0 && scoring != 1) return fail("moe_route: scoring 0 (softmax) or 1 (sigmoid + bias)");
  if (scoring == 1 && bias == nullptr) return fail("moe_route: sigmoid scoring needs the bias");
  int wave_counts = 0;
  size_t lds = 0;
  if (int rc = marlin::align_checks(M * topk, num_experts, block_size, sorted_numel, expert_ids_numel,
                                    wave_counts, lds)) {
    return rc;
  }
  const hipStream_t s = static_cast<hipStream_t>(stream);
  // tiles of 16 x 16 (the most workgroups) for few rows, 32 x 32 and then
  // 64 x 64 (the router matrix read once per 32 / 64 rows) for more
  const int tile = M > marlin::kLogitsTile64Rows ? 4 : (M > marlin::kLogitsTile32Rows ? 2 : 1);
  const dim3 grid(unsigned((num_experts + 16 * tile - 1) / (16 * tile)), unsigned((M + 16 * tile - 1) / (16 * tile)));
#define VQ_LOGITS(B, T)                                                                            \
  hipLaunchKernelGGL((marlin::route_logits_kernel<B, T, T>), grid, dim3(256), 0, s,                 \
                     static_cast<const uint16_t*>(x), x_stride, static_cast<const uint16_t*>(weight), \
                     M, K, num_experts, logits)
  if (x_dtype == kBF16) {
    if (tile == 4) VQ_LOGITS(true, 4); else if (tile == 2) VQ_LOGITS(true, 2); else VQ_LOGITS(true, 1);
  } else {
    if (tile == 4) VQ_LOGITS(false, 4); else if (tile == 2) VQ_LOGITS(false, 2); else VQ_LOGITS(false, 1);
  }
#undef VQ_LOGITS
  if (int rc = check_launch("moe_route logits")) return rc;
  // four rows a workgroup, at most 64 Ki workgroups (rows beyond loop);
  // kPer = experts a lane
  const unsigned select_groups = unsigned(std::min<int64_t>((M + 3) / 4, 65536));
  const int per = int((num_experts + 63) / 64);
#define VQ_SELECT(P)                                                                                \
  hipLaunchKernelGGL(marlin::route_select_kernel<P>, dim3(select_groups), dim3(256), 0, s, logits, bias, \
                     M, int(num_experts), int(topk), scoring, renormalize, scale, is_padding,          \
                     topk_weights, topk_ids)
  if (per <= 1) VQ_SELECT(1); else if (per <= 2) VQ_SELECT(2); else if (per <= 4) VQ_SELECT(4);
  else if (per <= 5) VQ_SELECT(5); else if (per <= 8) VQ_SELECT(8); else VQ_SELECT(16);
#undef VQ_SELECT
  if (int rc = check_launch("moe_route select")) return rc;
  hipLaunchKernelGGL(marlin::moe_align_kernel, dim3(1), dim3(marlin::kAlignThreads), lds, s, topk_ids,
                     M * topk, int(num_experts), int(block_size), nullptr, sorted, sorted_numel, expert_ids,
                     expert_ids_numel, ntpp, wave_counts);
  return check_launch("moe_route align");
}

extern "C" int marlin_moe_align_permute(const int32_t* topk_ids, int64_t numel, int64_t num_experts,
                                        int64_t block_size, const int32_t* expert_map, int32_t* sorted,
                                        int64_t sorted_numel, int32_t* expert_ids,
                                        int64_t expert_ids_numel, int32_t* ntpp, const void* a,
                                        int act_dtype, int64_t rows, int64_t cols, int64_t a_stride,
                                        void* out, int64_t out_stride, void* stream) {
  using namespace vq;
  int wave_counts = 0;
  size_t lds = 0;
  if (int rc = marlin::align_checks(numel, num_experts, block_size, sorted_numel, expert_ids_numel,
                                    wave_counts, lds)) {
    return rc;
  }
  if (act_dtype != kBF16 && act_dtype != kFP16) return fail("a: bf16 or fp16 activations");
  if (rows < 0 || cols <= 0 || cols % 32 != 0 || cols > INT_MAX) return fail("permute: cols % 32");
  if (a_stride < cols || out_stride < cols || a_stride % 2 != 0 || out_stride % 8 != 0) {
    return fail("permute: row strides of at least cols (even; output a multiple of 8)");
  }
  if ((reinterpret_cast<uintptr_t>(a) & 3) != 0 || (reinterpret_cast<uintptr_t>(out) & 15) != 0) {
    return fail("permute: 4-byte aligned input and 16-byte aligned output rows");
  }
  const int64_t chunks = rows * (cols / 8);
  const int64_t permute_groups = (chunks + marlin::kAlignThreads - 1) / marlin::kAlignThreads;
  if (permute_groups + 1 > INT_MAX) return fail("permute: too many rows");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(marlin::moe_align_permute_kernel, dim3(unsigned(1 + permute_groups)),
                     dim3(marlin::kAlignThreads), lds, s, topk_ids, numel, int(num_experts),
                     int(block_size), expert_map, sorted, sorted_numel, expert_ids, expert_ids_numel, ntpp,
                     wave_counts, static_cast<const uint16_t*>(a), a_stride, rows, int(cols),
                     static_cast<uint16_t*>(out), out_stride);
  return check_launch("marlin_moe_align_permute");
}
