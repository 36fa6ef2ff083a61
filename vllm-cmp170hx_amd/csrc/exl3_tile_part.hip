// One part of the tile GEMM's instantiations (exl3_tile.h): the formats i
// of VQ_EXL3_FORMATS with i % kTileParts == VQ_TILE_PART, dense at both
// activation precisions and, for mul1 rates, MoE.  build.py compiles this
// file once per part, in parallel.
#include "exl3_tile.h"

#ifndef VQ_TILE_PART
#error "build with -DVQ_TILE_PART=<part>"
#endif

namespace exl3 {
namespace {

template <int kBitsX2, int kCodebook, bool kMoe>
int launch(bool lo, const TileArgs& a, dim3 grid, hipStream_t stream) {
  if (lo) {
    hipLaunchKernelGGL((tile_gemm<kBitsX2, kCodebook, kMoe, true>), grid, dim3(kTileThreads), 0, stream, a);
  } else {
    hipLaunchKernelGGL((tile_gemm<kBitsX2, kCodebook, kMoe, false>), grid, dim3(kTileThreads), 0, stream, a);
  }
  return vq::check_launch(kMoe ? "exl3 moe tile_gemm" : "exl3 tile_gemm");
}

}  // namespace

template <>
int tile_launch_part<VQ_TILE_PART>(int64_t bits_x2, int64_t codebook, bool moe, bool lo, const TileArgs& a,
                                   dim3 grid, hipStream_t stream) {
#define VQ_CASE(B, C)                                                      \
  if constexpr (format_index(B, C) % kTileParts == VQ_TILE_PART) {         \
    if (bits_x2 == B && codebook == C) {                                   \
      if (!moe) return launch<B, C, false>(lo, a, grid, stream);           \
      if constexpr (C == 2) return launch<B, C, true>(lo, a, grid, stream); \
      return vq::fail("EXL3 MoE: no tile GEMM for this codebook");        \
    }                                                                      \
  }
  VQ_EXL3_FORMATS(VQ_CASE)
#undef VQ_CASE
  return vq::fail("Unsupported EXL3 rate/codebook combination");
}

}  // namespace exl3
