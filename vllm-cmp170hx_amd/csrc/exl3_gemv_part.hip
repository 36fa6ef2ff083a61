// One part of the small-M GEMV instantiations (exl3_gemv.h): the formats i
// of VQ_EXL3_FORMATS with i % kGemvParts == VQ_GEMV_PART.  build.py compiles
// this file once per part, in parallel.
#include "exl3_gemv.h"

#ifndef VQ_GEMV_PART
#error "build with -DVQ_GEMV_PART=<part>"
#endif

namespace exl3 {

template <>
int gemv_launch_part<VQ_GEMV_PART>(int64_t bits_x2, int64_t codebook, bool aligned, int load,
                                   const GemvArgs* gemv, int gemv_blocks, int gemv_groups, dim3 grid,
                                   hipStream_t stream, const uint8_t* trellis, int64_t tiles_k,
                                   int64_t tiles_n, uint16_t* decoded) {
#define VQ_CASE(B, C)                                                                              \
  if constexpr (format_index(B, C) % kGemvParts == VQ_GEMV_PART) {                                 \
    if (bits_x2 == B && codebook == C) {                                                           \
      return launch_format<B, C>(aligned, load, gemv, gemv_blocks, gemv_groups, grid, stream, trellis, \
                                 tiles_k, tiles_n, decoded);                                       \
    }                                                                                              \
  }
  VQ_EXL3_FORMATS(VQ_CASE)
#undef VQ_CASE
  return vq::fail("Unsupported EXL3 rate/codebook combination");
}

}  // namespace exl3
