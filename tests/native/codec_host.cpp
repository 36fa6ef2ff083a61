// Host build of the device trellis decode (vllm-cmp170hx_amd/csrc/
// exl3_codec.h), for the CPU tests: the same per-lane word selection,
// window realignment, state extraction, hash and codebook code the gfx950
// kernels run, executed on the host for every (tile, encoder lane) and
// scattered with the format's lane map.  Test infrastructure only.
#include "../../vllm-cmp170hx_amd/csrc/exl3_codec.h"

namespace {

template <int B, int C>
void decode_all(const uint16_t* trellis, int64_t tiles_k, int64_t tiles_n, uint16_t* out) {
  using namespace exl3;
  const int64_t cols = 16 * tiles_n;
  for (int64_t tile = 0; tile < tiles_k * tiles_n; ++tile) {
    const uint16_t* t = trellis + tile * 8 * B;
    const int64_t tr = tile / tiles_n, tc = tile % tiles_n;
    for (int L = 0; L < 32; ++L) {
      int idx[LaneLoad<B>::kWords];
      lane_word_index<B>(L, idx);
      uint32_t words[LaneLoad<B>::kWords];
      for (int i = 0; i < LaneLoad<B>::kWords; ++i)
        words[i] = uint32_t(t[2 * idx[i]]) | (uint32_t(t[2 * idx[i] + 1]) << 16);
      uint32_t pair[4];
      decode_words<B, C>(L, words, pair);
      for (int j = 0; j < 8; ++j) {
        const int64_t row = tr * 16 + 2 * (L & 3) + (j & 1) + 8 * ((j >> 1) & 1);
        const int64_t col = tc * 16 + (L >> 2) + 8 * (j >> 2);
        out[row * cols + col] = uint16_t(pair[j >> 1] >> (16 * (j & 1)));
      }
    }
  }
}

}  // namespace

extern "C" int codec_host_decode(const uint16_t* trellis, int64_t tiles_k, int64_t tiles_n,
                                 int bits_x2, int codebook, uint16_t* out) {
#define CASE(B, C) if (bits_x2 == B && codebook == C) { decode_all<B, C>(trellis, tiles_k, tiles_n, out); return 0; }
  CASE(2, 1) CASE(4, 1) CASE(6, 1) CASE(8, 1) CASE(10, 1) CASE(12, 1) CASE(14, 1) CASE(16, 1)
  CASE(2, 2) CASE(3, 2) CASE(4, 2) CASE(5, 2) CASE(6, 2) CASE(7, 2) CASE(8, 2) CASE(10, 2)
  CASE(12, 2) CASE(14, 2) CASE(16, 2)
#undef CASE
  return 1;
}
