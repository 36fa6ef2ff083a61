// EXL3 many-row GEMM for gfx950: decode in registers, activations through LDS.
//
// C[r][n] = sum_k A[r][k] W[k][n] for a tile of up to 128 rows x 256 output
// columns, on v_mfma_f32_16x16x32_f16, then the output transform (unscale
// the row, H128 over each 128-column block, times svh).  Serves the dense
// linear above 32 rows (exl3_gemm.hip) and the MoE projections of
// prefill-sized calls (exl3_moe.hip: the tile's rows are one expert's routed
// assignments).
//
// Workgroup: 4 wavefronts (one per SIMD), two workgroups per CU.  Wavefront
// w owns output columns [64 w, 64 w + 64) of the tile: four tile columns, two
// pairs.  Per 32-input step (two tile rows) each lane decodes four encoder
// lanes (two pairs x two tile rows) straight into MFMA B operands, with the
// small-M kernel's lane map: lane (g, m) = (lane >> 4, lane & 15) decodes
// encoder lane L = 4 (m & 7) + g of tile column (m >> 3) of a pair; values
// 0-3 are B column m of the pair's first MFMA (tile column m & 7), values 4-7
// of its second (tile column (m & 7) + 8), k slots {2g, 2g+1, 2g+8, 2g+9} of
// the two tile rows.  The activations are stored in that k order (every
// 32-input step: [g 0..3][8 halves]), so no weight ever moves between lanes
// or through LDS.  The A operand of a 16-row block is then, for lane (g, m),
// the 16 bytes of group g of row m: stored in LDS as [g][m] (1 KB per block),
// read with one ds_read_b128 at 16 * lane, conflict-free.
//
// Activations: each rotated input at a per-row power-of-two scale, split
// into FP16 high and low parts (t 2^e = hi + lo, ~22 bits) with both parts
// multiplied against the exact FP16 weight into one FP32 accumulator (kLo,
// the default: the activation precision of the reference's tensor-core
// kernels, csrc/exl3/dense_prefill_tc.h:5-12), or the high part alone
// (!kLo: each rotated input rounded once to FP16, half the MFMAs; an
// explicit opt-in).
//
// Pipeline, per wavefront (one barrier a step):
//   * trellis: LDS-DMA (buffer_load ... lds), 128 bits_x2 bytes per step
//     (one 1 KB load up to 4 bits per weight, two above), into a ring of 4
//     slots, issued 4 steps ahead; a step's ring words are read and decoded
//     (into registers) one step before its MFMAs;
//   * activations: LDS-DMA of the tile's 8 row blocks per step (and their
//     low parts), 2 (4) per wavefront, into 3 buffers, issued 2 steps ahead;
//     the operands of row block rb + 2 are read under the MFMAs of rb;
//   * step s: issue the activation loads of s + 2, read the words of s + 1,
//     issue the trellis load of s + 4, run the MFMAs of s with the decode of
//     s + 1 between them (the VALU work of one step under the matrix work of
//     the other), wait for this wavefront's loads of s + 1, barrier.
//   Loads past the last step reload the last step (into a buffer or slot no
//   one reads again), so the loop has no branch around a load and every wait
//   count is a constant.
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>

#include "common.h"
#include "exl3_codec.h"
#include "exl3_internal.h"

namespace exl3 {

constexpr int kTileWaves = 4;
constexpr int kTileThreads = 64 * kTileWaves;
constexpr int kTileCols = 64 * kTileWaves;          // 256
constexpr int kTileRows = 128;
constexpr int kTileBlocks = kTileRows / 16;         // 16-row blocks
constexpr int kTileABufs = 3;
constexpr int kTileRing = 4;
constexpr int kTileADma = kTileBlocks / kTileWaves;  // 1 KB activation loads per wave and step
constexpr int kTileRedStride = kTileCols + 4;       // epilogue row stride (floats)

// The tile GEMM serves every rate: the trellis of one step of a wavefront
// (four tile columns x two tile rows, 128 bits_x2 bytes) is one 1 KB load
// up to 4 bits per weight, two above.
constexpr bool tile_rate(int64_t bits_x2) { return bits_x2 >= 2 && bits_x2 <= 16; }
constexpr int tile_slot_bytes(int bits_x2) { return bits_x2 <= 8 ? 1024 : 2048; }

struct TileArgs {
  // activation rows: row r at act + r * act_row_bytes, [high: kp halves]
  // [low: kp halves], each 32-input step in the k order above
  const uint8_t* act;
  int64_t act_row_bytes;   // 4 * kp
  int64_t act_rows;        // rows the activation buffer holds
  const int* row_exp;      // scale exponent of row r at row_exp[r * exp_stride]
  int64_t exp_stride;
  int64_t kp;
  int64_t np;
  // dense: the matrix, rows, and the output
  const uint8_t* trellis;
  const uint16_t* svh;
  int64_t tiles_n;
  int64_t rows;
  void* out;
  int out_dtype;
  int64_t logical_out;
  // MoE: the route table (header, sorted assignments, tasks) and the
  // projection of the experts' tables; FP32 outputs [assignment][np]
  const int* table;
  int64_t task_offset;     // int4 tasks at table + task_offset
  const int64_t* ptrs;
  const int64_t* meta;
  int projection;
  float* moe_out;
  const int* moe_row_exp;  // MoE: exponent of assignment a at moe_row_exp[a * exp_stride]
  int col_tiles;           // column tiles per task
  int task_group;          // tasks per group in an XCD's order (1..8)
};

typedef __attribute__((address_space(3))) void* tile_lds_ptr_t;

// f(std::integral_constant<int, i>) for i = 0 .. n - 1.
template <int n, int i = 0, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (i < n) {
    f(std::integral_constant<int, i>{});
    static_for<n, i + 1>(f);
  }
}

// LDS reads the compiler does not see (a read it sees, of LDS that LDS-DMA
// loads write, makes it wait for every such load in flight); a value is
// ready after a tile_wait* that names it.
template <int kOffset>
__device__ __forceinline__ void tile_read16(half8_t& v, uint32_t address) {
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(address), "i"(kOffset));
}
template <int kOffset>
__device__ __forceinline__ void tile_read4(uint32_t& v, uint32_t address) {
  asm volatile("ds_read_b32 %0, %1 offset:%2" : "=v"(v) : "v"(address), "i"(kOffset));
}
// At most n LDS reads still pending (they complete in order).
template <int n>
__device__ __forceinline__ void tile_lgkm() {
  asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(n));
}
// v is ready (after a tile_lgkm that covers its read).
__device__ __forceinline__ void tile_ready(half8_t& v) { asm volatile("" : "+v"(v)); }
template <int kWords>
__device__ __forceinline__ void tile_ready(uint32_t (&w)[2][2][kWords]) {
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < kWords; ++i) asm volatile("" : "+v"(w[p][h][i]));
}

template <int kBitsX2, int kCodebook, bool kMoe, bool kLo>
__global__ __launch_bounds__(kTileThreads, 2) void tile_gemm(TileArgs a) {
  constexpr int kRows = kTileRows;
  constexpr int kBlocks = kRows / 16;
  constexpr int kADma = kBlocks / kTileWaves;
  constexpr int kParts = kLo ? 2 : 1;      // activation parts: high (and low)
  constexpr int kAL = kParts * kADma;      // activation loads per wavefront and step
  static_assert(tile_rate(kBitsX2), "a rate the tile GEMM serves");
  constexpr int kWords = LaneLoad<kBitsX2>::kWords;
  constexpr int kTileBytes = 16 * kBitsX2;
  constexpr int kRowChunk = 4 * kTileBytes;  // one tile row of a wavefront's four tile columns
  constexpr int kSlot = tile_slot_bytes(kBitsX2);
  constexpr int kTL = kSlot / 1024;          // trellis loads per wavefront and step
  constexpr int kChunkLanes = kRowChunk / 16;
  static_assert(kRowChunk % 16 == 0 && 2 * kRowChunk <= kSlot, "a step's trellis fits its slot");
  // 80 KB at most (two workgroups per CU in 160 KB)
  __shared__ __attribute__((aligned(16))) uint8_t a_lds[kTileABufs][kParts * kBlocks][1024];
  __shared__ __attribute__((aligned(16))) uint8_t t_lds[kTileWaves][kTileRing][kSlot];
  static_assert(sizeof(a_lds) + sizeof(t_lds) <= 80 * 1024, "two workgroups per CU");
  static_assert(sizeof(t_lds) >= 2 * kRows * sizeof(int), "the epilogue's row table fits the ring");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = vq::uniform(tid >> 6);
  const int g = lane >> 4;
  const int m = lane & 15;
  const int L = 4 * (m & 7) + g;
  // Dense: grid (column tile, row tile).  MoE: a 1-D grid; workgroups are
  // dispatched to the 8 XCDs round-robin (workgroup p on XCD p % 8, its
  // p / 8-th).  XCD x runs the contiguous task range [x P, x P + P),
  // P = ceil(tasks / 8): the tasks of one expert share an XCD.  Within it,
  // groups of task_group tasks run column-major (column tile 0 of each task
  // of the group, then column tile 1, ...), so the workgroups resident at
  // once on the XCD hold a few tasks x a few column tiles at the same K
  // steps, and its L2 fetches each activation tile and each weight stripe
  // once for all of them.
  int64_t col_tile = blockIdx.x;
  int moe_task = 0;
  if constexpr (kMoe) {
    const int local = int(blockIdx.x >> 3);
    const int span = a.task_group * a.col_tiles;
    const int group = local / span;
    const int in_group = local - group * span;
    col_tile = in_group / a.task_group;
    const int idx = group * a.task_group + (in_group - int(col_tile) * a.task_group);
    const int per_xcd = (vq::uniform(a.table[2]) + 7) >> 3;
    if (idx >= per_xcd) return;
    moe_task = int(blockIdx.x & 7) * per_xcd + idx;
  }
  const int64_t col0 = col_tile * kTileCols;

  // ---- the tile's rows, matrix and scales ----
  int nrows;
  const uint8_t* trellis;
  const uint16_t* svh;
  int64_t tiles_n;
  int first = 0;
  if constexpr (kMoe) {
    // tile tasks: table[2] of them from task table[3] on
    const int task = moe_task;
    if (task >= a.table[2]) return;
    const int4 tk = reinterpret_cast<const int4*>(a.table + a.task_offset)[a.table[3] + task];
    const int expert = vq::uniform(tk.x);
    first = vq::uniform(tk.y);
    nrows = vq::uniform(tk.z);
    const int64_t* ptrs = a.ptrs + expert * 9 + a.projection * 3;
    const int64_t* meta = a.meta + expert * 12 + a.projection * 4;
    trellis = reinterpret_cast<const uint8_t*>(vq::uniform(ptrs[0]));
    svh = reinterpret_cast<const uint16_t*>(vq::uniform(ptrs[2]));
    tiles_n = vq::uniform(meta[1]) / 16;
    // an expert of another geometry or rate is never read: NaN rows
    const bool bad = vq::uniform(meta[0]) != a.kp || vq::uniform(meta[1]) != a.np ||
                     vq::uniform(meta[2]) != kBitsX2 || vq::uniform(meta[3]) != kCodebook;
    if (bad) {
      for (int r = wave; r < nrows; r += kTileWaves) {
        float* dst = a.moe_out + int64_t(a.table[4 + first + r]) * a.np + col0;
        for (int c = lane; c < kTileCols; c += 64) {
          if (col0 + c < a.np) dst[c] = __builtin_nanf("");
        }
      }
      return;
    }
  } else {
    const int64_t row0 = int64_t(blockIdx.y) * kRows;
    nrows = int(a.rows - row0 < kRows ? a.rows - row0 : kRows);
    trellis = a.trellis;
    svh = a.svh;
    tiles_n = a.tiles_n;
  }
  // the activation row of the tile's row t (rows past the tile repeat its
  // last row)
  auto row_of = [&](int t) -> int {
    t = t < nrows ? t : nrows - 1;
    if constexpr (kMoe) {
      return a.table[4 + first + t];
    } else {
      return int(int64_t(blockIdx.y) * kRows + t);
    }
  };
  // thread t < kRows keeps row t's id and exponent for the epilogue
  int my_row = 0, my_e = 0;
  if (tid < kRows) {
    my_row = row_of(tid);
    my_e = a.row_exp[int64_t(my_row) * a.exp_stride];
  }

  const int nblocks = (nrows + 15) >> 4;  // 16-row blocks with rows
  const int steps = int(a.kp / 32);
  const int last = steps - 1;
  const int row_bytes = int(tiles_n * kTileBytes);
  const int64_t tc0 = col0 / 16 + 4 * wave;  // this wavefront's first tile column
  // columns past the matrix (a partial last tile) read tile column 0 again
  // and are never stored
  const int64_t tc_load = tc0 + 4 <= tiles_n ? tc0 : 0;

  // ---- loads ----
  // trellis: 16-byte chunk c = lane + 64 u of load u (chunks past the
  // step's two tile rows copy the first chunk again, into the slot's unread
  // tail); chunk c lands at byte 16 c of the slot
  const __amdgpu_buffer_rsrc_t t_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(trellis + tc_load * kTileBytes), 0, (steps * 2 - 1) * row_bytes + kRowChunk,
      0x00020000);
  int t_voff[kTL];
#pragma unroll
  for (int u = 0; u < kTL; ++u) {
    const int c = lane + 64 * u;
    t_voff[u] = c < 2 * kChunkLanes ? (c / kChunkLanes) * row_bytes + 16 * (c % kChunkLanes) : 0;
  }
  // (each builtin's offsets are locals: an array element passed straight
  // to the builtin makes the host compilation drop the kernel's launch stub)
  auto load_trellis = [&](int s) {
#pragma unroll
    for (int u = 0; u < kTL; ++u) {
      const int voff = t_voff[u];
      __builtin_amdgcn_raw_ptr_buffer_load_lds(t_rsrc, (tile_lds_ptr_t)&t_lds[wave][s % kTileRing][1024 * u], 16,
                                               voff, s * 2 * row_bytes, 0, 0);
    }
  };
  // activations: this wavefront's row blocks rb = kADma * wave + i; lane
  // (g, m) copies group g of row 16 rb + m, its high part into block rb of
  // the buffer and its low part (2 kp bytes on) into block kBlocks + rb
  const __amdgpu_buffer_rsrc_t a_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(a.act), 0, int(a.act_rows * a.act_row_bytes), 0x00020000);
  const int lo_off = int(2 * a.kp);
  int a_voff[kADma];
#pragma unroll
  for (int i = 0; i < kADma; ++i) {
    const int rb = kADma * wave + i;
    a_voff[i] = int(int64_t(row_of(16 * rb + m)) * a.act_row_bytes + 16 * g);
  }
  auto load_act = [&](int s) {
    const int buf = s % kTileABufs;
#pragma unroll
    for (int i = 0; i < kADma; ++i) {
      const int hi_voff = a_voff[i];
      __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rsrc, (tile_lds_ptr_t)&a_lds[buf][kADma * wave + i][0],
                                               16, hi_voff, s * 64, 0, 0);
      if constexpr (kLo) {
        const int lo_voff = hi_voff + lo_off;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rsrc,
                                                 (tile_lds_ptr_t)&a_lds[buf][kBlocks + kADma * wave + i][0],
                                                 16, lo_voff, s * 64, 0, 0);
      }
    }
  };

  // ring words: tile column t = 2 p + (m >> 3) of tile row h of the slot
  int word_off[2][2][kWords];
  {
    int idx[kWords];
    lane_word_index<kBitsX2>(L, idx);
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < kWords; ++i)
          word_off[p][h][i] = h * kRowChunk + (2 * p + (m >> 3)) * kTileBytes + 4 * idx[i];
  }
  f32x4_t acc[kBlocks][2][2];
#pragma unroll
  for (int rb = 0; rb < kBlocks; ++rb)
#pragma unroll
    for (int p = 0; p < 2; ++p) acc[rb][p][0] = acc[rb][p][1] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  // LDS reads in the loop go through tile_read* (outside the compiler's
  // tracking of the LDS-DMA loads, which would make each read wait for
  // every load in flight); tile_ready names the values a wait made ready.
  const uint32_t a_lane = vq::lds_address(&a_lds[0][0][0]) + 16 * lane;
  const uint32_t t_base = vq::lds_address(&t_lds[wave][0][0]);
  uint32_t word_addr[2][2][kWords];
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < kWords; ++i) word_addr[p][h][i] = t_base + word_off[p][h][i];
  uint32_t words[2][2][kWords];
  auto read_words = [&](auto slot) {
    constexpr int kSlotIdx = decltype(slot)::value;
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < kWords; ++i) tile_read4<kSlotIdx * kSlot>(words[p][h][i], word_addr[p][h][i]);
  };

  // decode of step words w into B operands of pair p: first / second MFMA
  auto decode_pair = [&](const uint32_t (&w)[2][2][kWords], int p, half8_t (&b)[2][2]) {
    uint32_t q0[4], q1[4];
    decode_words<kBitsX2, kCodebook>(L, w[p][0], q0);
    decode_words<kBitsX2, kCodebook>(L, w[p][1], q1);
    b[p][0] = __builtin_bit_cast(half8_t, u32x4_t{q0[0], q0[1], q1[0], q1[1]});
    b[p][1] = __builtin_bit_cast(half8_t, u32x4_t{q0[2], q0[3], q1[2], q1[3]});
  };

  half8_t b_cur[2][2];  // step s's B operands

  // step s, its trellis in ring slot kS = s % 4 (the loop runs four steps
  // an iteration: steps is a multiple of 4): the MFMAs of kRB row blocks of
  // step s on b_cur (high parts, then low parts), with the words of step
  // s + 1 read and decoded between them
  auto step = [&](int s, auto slot, auto row_blocks) __attribute__((always_inline)) {
    constexpr int kS = decltype(slot)::value;
    constexpr int kRB = decltype(row_blocks)::value;
    static_assert(kRB >= 2, "two row blocks read ahead");
    load_act(min(s + 2, last));
    // T(s + 1) landed: after it came A(s), T(s + 2), A(s + 1), T(s + 3),
    // A(s + 2)
    vq::wait_vmcnt<3 * kAL + 2 * kTL>();
    read_words(std::integral_constant<int, (kS + 1) % kTileRing>{});  // (past the last step: unused)
    // this step's slot (its words read and decoded a step ago) takes step s + 4
    load_trellis(min(s + 4, last));

    half8_t b_next[2][2];
    const uint32_t a_buf = a_lane + uint32_t(s % kTileABufs) * (kParts * kBlocks * 1024);
    half8_t ah[kRB], al[kRB];
    auto read_a = [&](auto rb_tag) {
      constexpr int rb = decltype(rb_tag)::value;
      tile_read16<rb * 1024>(ah[rb], a_buf);
      if constexpr (kLo) tile_read16<(kBlocks + rb) * 1024>(al[rb], a_buf);
    };
    read_a(std::integral_constant<int, 0>{});
    read_a(std::integral_constant<int, 1>{});
    static_for<kRB>([&](auto rb_tag) {
      constexpr int rb = decltype(rb_tag)::value;
      // the reads of row block rb + 1 may still be pending (the words were
      // read before row block 0's)
      tile_lgkm<rb + 1 < kRB ? kParts : 0>();
      tile_ready(ah[rb]);
      if constexpr (kLo) tile_ready(al[rb]);
      if constexpr (rb == 0) tile_ready(words);
      if constexpr (rb + 2 < kRB) read_a(std::integral_constant<int, rb + 2>{});
      if constexpr (rb == 0) {
        decode_pair(words, 0, b_next);
        decode_pair(words, 1, b_next);
      }
#pragma unroll
      for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[rb][p][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[rb], b_cur[p][j], acc[rb][p][j], 0, 0, 0);
      if constexpr (kLo) {
#pragma unroll
        for (int p = 0; p < 2; ++p)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[rb][p][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[rb], b_cur[p][j], acc[rb][p][j], 0, 0, 0);
      }
    });
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      b_cur[p][0] = b_next[p][0];
      b_cur[p][1] = b_next[p][1];
    }
    // A(s + 1) of this wavefront landed: after it came T(s + 3), A(s + 2),
    // T(s + 4); then every wavefront's (and every read of buffer s) is done
    vq::wait_vmcnt<kAL + 2 * kTL>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  // Row blocks past the tile's rows hold copies of its last row: a tile of
  // up to half the rows runs the half-height loop, any other the full one;
  // an MoE task (an expert's rows, often well under 128) the loop of its
  // height rounded up to 2, 4, 5, 6 or 8 row blocks.  None branches around
  // an MFMA.
  auto run = [&](auto row_blocks) __attribute__((always_inline)) {
    for (int s = 0; s < steps; s += kTileRing) {
      step(s, std::integral_constant<int, 0>{}, row_blocks);
      step(s + 1, std::integral_constant<int, 1>{}, row_blocks);
      step(s + 2, std::integral_constant<int, 2>{}, row_blocks);
      step(s + 3, std::integral_constant<int, 3>{}, row_blocks);
    }
  };
  static_assert(kBlocks == 8, "row-block heights below");
  // A wavefront whose tile columns all lie past the matrix (in the last
  // column tile of a projection whose width is no multiple of 256) only
  // loads its share of the activation tiles and meets every barrier: its
  // SIMD serves the CU's other wavefronts meanwhile.
  const bool idle = tc0 >= tiles_n;
  if (idle) {
    asm volatile("" ::: "memory");
    load_act(0);
    load_act(min(1, last));
    vq::wait_vmcnt<kAL>();  // A(0) of this wavefront landed
    __builtin_amdgcn_s_barrier();
    for (int s = 0; s < steps; ++s) {
      asm volatile("" ::: "memory");
      load_act(min(s + 2, last));
      vq::wait_vmcnt<kAL>();  // A(s + 1) of this wavefront landed
      __builtin_amdgcn_s_barrier();
    }
    asm volatile("" ::: "memory");
  } else {
    // ---- prologue: T(0), T(1), A(0), T(2), A(1), T(3) in that order ----
    asm volatile("" ::: "memory");
    load_trellis(0);
    load_trellis(min(1, last));
    load_act(0);
    load_trellis(min(2, last));
    load_act(min(1, last));
    load_trellis(min(3, last));
    vq::wait_vmcnt<kAL + 2 * kTL>();  // T(0), T(1) and A(0) of this wavefront landed
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    read_words(std::integral_constant<int, 0>{});
    tile_lgkm<0>();
    tile_ready(words);
    decode_pair(words, 0, b_cur);
    decode_pair(words, 1, b_cur);
    if constexpr (kMoe) {
      if (nblocks > 6) {
        run(std::integral_constant<int, 8>{});
      } else if (nblocks > 5) {
        run(std::integral_constant<int, 6>{});
      } else if (nblocks > 4) {
        run(std::integral_constant<int, 5>{});
      } else if (nblocks > 2) {
        run(std::integral_constant<int, 4>{});
      } else {
        run(std::integral_constant<int, 2>{});
      }
    } else if (nblocks > kBlocks / 2) {
      run(std::integral_constant<int, kBlocks>{});
    } else {
      run(std::integral_constant<int, kBlocks / 2>{});
    }
  }

  // ---- epilogue ----
  // the clamped loads past the last step may still be landing in the LDS
  // the epilogue reuses
  vq::wait_vmcnt<0>();
  __syncthreads();
  int* row_id = reinterpret_cast<int*>(&t_lds[0][0][0]);
  int* row_e = row_id + kRows;
  if (tid < kRows) {
    row_id[tid] = my_row;
    row_e[tid] = my_e;
  }
  __syncthreads();
  // Wavefront w finishes 128-column block blk = w & 1 of the tile: in each
  // row block, rows 8 (w >> 1) + 4 b + q (b = 0, 1), one per 16-lane row q
  // = lane >> 4, lane l = lane & 15 holding the block's columns 8 l .. 8 l +
  // 7, so the output H128 runs in registers and DPP (h128_rows) and each
  // lane stores its eight outputs together.  The lane's eight svh values are
  // loaded once, here (loads and stores share one in-order counter: a load
  // waited for after an output store also waits for the store).
  const int blk = wave & 1;
  const int q = lane >> 4;
  const int l = lane & 15;
  const int64_t c0 = col0 + 128 * blk + 8 * l;  // the lane's first column
  float sv[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) sv[j] = c0 + j < a.np ? vq::f16_to_f32(svh[c0 + j]) : 0.0f;
  float* red = reinterpret_cast<float*>(&a_lds[0][0][0]);  // [16][kTileRedStride]
  static_assert(sizeof(a_lds) >= 16 * kTileRedStride * sizeof(float), "epilogue rows fit");
#pragma unroll
  for (int rb = 0; rb < kBlocks; ++rb) {
    // (row blocks past the tile's rows store nothing: the workgroup stops
    // there, all its threads together)
    if (rb > 0 && 16 * rb >= nrows) break;
    // lane (g, m) holds rows 4 g + i of the block, column m of each MFMA
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * g + i;
      const int e = row_e[16 * rb + r];
#pragma unroll
      for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int col = 64 * wave + 32 * p + 16 * (m >> 3) + (m & 7) + 8 * j;
          red[r * kTileRedStride + col] = ldexpf(acc[rb][p][j][i], -e);
        }
    }
    __syncthreads();
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int r = 8 * (wave >> 1) + 4 * b + q;
      const int tr = 16 * rb + r;
      const float* src = red + r * kTileRedStride + 128 * blk + 8 * l;
      const f32x4_t x0 = *reinterpret_cast<const f32x4_t*>(src);
      const f32x4_t x1 = *reinterpret_cast<const f32x4_t*>(src + 4);
      float v[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float y0 = x0[j], y1 = x1[j];
        v[j] = y0;
        v[4 + j] = y1;
      }
      vq::h128_rows(v, l);
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] *= sv[j];
      if (tr < nrows) {
        if constexpr (kMoe) {
          vq::store8_act(a.moe_out, vq::kFP32, int64_t(row_id[tr]) * a.np + c0, v, a.np - c0);
        } else {
          const int64_t row = int64_t(blockIdx.y) * kRows + tr;
          vq::store8_act(a.out, a.out_dtype, row * a.logical_out + c0, v, a.logical_out - c0);
        }
      }
    }
    __syncthreads();
  }
}

// The tile GEMM's instantiations are split over kTileParts separately
// compiled objects (exl3_tile_part.hip): format i of VQ_EXL3_FORMATS lives
// in part i % kTileParts, with its dense kernels (both precisions) and, for
// mul1 rates, its MoE kernels.
constexpr int kTileParts = 4;

// Launches tile_gemm<bits_x2, codebook, moe, lo> for a format of part P
// (a format of another part is refused).
template <int P>
int tile_launch_part(int64_t bits_x2, int64_t codebook, bool moe, bool lo, const TileArgs& a, dim3 grid,
                     hipStream_t stream);

// Launches tile_gemm<bits_x2, codebook, moe, lo> from the part that holds it
// (exl3_gemm.hip).
int launch_tile_gemm(int64_t bits_x2, int64_t codebook, bool moe, bool lo, const TileArgs& a, dim3 grid,
                     hipStream_t stream);

}  // namespace exl3
