// EXL3 routed-expert MoE for gfx950: the reference's moe_out / moe_out_v2
// contract (csrc/exl3/moe.cu:304-446, csrc/exl3/moe_v2.h), rebuilt around a
// grouped small-M MFMA kernel.
//
// Launch sequence on the caller's stream (as the reference's run_moe_out):
//  1. moe_route groups the local assignments by local expert (counts,
//     scan, sorted list: the GEMV experts' rows, then the tile experts'
//     rows) and cuts each expert's rows into tasks of at most 32 rows (8 for
//     the run-time-format decode: the per-expert token sort): one workgroup
//     below 8192 routed slots, else moe_route_count / moe_route /
//     moe_route_fill over many workgroups.
//  2. per projection (gate, up): moe_form builds t = H128(x[a / topk] * suh)
//     of every local assignment, as FP16 high/low parts in MFMA B-operand
//     order with one power-of-two scale per assignment row (the high parts
//     alone for the tile experts' rows when the tile GEMM runs at FP16
//     precision); moe_gemv runs
//     every task against its expert's matrix: one workgroup = (task, 128
//     output columns) over the whole K range, trellis streamed with
//     coalesced buffer loads, decoded in registers, each decoded operand fed
//     to v_mfma_f32_16x16x32_f16 for every 8-row sub-block of the task, then
//     the output H128 and svh in the same kernel.  Experts with at least
//     48 routed rows (a call's fixed rate, 16-byte aligned matrices) run
//     instead on the tile GEMM (exl3_tile.h: 128-row tasks x 256 columns,
//     high and low parts, or the high parts alone under
//     exl3_set_tile_precision(1)), when their tasks make enough
//     workgroups to fill the chip.
//  3. moe_form (activation): clamp, SiLU(gate) * up * suh_down, H128 - the
//     down projection's activations, in the same B-operand form.
//  4. moe_gemv for the down projection.
//  5. moe_combine: per token, one FMA per local route in route order with
//     the routing weight, rounded to the output dtype.
//
// Expert formats come from packed_meta on the device.  moe_out decodes any
// admitted format at run time; moe_out_v2 (one bits_x2 for the layer, mul1)
// runs the decode specialized for that rate.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <climits>
#include <type_traits>

#include "../../include/vllm_mi355x.h"
#include "common.h"
#include "exl3_codec.h"
#include "exl3_internal.h"
#include "exl3_tile.h"

namespace exl3 {
namespace {

constexpr int kRouteThreads = 1024;
constexpr int64_t kMaxRouteExperts = 4096;
// Rows of one expert per GEMV task: every decoded weight operand feeds the
// MFMAs of up to four 8-row sub-blocks, so a fixed-rate expert's weights
// are decoded once per 32 of its rows.  The run-time-format decode needs the
// registers the extra accumulators would take: 8 rows there.
constexpr int kTaskRows = 32;
constexpr int task_rows(int bits_x2) { return bits_x2 > 0 ? kTaskRows : 8; }
// The rate of the fixed-rate GEMV serving a call's bits_x2 (moe_out_v2's
// mul1 rates 2..16 and moe_out_prefill's 10, decoded by specialized
// kernels), or 0: the run-time-format decode, which serves moe_out (any
// admitted format per expert).
constexpr int fixed_rate(int64_t bits_x2) { return bits_x2 >= 2 && bits_x2 <= 16 ? int(bits_x2) : 0; }

// Routing of one call (reference: csrc/exl3/moe.cu:19-55).
struct Routing {
  const void* ids;          // [rows][topk] int32 or int64 global expert ids
  const void* expert_map;   // [global] int32 or int64: local id or -1
  const int64_t* ptrs;      // [local][3][3]: trellis, suh, svh
  const int64_t* meta;      // [local][3][4]: padded_in, padded_out, bits_x2, codebook
  int64_t global_experts;
  int64_t local_experts;
  int64_t topk;
  bool ids64;
  bool map64;
};

__device__ __forceinline__ int64_t integer_at(const void* p, bool wide, int64_t i) {
  return wide ? static_cast<const int64_t*>(p)[i] : static_cast<const int32_t*>(p)[i];
}

__device__ __forceinline__ int64_t local_expert(const Routing& r, int64_t a) {
  const int64_t g = integer_at(r.ids, r.ids64, a);
  if (g < 0 || g >= r.global_experts) return -1;
  const int64_t l = integer_at(r.expert_map, r.map64, g);
  return l >= 0 && l < r.local_experts ? l : -1;
}

// Workspace layout (reference sizes: moe.cu:304-317; plus scale exponents).
struct MoeLayout {
  int64_t hpad, ipad, assignments;
  __host__ __device__ int64_t kmax() const { return hpad > ipad ? hpad : ipad; }
  // FP32 offsets
  __host__ __device__ int64_t input() const { return 0; }                       // A x hpad
  __host__ __device__ int64_t gate() const { return assignments * hpad; }        // A x ipad
  __host__ __device__ int64_t up() const { return gate() + assignments * ipad; } // A x ipad
  // the down projection's B operands (A x ipad): a region of their own, since
  // one block's halves would land on gate floats another wavefront still reads
  __host__ __device__ int64_t act() const { return up() + assignments * ipad; }
  __host__ __device__ int64_t ints() const { return act() + assignments * ipad; }
  // int32 offsets from ints(): header[4], sorted[A rounded to 4], tasks[A] (int4),
  // exponents[A][kmax / 128], the local expert of each sorted row[A]
  __host__ __device__ int64_t sorted() const { return 4; }
  __host__ __device__ int64_t tasks() const { return 4 + (assignments + 3) / 4 * 4; }
  __host__ __device__ int64_t exps() const { return tasks() + 4 * assignments; }
  __host__ __device__ int64_t row_experts() const { return exps() + assignments * (kmax() / 128); }
  __host__ __device__ int64_t total() const { return ints() + row_experts() + assignments; }
};

// ---- 1. route ------------------------------------------------------------------

// An expert of a fixed-rate call whose routed rows reach this count, and
// whose three matrices are 16-byte aligned (LDS-DMA), runs on the tile GEMM
// in tasks of up to 128 rows; the others run on the GEMV in tasks of up to
// task_rows rows.
constexpr int kTileMinRows = 48;
// Tile tasks run the whole K range each: a call uses them only when they
// make at least this many workgroups in the narrower projection's launch.
constexpr int64_t kMinTileBlocks = 128;
// exl3_set_moe_tile_rows: the threshold in use (0 = kTileMinRows), which
// also lifts the workgroup minimum (tests force the tile path with it)
std::atomic<int> g_tile_rows_override{0};
int tile_min_rows() {
  const int forced = g_tile_rows_override.load();
  return forced > 0 ? forced : kTileMinRows;
}
int tile_min_tasks(int automatic) { return g_tile_rows_override.load() > 0 ? 0 : automatic; }

__device__ __forceinline__ bool tile_expert(const Routing& r, int e, int rows, int min_rows) {
  if (rows < min_rows) return false;
  const int64_t* p = r.ptrs + int64_t(e) * 9;
  return ((p[0] | p[3] | p[6]) & 15) == 0;
}

// Table (int32, in the workspace): header {routed rows, GEMV tasks, tile
// tasks, first tile task}, the routed assignments sorted by local expert
// (the GEMV experts' rows first, then the tile experts' rows, each part in
// expert order), then the tasks {expert, first sorted row, rows, 0}: GEMV
// tasks first, tile tasks after them (every task has a row, so both fit in
// A entries).
// tile_rows: the routed-row threshold of the tile GEMM (0: no tile tasks);
// with fewer than min_tile_tasks tile tasks in all (too few workgroups to
// fill the chip: each runs the whole K range), every expert takes the GEMV.

// Local expert of global id g, or -1.
__device__ __forceinline__ int local_of(const Routing& r, int64_t g) {
  const bool in = g >= 0 && g < r.global_experts;
  const int64_t l = in ? integer_at(r.expert_map, r.map64, g) : -1;
  return l >= 0 && l < r.local_experts ? int(l) : -1;
}

// Calls of at least kRouteSplitMin routed slots group their rows over many
// workgroups in three launches: moe_route_count (per part of kRoutePart
// slots: each slot's expert and place among the part's rows of that expert,
// and the part's histogram), moe_route with parts > 0 (counts summed from
// the histograms, the tables, and each (part, expert)'s first sorted row
// written back over its histogram entry), moe_route_fill (each slot to its
// sorted row).  The packed slots and the histograms live in the workspace's
// gate-result region, which no launch reads before the gate projection
// writes it.
constexpr int64_t kRouteSplitMin = 8192;
constexpr int kRoutePartThreads = 256;
constexpr int kRoutePartSlots = 8;  // slots a thread of a part takes
constexpr int kRoutePart = kRoutePartThreads * kRoutePartSlots;
// the one-workgroup route: slots a thread holds; histogram entries loaded
// at a time
constexpr int kRouteHeld = int(kRouteSplitMin / kRouteThreads);
constexpr int kRouteBatch = 8;

// packed[a] = expert << 16 | place of slot a among its part's rows of that
// expert (or -1: not routed here); hist[part][expert] = the part's rows.
__global__ __launch_bounds__(kRoutePartThreads) void moe_route_count(Routing routing, int64_t assignments,
                                                                     int* packed, int* hist) {
  extern __shared__ int part_count[];
  const int experts = int(routing.local_experts);
  for (int e = threadIdx.x; e < experts; e += kRoutePartThreads) part_count[e] = 0;
  __syncthreads();
  const int64_t a0 = int64_t(blockIdx.x) * kRoutePart + threadIdx.x;
  int64_t g[kRoutePartSlots];
#pragma unroll
  for (int u = 0; u < kRoutePartSlots; ++u) {
    const int64_t a = a0 + u * kRoutePartThreads;
    g[u] = a < assignments ? integer_at(routing.ids, routing.ids64, a) : -1;
  }
  int e[kRoutePartSlots];
#pragma unroll
  for (int u = 0; u < kRoutePartSlots; ++u) e[u] = local_of(routing, g[u]);
#pragma unroll
  for (int u = 0; u < kRoutePartSlots; ++u) {
    const int64_t a = a0 + u * kRoutePartThreads;
    const int v = e[u] >= 0 ? (e[u] << 16) | atomicAdd(&part_count[e[u]], 1) : -1;
    if (a < assignments) packed[a] = v;
  }
  __syncthreads();
  for (int x = threadIdx.x; x < experts; x += kRoutePartThreads) {
    hist[int64_t(blockIdx.x) * experts + x] = part_count[x];
  }
}

// sorted[first row of (part, expert) + place] = a for every routed slot a,
// and row_expert[that row] = its expert.
__global__ __launch_bounds__(kRoutePartThreads) void moe_route_fill(int64_t assignments, int experts,
                                                                    const int* packed, const int* first,
                                                                    int* sorted, int* row_expert) {
  const int64_t a0 = int64_t(blockIdx.x) * kRoutePart + threadIdx.x;
  const int* part_first = first + int64_t(blockIdx.x) * experts;
  int v[kRoutePartSlots];
#pragma unroll
  for (int u = 0; u < kRoutePartSlots; ++u) {
    const int64_t a = a0 + u * kRoutePartThreads;
    v[u] = a < assignments ? packed[a] : -1;
  }
#pragma unroll
  for (int u = 0; u < kRoutePartSlots; ++u) {
    if (v[u] >= 0) {
      const int row = part_first[v[u] >> 16] + (v[u] & 0xffff);
      sorted[row] = int(a0 + u * kRoutePartThreads);
      row_expert[row] = v[u] >> 16;
    }
  }
}

// The route in one workgroup.  parts == 0 (calls of fewer than
// kRouteSplitMin slots): from the ids, each thread's slots held in
// registers: one round of id loads, one of expert-map loads, and the
// counting atomic returns each slot's place among its expert's rows, so the
// sorted list is written without a second pass.  parts > 0: the counts are
// the sums of moe_route_count's histograms, each of whose entries is
// replaced by the first sorted row of that (part, expert), and
// moe_route_fill writes the sorted list.
__global__ __launch_bounds__(kRouteThreads) void moe_route(Routing routing, int64_t assignments,
                                                           int task_rows, int tile_rows,
                                                           int min_tile_tasks, int* table, int* row_expert,
                                                           int* hist, int parts) {
  extern __shared__ int route_shared[];
  const int experts = int(routing.local_experts);
  int* count = route_shared;               // rows per expert
  int* row_begin = count + experts;
  int* task_begin = row_begin + experts;   // GEMV tasks, experts + 1 entries
  int* tile_begin = task_begin + experts + 1;  // tile tasks, experts + 1 entries
  constexpr int kWaves = kRouteThreads / 64;
  __shared__ int wave_sums[kWaves][4];     // per wavefront: GEMV rows, tile rows, GEMV tasks, tile tasks
  __shared__ int tiles_in_all;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  if (parts > 0) {
    for (int e = tid; e < experts; e += kRouteThreads) {
      int c = 0;
      for (int p0 = 0; p0 < parts; p0 += kRouteBatch) {
        int n[kRouteBatch];  // a batch of parts' loads in flight together
#pragma unroll
        for (int u = 0; u < kRouteBatch; ++u) n[u] = p0 + u < parts ? hist[int64_t(p0 + u) * experts + e] : 0;
#pragma unroll
        for (int u = 0; u < kRouteBatch; ++u) c += n[u];
      }
      count[e] = c;
    }
  } else {
    for (int e = tid; e < experts; e += kRouteThreads) count[e] = 0;
  }
  if (tid == 0) tiles_in_all = 0;
  __syncthreads();
  // parts == 0: slot tid + kRouteThreads * u as (expert << 16 | its place
  // among that expert's rows), or -1
  int hv[kRouteHeld];
  if (parts == 0) {
    int64_t g[kRouteHeld];
#pragma unroll
    for (int u = 0; u < kRouteHeld; ++u) {
      const int64_t a = tid + int64_t(u) * kRouteThreads;
      g[u] = a < assignments ? integer_at(routing.ids, routing.ids64, a) : -1;
    }
    int e[kRouteHeld];
#pragma unroll
    for (int u = 0; u < kRouteHeld; ++u) e[u] = local_of(routing, g[u]);
#pragma unroll
    for (int u = 0; u < kRouteHeld; ++u) hv[u] = e[u] >= 0 ? (e[u] << 16) | atomicAdd(&count[e[u]], 1) : -1;
  }
  __syncthreads();
  // each thread a contiguous run of experts
  const int per = (experts + kRouteThreads - 1) / kRouteThreads;
  const int e0 = min(experts, tid * per);
  const int e1 = min(experts, e0 + per);
  if (tile_rows > 0) {
    int mine = 0;
    for (int e = e0; e < e1; ++e) {
      if (tile_expert(routing, e, count[e], tile_rows)) mine += (count[e] + kTileRows - 1) / kTileRows;
    }
    if (mine > 0) atomicAdd(&tiles_in_all, mine);
    __syncthreads();
    if (tiles_in_all < min_tile_tasks) tile_rows = 0;
  }
  // exclusive scan of (GEMV rows, tile rows, GEMV tasks, tile tasks) over
  // experts: within each wavefront, then over the wavefronts' sums
  int own[4] = {0, 0, 0, 0};
  for (int e = e0; e < e1; ++e) {
    const int c = count[e];
    if (tile_rows > 0 && tile_expert(routing, e, c, tile_rows)) {
      own[1] += c;
      own[3] += (c + kTileRows - 1) / kTileRows;
    } else {
      own[0] += c;
      own[2] += (c + task_rows - 1) / task_rows;
    }
  }
  int inc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    inc[i] = own[i];
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int v = __shfl_up(inc[i], d, 64);
      if (lane >= d) inc[i] += v;
    }
  }
  if (lane == 63) {
#pragma unroll
    for (int i = 0; i < 4; ++i) wave_sums[wave][i] = inc[i];
  }
  __syncthreads();
  int before[4] = {0, 0, 0, 0}, total[4] = {0, 0, 0, 0};
  for (int w = 0; w < kWaves; ++w) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int v = wave_sums[w][i];
      if (w < wave) before[i] += v;
      total[i] += v;
    }
  }
  const int gemv_rows = total[0];
  int row_at = before[0] + inc[0] - own[0];
  int trow_at = gemv_rows + before[1] + inc[1] - own[1];
  int task_at = before[2] + inc[2] - own[2];
  int tile_at = before[3] + inc[3] - own[3];
  for (int e = e0; e < e1; ++e) {
    const int c = count[e];
    const bool tile = tile_rows > 0 && tile_expert(routing, e, c, tile_rows);
    row_begin[e] = tile ? trow_at : row_at;
    task_begin[e] = task_at;
    tile_begin[e] = tile_at;
    if (parts > 0) {
      // the parts' rows of this expert follow each other in part order
      int at = row_begin[e];
      for (int p0 = 0; p0 < parts; p0 += kRouteBatch) {
        int n[kRouteBatch];
#pragma unroll
        for (int u = 0; u < kRouteBatch; ++u) n[u] = p0 + u < parts ? hist[int64_t(p0 + u) * experts + e] : 0;
#pragma unroll
        for (int u = 0; u < kRouteBatch; ++u) {
          if (p0 + u < parts) hist[int64_t(p0 + u) * experts + e] = at;
          at += n[u];
        }
      }
    }
    if (tile) {
      trow_at += c;
      tile_at += (c + kTileRows - 1) / kTileRows;
    } else {
      row_at += c;
      task_at += (c + task_rows - 1) / task_rows;
    }
  }
  const int total_rows = gemv_rows + total[1];
  const int total_tasks = total[2];
  const int total_tiles = total[3];
  if (tid == 0) {
    task_begin[experts] = total_tasks;
    tile_begin[experts] = total_tiles;
    table[0] = total_rows;
    table[1] = total_tasks;
    table[2] = total_tiles;
    table[3] = total_tasks;
  }
  __syncthreads();
  int4* task_table = reinterpret_cast<int4*>(table + MoeLayout{0, 0, assignments}.tasks());
  // task t of a list: the last expert whose first task is at or before t
  // (experts without tasks of that list share their successor's start, so
  // the search lands on the owner)
  auto owner = [&](const int* begin, int t) {
    int lo = 0, hi = experts;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (begin[mid] <= t) lo = mid; else hi = mid;
    }
    return lo;
  };
  for (int t = tid; t < total_tasks; t += kRouteThreads) {
    const int e = owner(task_begin, t);
    const int first = row_begin[e] + (t - task_begin[e]) * task_rows;
    const int end = row_begin[e] + count[e];
    task_table[t] = make_int4(e, first, min(task_rows, end - first), 0);
  }
  for (int t = tid; t < total_tiles; t += kRouteThreads) {
    const int e = owner(tile_begin, t);
    const int first = row_begin[e] + (t - tile_begin[e]) * kTileRows;
    const int end = row_begin[e] + count[e];
    task_table[total_tasks + t] = make_int4(e, first, min(kTileRows, end - first), 0);
  }
  if (parts > 0) return;  // moe_route_fill writes the sorted list
  int* sorted = table + 4;
#pragma unroll
  for (int u = 0; u < kRouteHeld; ++u) {
    if (hv[u] >= 0) {
      const int row = row_begin[hv[u] >> 16] + (hv[u] & 0xffff);
      sorted[row] = int(tid + u * kRouteThreads);
      row_expert[row] = hv[u] >> 16;
    }
  }
}

// ---- 2/3. activations in B-operand form ----------------------------------------

// Half offset, within one assignment's [hi: k halves][lo: k halves], of
// input k's high part: each 32-input step is [g 0..3][8 slots], slot order
// {2g, 2g+1, 2g+8, 2g+9} of its two 16-input tile rows.
__device__ __forceinline__ int b_order(int k) {
  const int w = k & 31;
  const int g = (w & 7) >> 1;
  const int slot = 4 * (w >> 4) + (w & 1) + 2 * ((w >> 3) & 1);
  return (k & ~31) + g * 8 + slot;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, int(bytes), 0x00020000);
}

// Writes inputs k0 .. k0 + 7 (k0 % 8 == 0) of t, scaled by the row's
// power-of-two exponent, into the row's B-operand arrays: in b_order, inputs
// 2i and 2i + 1 of the eight are adjacent halves (one dword store each) at
// (k0 & ~31) + 8 i + 4 ((k0 >> 4) & 1) + 2 ((k0 >> 3) & 1).  The low parts
// only when `lo` (rows of tile experts use the high parts alone).
__device__ __forceinline__ void store8(__amdgpu_buffer_rsrc_t dst, int kp, int k0, const float (&v)[8],
                                       int e, bool lo) {
  const int base = (k0 & ~31) + 4 * ((k0 >> 4) & 1) + 2 * ((k0 >> 3) & 1);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float t0 = ldexpf(v[2 * i], e);
    const float t1 = ldexpf(v[2 * i + 1], e);
    const _Float16 h0 = _Float16(t0), h1 = _Float16(t1);
    const _Float16 l0 = _Float16(t0 - float(h0)), l1 = _Float16(t1 - float(h1));
    const uint32_t hw = uint32_t(__builtin_bit_cast(uint16_t, h0)) | (uint32_t(__builtin_bit_cast(uint16_t, h1)) << 16);
    const uint32_t lw = uint32_t(__builtin_bit_cast(uint16_t, l0)) | (uint32_t(__builtin_bit_cast(uint16_t, l1)) << 16);
    const int o = 2 * (base + 8 * i);  // bytes
    __builtin_amdgcn_raw_buffer_store_b32(hw, dst, o, 0, 0);
    if (lo) __builtin_amdgcn_raw_buffer_store_b32(lw, dst, o, 2 * kp, 0);
  }
}

// kActivate false: gate/up input, t = H128(x[a / topk] * suh_projection);
// true: down input from the gate/up results (already H128 * svh):
// clamp, SiLU(g) * u * suh_down, H128, into the act region.
// A wavefront forms four blocks at a time (block group G: blocks 4 G ..
// 4 G + 3, one per 16-lane row, eight inputs a lane), the first kCache
// groups it takes kept in registers (their loads issued together at clamped
// group indices), for the row maximum of |t|, then writes the high / low
// parts at the row's one power-of-two scale, so the expert GEMV sums the
// whole row before it unscales; groups past the register cache are formed
// again (the same operations, so the same values).  kWaveRow: each
// wavefront forms a sorted row of its own (four rows a workgroup: rows of
// up to 4 kCache groups, whose chains of dependent loads then overlap four
// times as deep); otherwise one workgroup a row, wavefront w taking groups
// w, w + 4, ... and the maximum met in LDS.  An expert whose matrix is not
// kp rows long gets NaN operands (its suh is not read).
// The longest rows formed one wavefront a row: gate / up inputs, and the
// down input (whose SwiGLU makes a row's groups VALU work better spread over
// four wavefronts beyond two groups); the fewest routed slots formed so.
constexpr int64_t kFormRowGroups = 6;
constexpr int64_t kFormRowGroupsActivate = 2;
constexpr int64_t kFormRowMin = 8192;
template <bool kActivate, int kCache, bool kWaveRow>
__global__ __launch_bounds__(256) void moe_form(Routing routing, const void* x, int x_dtype,
                                                int64_t hidden, int64_t intermediate, int projection,
                                                const int* table, float* ws, MoeLayout lay,
                                                float limit, bool tile_lo) {
  __shared__ uint32_t row_max;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int q = lane >> 4;   // the lane's block within a group
  const int l = lane & 15;   // its eight inputs within the block: 8 l ..
  const int64_t kp = kActivate ? lay.ipad : lay.hpad;
  const int64_t blocks = kp / 128;
  const int64_t groups = (blocks + 3) / 4;
  // the sorted row, the wavefront's first group and its group stride
  const int row = kWaveRow ? int(blockIdx.x) * 4 + wave : int(blockIdx.x);
  const int g0 = kWaveRow ? 0 : wave;
  constexpr int kStride = kWaveRow ? 1 : 4;
  if (row >= table[0]) return;
  const int64_t a = table[4 + row];
  const int64_t e = reinterpret_cast<const int*>(ws + lay.ints())[lay.row_experts() + row];
  const int64_t* ptrs = routing.ptrs + e * 9;
  // the tile experts' rows (sorted rows from the first tile task's first
  // on) feed only the tile GEMM, which reads the low parts unless it runs
  // at FP16 precision
  const bool lo = tile_lo || table[2] == 0 ||
                  row < reinterpret_cast<const int4*>(table + lay.tasks())[table[3]].y;
  int* exps = reinterpret_cast<int*>(ws + lay.ints()) + lay.exps() + a * (lay.kmax() / 128);
  const __amdgpu_buffer_rsrc_t dst =
      make_rsrc(ws + (kActivate ? lay.act() : lay.input()) + a * kp, uint32_t(kp) * 4u);
  const bool bad = routing.meta[e * 12 + projection * 4] != kp;
  const uint16_t* suh = reinterpret_cast<const uint16_t*>(ptrs[projection * 3 + 1]);
  // Buffer resources over the row's inputs (32-bit offsets; loads past the
  // end of x's row or of suh return zero, which forms zero).
  const int in_len = int(kActivate ? intermediate : hidden);
  const __amdgpu_buffer_rsrc_t suh_r = make_rsrc(suh, uint32_t(in_len) * 2u);
  const __amdgpu_buffer_rsrc_t x_r =
      make_rsrc(static_cast<const uint16_t*>(x) + (a / routing.topk) * hidden, uint32_t(hidden) * 2u);
  const __amdgpu_buffer_rsrc_t g_r = make_rsrc(ws + lay.gate() + a * lay.ipad, uint32_t(lay.ipad) * 4u);
  const __amdgpu_buffer_rsrc_t u_r = make_rsrc(ws + lay.up() + a * lay.ipad, uint32_t(lay.ipad) * 4u);
  // the first input of the lane's eight in group G (clamped to the last block)
  auto first_k = [&](int64_t G) { return int(min(4 * G + q, blocks - 1)) * 128 + 8 * l; };
  // eight 16-bit inputs k0 .. k0 + 7 of a buffer of len valid ones: one
  // 16-byte load, or, for the chunk that reaches past len, 2-byte loads
  // (a buffer load partly past the end returns zero as a whole; each 2-byte
  // load past it returns zero)
  auto load8 = [&](__amdgpu_buffer_rsrc_t r, int k0, int len, uint16_t (&h)[8]) {
    if (k0 + 8 <= len) {
      const u32x4_t w = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, 2 * k0, 0, 0));
#pragma unroll
      for (int j = 0; j < 8; ++j) h[j] = uint16_t(w[j >> 1] >> (16 * (j & 1)));
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) h[j] = __builtin_amdgcn_raw_buffer_load_b16(r, 2 * (k0 + j), 0, 0);
    }
  };
  auto form = [&](int64_t G, float (&v)[8]) {
    const int k0 = first_k(G);
    if (bad) {
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = __builtin_nanf("");
      return;
    }
    if constexpr (!kActivate) {
      uint16_t xh[8], sh[8];
      load8(x_r, k0, in_len, xh);
      load8(suh_r, k0, in_len, sh);
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = u16_act(xh[j], x_dtype) * vq::f16_to_f32(sh[j]);
    } else {
      float gv[8], uv[8];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const u32x4_t gq = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(g_r, 4 * k0 + 16 * h, 0, 0));
        const u32x4_t uq = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(u_r, 4 * k0 + 16 * h, 0, 0));
        // each element to a scalar before the bit cast: a bit cast of a
        // vector element expression is emitted as a read of element 0
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t gw = gq[i], uw = uq[i];
          gv[4 * h + i] = __builtin_bit_cast(float, gw);
          uv[4 * h + i] = __builtin_bit_cast(float, uw);
        }
      }
      uint16_t sd[8];
      load8(suh_r, k0, in_len, sd);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        v[j] = 0.0f;
        if (k0 + j < intermediate) {
          float gg = gv[j], uu = uv[j];
          if (limit > 0.0f) {
            gg = fminf(gg, limit);
            uu = fminf(fmaxf(uu, -limit), limit);
          }
          const float silu = gg / (1.0f + expf(-gg));
          v[j] = (silu * uu) * vq::f16_to_f32(sd[j]);
        }
      }
    }
    vq::h128_rows(v, l);
  };
  auto live = [&](int64_t G) { return 4 * G + q < blocks; };
  if constexpr (!kWaveRow) {
    if (threadIdx.x == 0) row_max = 0u;
    __syncthreads();
  }
  float mx = 0.0f;
  float c[kCache][8];
#pragma unroll
  for (int i = 0; i < kCache; ++i) {
    form(min(int64_t(g0 + kStride * i), groups - 1), c[i]);
  }
#pragma unroll
  for (int i = 0; i < kCache; ++i) {
    if (g0 + kStride * i < groups && live(g0 + kStride * i)) {
#pragma unroll
      for (int j = 0; j < 8; ++j) mx = fmaxf(mx, fabsf(c[i][j]));
    }
  }
  for (int64_t G = g0 + kStride * kCache; G < groups; G += kStride) {
    float v[8];
    form(G, v);
    if (live(G)) {
#pragma unroll
      for (int j = 0; j < 8; ++j) mx = fmaxf(mx, fabsf(v[j]));
    }
  }
  mx = vq::wave_max(mx, lane);
  int ex;
  if constexpr (kWaveRow) {
    ex = scale_exponent(__builtin_bit_cast(uint32_t, mx));
    if (lane == 0) exps[0] = ex;
  } else {
    if (lane == 0) atomicMax(&row_max, __builtin_bit_cast(uint32_t, mx));
    __syncthreads();
    ex = scale_exponent(row_max);
    if (threadIdx.x == 0) exps[0] = ex;
  }
#pragma unroll
  for (int i = 0; i < kCache; ++i) {
    if (g0 + kStride * i < groups && live(g0 + kStride * i)) store8(dst, int(kp), first_k(g0 + kStride * i), c[i], ex, lo);
  }
  for (int64_t G = g0 + kStride * kCache; G < groups; G += kStride) {
    float v[8];
    form(G, v);
    if (live(G)) store8(dst, int(kp), first_k(G), v, ex, lo);
  }
}

// ---- grouped expert GEMV ----------------------------------------------------------

// Decode of encoder lane L of a tile at run-time rate / codebook (moe_out):
// the scalar ring arithmetic, four window words, values as FP16 pairs.
__device__ __forceinline__ void decode_runtime(const uint8_t* tile, bool aligned, int bits_x2,
                                               int codebook, int L, uint32_t (&pair)[4]) {
  const int whole = bits_x2 >> 1;
  const int odd = bits_x2 & 1;
  const int ring = 128 * bits_x2;
  const int words = 4 * bits_x2;
  const int start = ((8 * L + 1) * whole + (odd ? 4 * L : 0) - 16 + ring) % ring;
  int w = start >> 5;
  uint32_t wd[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    wd[i] = aligned ? tile_word<true>(tile, 4 * w) : tile_word<false>(tile, 4 * w);
    w = w + 1 == words ? 0 : w + 1;
  }
  const int shift = start & 31;
  uint32_t u[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    const uint64_t two = (uint64_t(wd[i]) << 32) | wd[i + 1];
    u[i] = uint32_t(two >> (32 - shift));
  }
  uint32_t s[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int o = j * whole + (odd ? (j + 1) / 2 : 0);
    const int q = o >> 5;
    const uint32_t hi = q == 0 ? u[0] : (q == 1 ? u[1] : u[2]);
    const uint32_t lo = q == 0 ? u[1] : u[2];
    s[j] = uint32_t(((uint64_t(hi) << 32 | lo) >> (48 - (o & 31))) & 0xffffu);
  }
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    pair[p] = codebook == 1 ? codebook_pair<1>(s[2 * p], s[2 * p + 1])
                            : codebook_pair<2>(s[2 * p], s[2 * p + 1]);
  }
}

// Wave priority from progress (quarter q of the wavefront's steps: 3 - q).
// The SIMD issues from its oldest wavefront first: equal wavefronts sharing a
// saturated SIMD would otherwise finish one after another, and the last
// ones, left alone, cannot keep it busy.  Ranking them by progress keeps
// them level.
// Compares rather than a division (none in hardware).
__device__ __forceinline__ void progress_priority(int step, int steps) {
  const int q = 4 * step;
  if (q < steps) {
    __builtin_amdgcn_s_setprio(3);
  } else if (q < 2 * steps) {
    __builtin_amdgcn_s_setprio(2);
  } else if (q < 3 * steps) {
    __builtin_amdgcn_s_setprio(1);
  } else {
    __builtin_amdgcn_s_setprio(0);
  }
}

// One workgroup = (task, 128 output columns); wavefront w owns the column
// pair (two tile columns) 4 * blockIdx.x + w over the whole K range.  Each
// decoded step (two tile rows, 16 weights a lane) is an A operand of the
// MFMAs of every 8-row sub-block of the task (B columns 2r, 2r + 1: row r's
// high and low parts); the sums run over the whole row (one scale per
// assignment row) and fold once.
// kBitsX2 = 0: the expert's format at run time.
// want_bits (run-time decode only): the layer's mul1 rate every expert must
// have (moe_out_v2 above 4 bits), or 0 for any admitted format (moe_out).
template <int kBitsX2>
__global__ __launch_bounds__(256, kBitsX2 > 8 ? 3 : (kBitsX2 > 0 ? 4 : 2)) void moe_gemv(Routing routing, int projection, int64_t kp,
                                                int64_t np, const int* table, float* ws,
                                                MoeLayout lay, int64_t in_offset,
                                                int64_t out_offset, int want_bits) {
  constexpr bool kFixed = kBitsX2 > 0;
  // steps of trellis loads in flight: one B block, so the loop body below
  // is one block with no branch around a load (steps is a multiple of 4)
  constexpr int kDepth = 4;
  constexpr int kRows = task_rows(kBitsX2);
  constexpr int kSub = kRows / 8;
  constexpr int kCols = 2 * kRows;
  constexpr int kChunks = kCols / 16;  // 16-byte B chunks per thread per block
  // one 128-input block of B operands: [buf][step][g][column][8 halves]
  // (the epilogue's per-row sums reuse it: kRows x 128 floats)
  __shared__ __attribute__((aligned(16))) _Float16 bop[2][4][4][kCols][8];
  __shared__ int rexp[kRows];
  static_assert(sizeof(bop) >= sizeof(float) * kRows * 128, "row sums fit the B staging");
  float (*red)[128] = reinterpret_cast<float (*)[128]>(&bop[0][0][0][0][0]);

  const int64_t task = blockIdx.y;
  if (task >= table[1]) return;
  // the task, the expert's pointers and geometry are read with vector loads
  // (the table lies in the workspace this kernel writes): uniform() keeps
  // them, and the buffer resources built from them, in scalar registers
  const int4 tk = reinterpret_cast<const int4*>(table + lay.tasks())[task];
  const int expert = vq::uniform(tk.x);
  const int first = vq::uniform(tk.y);
  const int nrows = vq::uniform(tk.z);
  const int nsub = (nrows + 7) >> 3;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = vq::uniform(tid >> 6);
  const int g = lane >> 4;
  const int m = lane & 15;
  const int L = 4 * (m & 7) + g;
  const int* sorted = table + 4;
  const int64_t* ptrs = routing.ptrs + expert * 9 + projection * 3;
  const int64_t* meta_p = routing.meta + expert * 12 + projection * 4;
  const int64_t meta[4] = {vq::uniform(meta_p[0]), vq::uniform(meta_p[1]), vq::uniform(meta_p[2]),
                           vq::uniform(meta_p[3])};
  const uint8_t* trellis = reinterpret_cast<const uint8_t*>(vq::uniform(ptrs[0]));
  const uint16_t* svh = reinterpret_cast<const uint16_t*>(vq::uniform(ptrs[2]));
  const int64_t tiles_n = meta[1] / 16;
  const int bits_x2 = kFixed ? kBitsX2 : int(meta[2]);
  const int codebook = kFixed ? 2 : int(meta[3]);
  // An expert whose geometry or format disagrees with the call (its matrix
  // is not kp x np, or not the layer's rate in a fixed-rate launch, or no
  // admitted format) would be read out of bounds: its rows get NaN instead.
  const bool bad = meta[0] != kp || meta[1] != np ||
                   (kFixed ? (meta[2] != kBitsX2 || meta[3] != 2)
                           : (want_bits > 0 && (meta[2] != want_bits || meta[3] != 2)) ||
                                 !(meta[3] == 1 ? (bits_x2 >= 2 && bits_x2 <= 16 && bits_x2 % 2 == 0)
                                                : (meta[3] == 2 && bits_x2 >= 2 && bits_x2 <= 16 &&
                                                   (bits_x2 % 2 == 0 || bits_x2 <= 7))));
  if (bad) {
    for (int r = wave; r < nrows; r += 4) {
      float* dst = ws + out_offset + int64_t(table[4 + first + r]) * np + 128 * int64_t(blockIdx.x);
      dst[lane] = __builtin_nanf("");
      dst[lane + 64] = __builtin_nanf("");
    }
    return;
  }
  const bool aligned = (reinterpret_cast<uintptr_t>(trellis) & 3) == 0;
  const int tile_bytes = 16 * bits_x2;
  const int64_t row_bytes = tiles_n * tile_bytes;
  // (int: the host keeps the A x kp floats of a region below 2 GiB)
  const int steps = int(kp / 32);
  const int kblocks = int(kp / 128);
  // the wavefront's two tiles of tile row 0
  const uint8_t* chunk = trellis + 2 * (4 * int64_t(blockIdx.x) + wave) * tile_bytes;

  // B-operand staging of a block for the first kNs 8-row sub-blocks (kc =
  // 16 kNs columns: rows 0 .. 8 kNs - 1, high and low parts): chunk c = tid +
  // 256 i (i < kc / 16) is 16 bytes (step, g, column) = (c / (4 kc), c / kc
  // % 4, c % kc), kept at that column of the kCols-wide LDS layout; columns
  // of rows past the task read its last row again (their MFMA columns are
  // never used).  Tasks of fewer rows stage (and read) fewer columns.
  //    The B operands are read through a buffer over the input region
  //    (32-bit byte offsets: the region is A x kp floats, checked on the host).
  const __amdgpu_buffer_rsrc_t st_buf = __builtin_amdgcn_make_buffer_rsrc(
      ws + in_offset, 0, int(lay.assignments * kp * 4), 0x00020000);
  auto stage_offsets = [&](auto ns_tag, uint32_t (&off)[kChunks]) {
    constexpr int kc = 16 * decltype(ns_tag)::value;
#pragma unroll
    for (int i = 0; i < kc / 16; ++i) {
      const int c = tid + 256 * i;
      const int col = c % kc;
      const int64_t a = sorted[first + min(col >> 1, nrows - 1)];
      off[i] = uint32_t((a * 2 * kp + (col & 1) * kp + (c / (4 * kc)) * 32 + (c / kc % 4) * 8) * 2);
    }
  };
  auto stage = [&](auto ns_tag, const uint32_t (&off)[kChunks], int kb, u32x4_t (&v)[kChunks]) {
    constexpr int kc = 16 * decltype(ns_tag)::value;
#pragma unroll
    for (int i = 0; i < kc / 16; ++i) {
      v[i] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(st_buf, int(off[i]),
                                                                               int(kb * 256), 0));
    }
  };
  auto put = [&](auto ns_tag, int buf, const u32x4_t (&v)[kChunks]) {
    constexpr int kc = 16 * decltype(ns_tag)::value;
#pragma unroll
    for (int i = 0; i < kc / 16; ++i) {
      const int c = tid + 256 * i;
      *reinterpret_cast<u32x4_t*>(&bop[buf][c / (4 * kc)][c / kc % 4][c % kc][0]) = v[i];
    }
  };
  if (tid < kRows) {
    const int* exps = reinterpret_cast<const int*>(ws + lay.ints()) + lay.exps();
    rexp[tid] = exps[int64_t(sorted[first + min(tid, nrows - 1)]) * (lay.kmax() / 128)];
  }

  // trellis ring (fixed rate up to 4 bits per weight: one coalesced dword
  // per lane per tile row, words gathered with ds_bpermute; wider fixed
  // rates: each lane loads its own window words; run-time rate: decoded
  // from the tile directly)
  constexpr bool kGather = kFixed && kBitsX2 <= 8;
  constexpr int kWords = LaneLoad<kFixed ? kBitsX2 : 8>::kWords;
  constexpr int kRaw = kGather ? 1 : kWords;
  const int raw_off = lane < 8 * bits_x2 ? 4 * lane : 0;
  int widx[kWords];
  lane_word_index<kFixed ? kBitsX2 : 8>(L, widx);
  int src[kWords];
#pragma unroll
  for (int i = 0; i < kWords; ++i) src[i] = 4 * ((m >> 3) * 4 * kBitsX2 + widx[i]);
  // Buffer loads over the wavefront's tile pair of every tile row (32-bit
  // offsets; the host keeps an expert's matrix below 2 GiB): vmcnt only, so
  // the LDS waits of each step (ds_bpermute) do not also wait for the
  // trellis loads in flight, as flat loads would make them.
  const __amdgpu_buffer_rsrc_t tr_buf = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(chunk), 0, int((steps * 2 - 1) * row_bytes + 2 * tile_bytes), 0x00020000);
  uint32_t raw[kDepth][2][kRaw];
  // (the alignment is a compile-time branch of the stream below: with a
  // run-time branch in the loop the compiler, unsure of the loads in flight
  // where the paths meet, waits for all of them before each use)
  auto load_word = [&](auto aligned_tag, int offset, int row) -> uint32_t {
    if constexpr (decltype(aligned_tag)::value) {
      return __builtin_amdgcn_raw_buffer_load_b32(tr_buf, offset, row, 0);
    } else {
      return uint32_t(__builtin_amdgcn_raw_buffer_load_b16(tr_buf, offset, row, 0)) |
             (uint32_t(__builtin_amdgcn_raw_buffer_load_b16(tr_buf, offset + 2, row, 0)) << 16);
    }
  };
  auto load_step = [&](auto aligned_tag, int slot, int s) {
    if constexpr (kFixed) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int row = int((2 * s + h) * row_bytes);
        if constexpr (kGather) {
          raw[slot][h][0] = load_word(aligned_tag, raw_off, row);
        } else {
#pragma unroll
          for (int k = 0; k < kRaw; ++k) {
            const int offset = (m >> 3) * tile_bytes + 4 * widx[k];
            raw[slot][h][k] = load_word(aligned_tag, offset, row);
          }
        }
      }
    }
  };

  f32x4_t acc1[kSub], acc2[kSub];
#pragma unroll
  for (int sb = 0; sb < kSub; ++sb) acc1[sb] = acc2[sb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  auto stream = [&](auto aligned_tag, auto ns_tag) {
    constexpr int kNs = decltype(ns_tag)::value;  // sub-blocks staged and read
    uint32_t st_off[kChunks];
    stage_offsets(ns_tag, st_off);
    // prologue: block 0's B operands, the first kDepth steps of trellis
    u32x4_t sv[kChunks];
    stage(ns_tag, st_off, 0, sv);
  #pragma unroll
    for (int i = 0; i < kDepth; ++i) load_step(aligned_tag, i, min(i, steps - 1));
    put(ns_tag, 0, sv);
    __syncthreads();

    // one 128-input block (4 steps) per iteration, branch-free around the
    // loads: the last block re-stages itself into the buffer no step reads
    // again, and the trellis loads past the end reload the last step
    for (int s0 = 0; s0 < steps; s0 += kDepth) {
  #pragma unroll
      for (int i = 0; i < kDepth; ++i) {
        const int s = s0 + i;
        {
          const int kb = s >> 2;
          const int buf = int(kb & 1);
          if (i == 0) {
            progress_priority(s, steps);
            stage(ns_tag, st_off, min(kb + 1, kblocks - 1), sv);
          }
          uint32_t q0[4], q1[4];
          if constexpr (kFixed) {
            uint32_t w0[kWords], w1[kWords];
  #pragma unroll
            for (int k = 0; k < kWords; ++k) {
              if constexpr (kGather) {
                w0[k] = uint32_t(__builtin_amdgcn_ds_bpermute(src[k], int(raw[i][0][0])));
                w1[k] = uint32_t(__builtin_amdgcn_ds_bpermute(src[k], int(raw[i][1][0])));
              } else {
                w0[k] = raw[i][0][k];
                w1[k] = raw[i][1][k];
              }
            }
            load_step(aligned_tag, i, min(s + kDepth, steps - 1));
            decode_words<kBitsX2, 2>(L, w0, q0);
            decode_words<kBitsX2, 2>(L, w1, q1);
          } else {
            const uint8_t* t0 = chunk + (2 * s) * row_bytes + (m >> 3) * tile_bytes;
            decode_runtime(t0, aligned, bits_x2, codebook, L, q0);
            decode_runtime(t0 + row_bytes, aligned, bits_x2, codebook, L, q1);
          }
          const u32x4_t a1 = {q0[0], q0[1], q1[0], q1[1]};
          const u32x4_t a2 = {q0[2], q0[3], q1[2], q1[3]};
          // the staged sub-blocks' B operands in one batch of LDS reads (the
          // staged columns past the task hold its last row: valid data),
          // then the MFMAs of the task's sub-blocks
          half8_t b[kSub];
  #pragma unroll
          for (int sb = 0; sb < kNs; ++sb) b[sb] = *reinterpret_cast<const half8_t*>(&bop[buf][s & 3][g][16 * sb + m][0]);
  #pragma unroll
          for (int sb = 0; sb < kNs; ++sb) {
            if (sb < nsub) {
              acc1[sb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, a1), b[sb], acc1[sb], 0, 0, 0);
              acc2[sb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, a2), b[sb], acc2[sb], 0, 0, 0);
            }
          }
          if (i == 3) {
            put(ns_tag, buf ^ 1, sv);
            __syncthreads();
          }
        }
      }
    }
  };
  // the loop for the fewest staged sub-blocks (1, 2 or kSub) that hold the
  // task's rows
  auto run = [&](auto aligned_tag) {
    if constexpr (kSub >= 4) {
      if (nsub <= 1) {
        stream(aligned_tag, std::integral_constant<int, 1>{});
      } else if (nsub <= 2) {
        stream(aligned_tag, std::integral_constant<int, 2>{});
      } else {
        stream(aligned_tag, std::integral_constant<int, kSub>{});
      }
    } else {
      stream(aligned_tag, std::integral_constant<int, kSub>{});
    }
  };
  if constexpr (kFixed) {
    if (aligned) {
      run(std::true_type{});
    } else {
      run(std::false_type{});
    }
  } else {
    run(std::true_type{});  // the run-time decode reads the tiles itself
  }

  // epilogue: high + low parts (adjacent lanes) unscaled per row, the rows'
  // 128 columns through LDS, then H128 and svh per row
#pragma unroll
  for (int sb = 0; sb < kSub; ++sb) {
    if (sb < nsub) {
      const int r = 8 * sb + (m >> 1);
      const int e = rexp[r];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float v1 = ldexpf(acc1[sb][k] + vq::xor_lanes<1>(acc1[sb][k], lane), -e);
        const float v2 = ldexpf(acc2[sb][k] + vq::xor_lanes<1>(acc2[sb][k], lane), -e);
        const int row = 4 * g + k;
        const int col = 32 * wave + (row & 7) + 16 * (row >> 3);
        if ((m & 1) == 0 && r < nrows) {
          red[r][col] = v1;
          red[r][col + 8] = v2;
        }
      }
    }
  }
  __syncthreads();
  // The rows' assignments and the block's svh are loaded before the first
  // output store: loads and stores share one in-order counter, so a load
  // waited for after a store also waits for the store to complete.
  const int64_t c0 = 128 * int64_t(blockIdx.x) + lane;
  const float svh0 = vq::f16_to_f32(svh[c0]);
  const float svh1 = vq::f16_to_f32(svh[c0 + 64]);
  int row_a[kRows / 4];
#pragma unroll
  for (int i = 0; i < kRows / 4; ++i) {
    const int r = wave + 4 * i;
    row_a[i] = r < nrows ? sorted[first + r] : 0;
  }
#pragma unroll
  for (int i = 0; i < kRows / 4; ++i) {
    const int r = wave + 4 * i;
    if (r < nrows) {
      float v0 = red[r][lane];
      float v1 = red[r][lane + 64];
      vq::h128_wave(v0, v1, lane);
      float* dst = ws + out_offset + int64_t(row_a[i]) * np;
      dst[c0] = v0 * svh0;
      dst[c0 + 64] = v1 * svh1;
    }
  }
}

// ---- 5. combine ------------------------------------------------------------------

// One workgroup per (token, 1024 columns): the token's routes (whether
// local, the row of the down output, the routing weight) are read once into
// LDS; each thread then sums its four columns over the local routes in route
// order, one FMA each (the reference's order), with the 16-byte loads of
// every route in flight together (a route that is not local loads a valid
// row and is not added: its own row may hold anything).
constexpr int kCombineCols = 4 * 256;
__global__ __launch_bounds__(256) void moe_combine(Routing routing, const float* down,
                                                   const float* weights, int64_t rows,
                                                   int64_t hidden, int64_t hpad, void* out,
                                                   int out_dtype, bool any_local) {
  constexpr int kRoutes = 32;  // routes staged per round
  __shared__ int64_t route_row[kRoutes];
  __shared__ float route_w[kRoutes];
  __shared__ int route_ok[kRoutes];
  // columns c .. c + 3 (hpad is a multiple of 128: a row's 16-byte loads stay in it)
  const int64_t c = int64_t(blockIdx.x) * kCombineCols + 4 * threadIdx.x;
  const bool mine = c < hidden;
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
    float sum[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (any_local) {
      for (int64_t k0 = 0; k0 < routing.topk; k0 += kRoutes) {
        const int n = int(routing.topk - k0 < kRoutes ? routing.topk - k0 : kRoutes);
        if (int(threadIdx.x) < n) {
          const int64_t a = r * routing.topk + k0 + threadIdx.x;
          const bool ok = local_expert(routing, a) >= 0;
          route_ok[threadIdx.x] = ok;
          route_row[threadIdx.x] = ok ? a * hpad : 0;
          route_w[threadIdx.x] = ok ? weights[a] : 0.0f;
        }
        __syncthreads();
        if (mine) {
#pragma unroll 8
          for (int k = 0; k < n; ++k) {
            const f32x4_t v = *reinterpret_cast<const f32x4_t*>(down + route_row[k] + c);
            if (route_ok[k]) {
#pragma unroll
              for (int i = 0; i < 4; ++i) sum[i] = fmaf(v[i], route_w[k], sum[i]);
            }
          }
        }
        __syncthreads();
      }
    }
    if (mine) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (c + i < hidden) vq::store_act(out, out_dtype, r * hidden + c + i, sum[i]);
      }
    }
  }
}

int64_t padded(int64_t n) { return (n + 127) / 128 * 128; }

}  // namespace
}  // namespace exl3

extern "C" int64_t exl3_moe_workspace_size(int64_t max_rows, int64_t hidden_size,
                                           int64_t intermediate_size, int64_t topk,
                                           int64_t local_experts) {
  if (max_rows < 0 || topk < 0 || local_experts < 0) {
    vq::fail("EXL3 rows/topk/local_experts must be nonnegative");
    return -1;
  }
  if (hidden_size <= 0 || intermediate_size <= 0 || hidden_size > INT_MAX - 127 ||
      intermediate_size > INT_MAX - 127) {
    vq::fail("EXL3 logical dimensions must be positive and fit int32 padding");
    return -1;
  }
  if (local_experts == 0) return 0;
  const exl3::MoeLayout lay{exl3::padded(hidden_size), exl3::padded(intermediate_size),
                            max_rows * topk};
  return lay.total();
}

extern "C" int exl3_moe_out(const void* x, int x_dtype, int64_t rows, int64_t hidden,
                            const void* topk_ids, int ids64, const float* topk_weights,
                            int64_t topk, const int64_t* packed_ptrs, const int64_t* packed_meta,
                            int64_t local_experts, const void* expert_map, int map64,
                            int64_t global_experts, int64_t intermediate_size, int64_t bits_x2,
                            void* out, int out_dtype, float* workspace, int64_t workspace_numel,
                            float swiglu_limit, void* stream) {
  using namespace vq;
  if (x_dtype != kBF16 && x_dtype != kFP16) return fail("x has incorrect dtype");
  if (out_dtype != x_dtype) return fail("out has incorrect dtype");
  if (!(swiglu_limit >= 0.0f) || swiglu_limit > 3.4e38f) {
    return fail("EXL3 swiglu_limit must be finite and nonnegative");
  }
  if (rows < 0 || topk < 0 || hidden <= 0) return fail("EXL3 MoE row/topk/output geometry mismatch");
  if (local_experts > exl3::kMaxRouteExperts) return fail("EXL3 MoE has too many local experts");
  if (intermediate_size <= 0) return fail("EXL3 logical dimensions must be positive and fit int32 padding");
  if (bits_x2 != 0 && !exl3::known_format(bits_x2, 2)) {
    return fail("EXL3 MoE v2 supports mul1 rates only");
  }
  const int64_t assignments = rows * topk;
  if (assignments > INT_MAX) return fail("EXL3 MoE has too many routed assignments");
  // the expert GEMV reads its B operands and each expert matrix through
  // 32-bit byte offsets
  if (assignments * exl3::padded(std::max(hidden, intermediate_size)) * 4 > INT_MAX) {
    return fail("EXL3 MoE: rows * topk * hidden too large for one call (split the rows)");
  }
  if (exl3::padded(hidden) * exl3::padded(intermediate_size) * 2 > INT_MAX) {
    return fail("EXL3 MoE: an expert matrix must stay below 2 GiB");
  }
  const int64_t need = exl3_moe_workspace_size(rows, hidden, intermediate_size, topk, local_experts);
  if (need < 0) return kInvalidArgument;
  if (workspace_numel < need) return fail("EXL3 MoE workspace is too small");
  if ((reinterpret_cast<uintptr_t>(workspace) & 15) != 0) {
    return fail("EXL3 MoE workspace must be 16-byte aligned");
  }
  if (rows == 0) return kOk;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const exl3::MoeLayout lay{exl3::padded(hidden), exl3::padded(intermediate_size), assignments};
  exl3::Routing routing{topk_ids, expert_map, packed_ptrs, packed_meta, global_experts,
                        local_experts, topk, ids64 != 0, map64 != 0};
  const bool any = local_experts > 0 && assignments > 0;
  // every check before the first launch
  const int fixed = exl3::fixed_rate(bits_x2);
  const int task_rows = exl3::task_rows(fixed);
  const int64_t max_tasks =
      std::min<int64_t>(assignments, (assignments + task_rows - 1) / task_rows + local_experts);
  // Experts with enough rows run on the tile GEMM (a call with one rate for
  // the layer, any rate).  Tile tasks = sum over those experts of
  // ceil(rows / 128), at most
  // assignments / tile_rows for a threshold up to 64 rows; when that bound
  // is under the workgroup minimum (enough tasks for kMinTileBlocks
  // workgroups in the narrower projection) no call can have tile tasks and
  // the tile launches are left out.
  const int tile_rows = exl3::tile_min_rows();
  const int64_t narrow = std::min(lay.hpad, lay.ipad);
  const int min_tile_tasks = exl3::tile_min_tasks(
      int((exl3::kMinTileBlocks * exl3::kTileCols + narrow - 1) / narrow));
  int64_t max_tiles = 0;
  const int tile_bits = bits_x2 > 0 && exl3::tile_rate(bits_x2) ? int(bits_x2) : 0;
  const bool tile_lo = !exl3::tile_fp16_only();
  if (tile_bits > 0 && assignments >= tile_rows) {
    max_tiles = tile_rows <= 64 ? assignments / tile_rows
                                : assignments / exl3::kTileRows + assignments / tile_rows + 1;
    max_tiles = std::min<int64_t>(max_tiles, assignments);
    if (max_tiles < min_tile_tasks) max_tiles = 0;
  }
  const bool tiles = max_tiles > 0;
  if (any && (max_tasks > 65535 || max_tiles > 65535)) {
    return fail("EXL3 MoE has too many routed assignments");
  }
  if (any) {
    int* table = reinterpret_cast<int*>(workspace + lay.ints());
    const size_t route_lds = size_t(4 * local_experts + 2) * sizeof(int);
    int* row_expert = table + lay.row_experts();
    if (assignments >= exl3::kRouteSplitMin) {
      // packed slots, then the parts' histograms, in the gate-result region
      // (A * ipad floats, ipad >= 128: room for A + parts * experts ints)
      const int64_t parts = (assignments + exl3::kRoutePart - 1) / exl3::kRoutePart;
      int* packed = reinterpret_cast<int*>(workspace + lay.gate());
      int* hist = packed + (assignments + 3) / 4 * 4;
      hipLaunchKernelGGL(exl3::moe_route_count, dim3(unsigned(parts)), dim3(exl3::kRoutePartThreads),
                         size_t(local_experts) * sizeof(int), s, routing, assignments, packed, hist);
      if (int rc = check_launch("exl3 moe_route_count")) return rc;
      hipLaunchKernelGGL(exl3::moe_route, dim3(1), dim3(exl3::kRouteThreads), route_lds, s, routing,
                         assignments, task_rows, tiles ? tile_rows : 0, min_tile_tasks, table, row_expert,
                         hist, int(parts));
      if (int rc = check_launch("exl3 moe_route")) return rc;
      hipLaunchKernelGGL(exl3::moe_route_fill, dim3(unsigned(parts)), dim3(exl3::kRoutePartThreads), 0, s,
                         assignments, int(local_experts), packed, hist, table + 4, row_expert);
      if (int rc = check_launch("exl3 moe_route_fill")) return rc;
    } else {
      hipLaunchKernelGGL(exl3::moe_route, dim3(1), dim3(exl3::kRouteThreads), route_lds, s, routing,
                         assignments, task_rows, tiles ? tile_rows : 0, min_tile_tasks, table, row_expert,
                         nullptr, 0);
      if (int rc = check_launch("exl3 moe_route")) return rc;
    }
    auto tile = [&](int projection, int64_t kp, int64_t np, int64_t in_off, int64_t out_off) {
      exl3::TileArgs t{};
      t.act = reinterpret_cast<const uint8_t*>(workspace + in_off);
      t.act_row_bytes = 4 * kp;
      t.act_rows = assignments;
      t.row_exp = reinterpret_cast<const int*>(workspace + lay.ints()) + lay.exps();
      t.exp_stride = lay.kmax() / 128;
      t.kp = kp;
      t.np = np;
      t.table = table;
      t.task_offset = lay.tasks();
      t.ptrs = packed_ptrs;
      t.meta = packed_meta;
      t.projection = projection;
      t.moe_out = workspace + out_off;
      t.col_tiles = int((np + exl3::kTileCols - 1) / exl3::kTileCols);
      // per XCD: up to ceil(max_tiles / 8) tasks in groups of task_group,
      // each group task_group x col_tiles workgroups
      const int64_t per_xcd = (max_tiles + 7) / 8;
      t.task_group = int(std::min<int64_t>(8, per_xcd));
      const int64_t groups = (per_xcd + t.task_group - 1) / t.task_group;
      const dim3 grid{unsigned(8 * groups * t.task_group * t.col_tiles), 1u, 1u};
      return exl3::launch_tile_gemm(tile_bits, 2, true, tile_lo, t, grid, s);
    };
    const int want_bits = fixed == 0 ? int(bits_x2) : 0;
    auto gemv = [&](int projection, int64_t kp, int64_t np, int64_t in_off, int64_t out_off) {
      const dim3 grid(unsigned(np / 128), unsigned(max_tasks));
      switch (fixed) {
#define VQ_MOE(B) case B: hipLaunchKernelGGL(exl3::moe_gemv<B>, grid, dim3(256), 0, s, routing, projection, kp, np, table, workspace, lay, in_off, out_off, 0); break;
        VQ_MOE(2) VQ_MOE(3) VQ_MOE(4) VQ_MOE(5) VQ_MOE(6) VQ_MOE(7) VQ_MOE(8)
        VQ_MOE(10) VQ_MOE(12) VQ_MOE(14) VQ_MOE(16)
#undef VQ_MOE
        default:
          hipLaunchKernelGGL(exl3::moe_gemv<0>, grid, dim3(256), 0, s, routing, projection, kp, np,
                             table, workspace, lay, in_off, out_off, want_bits);
      }
      return check_launch("exl3 moe_gemv");
    };
    // moe_form: calls of kFormRowMin rows or more whose rows have few
    // enough 4-block groups one wavefront a row (four rows a workgroup),
    // others one workgroup a row (fewer rows: each row's groups over four
    // wavefronts finish sooner); the register cache sized to the groups a
    // wavefront forms
    auto form = [&](bool activate, int projection) {
      const int64_t groups = ((activate ? lay.ipad : lay.hpad) / 128 + 3) / 4;
      const int64_t per_wave = (groups + 3) / 4;
      const dim3 grid{unsigned(assignments), 1u, 1u};
      const dim3 row_grid{unsigned((assignments + 3) / 4), 1u, 1u};
#define VQ_FORM(A, C, W)                                                                            \
  hipLaunchKernelGGL((exl3::moe_form<A, C, W>), W ? row_grid : grid, dim3(256), 0, s, routing, x,   \
                     x_dtype, hidden, intermediate_size, projection, table, workspace, lay,         \
                     swiglu_limit, tile_lo)
      if (groups <= (activate ? exl3::kFormRowGroupsActivate : exl3::kFormRowGroups) &&
          assignments >= exl3::kFormRowMin) {
        switch (int(groups) + (activate ? 8 : 0)) {
          case 1: VQ_FORM(false, 1, true); break;
          case 2: VQ_FORM(false, 2, true); break;
          case 3: VQ_FORM(false, 3, true); break;
          case 4: VQ_FORM(false, 4, true); break;
          case 5: VQ_FORM(false, 5, true); break;
          case 6: VQ_FORM(false, 6, true); break;
          case 9: VQ_FORM(true, 1, true); break;
          default: VQ_FORM(true, 2, true); break;
        }
      } else if (activate) {
        if (per_wave <= 1) VQ_FORM(true, 1, false); else if (per_wave <= 2) VQ_FORM(true, 2, false); else VQ_FORM(true, 4, false);
      } else {
        if (per_wave <= 1) VQ_FORM(false, 1, false); else if (per_wave <= 2) VQ_FORM(false, 2, false); else VQ_FORM(false, 4, false);
      }
#undef VQ_FORM
      return check_launch("exl3 moe_form");
    };
    for (int p = 0; p < 2; ++p) {
      if (int rc = form(false, p)) return rc;
      const int64_t out_off = p == 0 ? lay.gate() : lay.up();
      if (int rc = gemv(p, lay.hpad, lay.ipad, lay.input(), out_off)) return rc;
      if (tiles) {
        if (int rc = tile(p, lay.hpad, lay.ipad, lay.input(), out_off)) return rc;
      }
    }
    if (int rc = form(true, 2)) return rc;
    if (int rc = gemv(2, lay.ipad, lay.hpad, lay.act(), lay.input())) return rc;
    if (tiles) {
      if (int rc = tile(2, lay.ipad, lay.hpad, lay.act(), lay.input())) return rc;
    }
  }
  const dim3 combine_grid(unsigned((hidden + exl3::kCombineCols - 1) / exl3::kCombineCols),
                          unsigned(std::min<int64_t>(rows, 65535)));
  hipLaunchKernelGGL(exl3::moe_combine, combine_grid, dim3(256), 0, s,
                     routing, workspace + lay.input(), topk_weights, rows, hidden, lay.hpad, out,
                     out_dtype, any);
  return check_launch("exl3 moe_combine");
}

extern "C" int exl3_set_moe_tile_rows(int rows) {
  if (rows < 0) return vq::fail("EXL3 MoE tile threshold must be 0 (automatic) or positive");
  exl3::g_tile_rows_override.store(rows);
  return vq::kOk;
}
