// EXL3 dense linear for gfx950, host side: the C-ABI entry points
// exl3_linear_out / exl3_decode / exl3_linear_workspace_size, the small-M
// launch plan (K splits, column ranges, arrival-counter slots), and the
// separate output kernel of the small-M path.  The kernels are in
// exl3_gemv.h (instantiated by exl3_gemv_part.hip) and exl3_gemm.hip.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <climits>
#include <map>
#include <mutex>
#include <string>
#include <tuple>
#include <utility>

#include "../../include/vllm_mi355x.h"
#include "common.h"
#include "exl3_codec.h"
#include "exl3_gemv.h"
#include "exl3_internal.h"

namespace exl3 {

// The arrival-counter pool of the fused finish (see exl3_gemv.h).
__device__ uint32_t g_gemv_counters[kCounterRanges * kCounterSlots * kCounterStride];
// Launches that found no counter range (they used the separate finish).
std::atomic<long long> g_counter_fallbacks{0};

namespace {

// Unfused finish: one wavefront per (row, 128-column block).
__global__ __launch_bounds__(kThreads) void gemv_output(const float* __restrict__ partial, int splits,
                                                         int rows, int64_t np,
                                                         const uint16_t* __restrict__ svh,
                                                         int64_t logical_out, int64_t out_stride,
                                                         void* out, int out_dtype) {
  const int lane = threadIdx.x & 63;
  const int64_t blocks = np / 128;
  const int64_t task = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (task >= rows * blocks) return;
  const int64_t r = task / blocks;
  finish_row_block<false>(partial, splits, rows, np, r, (task - r * blocks) * 128, svh, logical_out,
                          out_stride, out, out_dtype, lane);
}

}  // namespace

int launch_output(const float* partial, int splits, int rows, int64_t np, const uint16_t* svh,
                  int64_t logical_out, int64_t out_stride, void* out, int out_dtype, hipStream_t stream) {
  const int64_t tasks = int64_t(rows) * (np / 128);
  hipLaunchKernelGGL(gemv_output, dim3(unsigned((tasks + 3) / 4)), dim3(kThreads), 0, stream, partial,
                     splits, rows, np, svh, logical_out, out_stride, out, out_dtype);
  return vq::check_launch("exl3 gemv_output");
}

namespace {

// Reaches the format's instantiations in their part of the build.
int dispatch(int64_t bits_x2, int64_t codebook, bool aligned, int load, const GemvArgs* gemv,
             int gemv_blocks, int gemv_groups, dim3 grid, hipStream_t stream,
             const uint8_t* trellis, int64_t tiles_k, int64_t tiles_n, uint16_t* decoded) {
  const int index = format_index(int(bits_x2), int(codebook));
  if (index < 0 || !known_format(bits_x2, codebook)) {
    return vq::fail("Unsupported EXL3 rate/codebook combination");
  }
  switch (index % kGemvParts) {
#define VQ_PART(P)                                                                                  \
  case P:                                                                                          \
    return gemv_launch_part<P>(bits_x2, codebook, aligned, load, gemv, gemv_blocks, gemv_groups, grid, \
                               stream, trellis, tiles_k, tiles_n, decoded);
    VQ_PART(0) VQ_PART(1) VQ_PART(2) VQ_PART(3) VQ_PART(4) VQ_PART(5) VQ_PART(6) VQ_PART(7)
#undef VQ_PART
  }
  return vq::fail("Unsupported EXL3 rate/codebook combination");
}

int check_padded(int64_t n) {
  // (the kernels address a row of x, suh or svh in bytes with 32-bit offsets)
  if (n <= 0 || n % 128 != 0 || n > INT_MAX / 4) {
    return vq::fail("EXL3 padded dimensions must be positive H128 multiples fitting int32");
  }
  return vq::kOk;
}

}  // namespace

// Arrival counters of a fused-finish launch over `blocks` column blocks:
// the pool's device address and the launch's first slot, or a null pool (the
// launch then uses the separate output kernel).  One range of kCounterSlots
// slots per (device, stream) for eager launches and one per (device, stream)
// for the launches recorded while that stream captures a graph: eager
// launches on one stream run in order and share its range; every graph
// captured on one stream shares that stream's capture range, so replays of
// such graphs must not overlap each other (replays on one stream, the way
// graphs are replayed, never do); a graph never shares a range with eager
// work, so a graph replayed on another stream while its capture stream runs
// eager launches cannot collide with them.  Ranges are kept for the life of
// the process (a graph may be replayed at any time); any number of captures
// reuse their stream's range.  Fallbacks (more streams than ranges) are
// counted (exl3_counter_fallbacks).
CounterSlots counter_slots(hipStream_t stream, int64_t blocks) {
  static std::mutex mutex;
  static std::map<std::tuple<int, hipStream_t, bool>, int> ranges;
  static std::map<int, int> used;
  static std::map<int, uint32_t*> pools;
  const CounterSlots none{nullptr, -1};
  if (blocks > kCounterSlots) {
    g_counter_fallbacks.fetch_add(1);
    return none;
  }
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) {
    (void)hipGetLastError();
    return none;
  }
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  unsigned long long capture = 0;
  if (hipStreamGetCaptureInfo(stream, &status, &capture) != hipSuccess) {
    (void)hipGetLastError();
    return none;
  }
  const bool capturing = status != hipStreamCaptureStatusNone;
  std::lock_guard<std::mutex> lock(mutex);
  uint32_t*& pool = pools[device];
  if (!pool) {
    // each device holds its own copy of the array, at its own address
    void* address = nullptr;
    if (hipGetSymbolAddress(&address, HIP_SYMBOL(g_gemv_counters)) != hipSuccess || !address) {
      (void)hipGetLastError();
      return none;
    }
    pool = static_cast<uint32_t*>(address);
  }
  const auto key = std::make_tuple(device, stream, capturing);
  const auto it = ranges.find(key);
  if (it != ranges.end()) return {pool, it->second};
  int& n = used[device];
  if (n >= kCounterRanges) {
    g_counter_fallbacks.fetch_add(1);
    return none;
  }
  const int base = n++ * kCounterSlots;
  ranges[key] = base;
  return {pool, base};
}

namespace {

// 128-input blocks per workgroup chosen automatically, always a divisor of
// padded_in / 128: the fewest (1, 2, 4 or 8) that keep the grid within ~7
// wavefronts per SIMD (all resident at once: one round, no second-round
// start-up) and the K splits within 32 (the fused finish reads every split's
// partial sums).
int auto_blocks(int64_t padded_in, int64_t padded_out) {
  const int64_t k_blocks = padded_in / 128;
  const int64_t col_waves = padded_out / 128 * 4;
  int best = 1;
  for (int b : {1, 2, 4, 8}) {
    if (k_blocks % b != 0) continue;
    best = b;
    if (col_waves * (k_blocks / b) <= 7168 && k_blocks / b <= 32) break;
  }
  return best;
}

// Test and tuning overrides (exl3_set_gemv_blocks / _groups / _finish).  A
// forced block count that does not divide the input blocks falls back to the
// automatic choice.
std::atomic<int> g_blocks_override{0};
std::atomic<int> g_groups_override{0};
// -1 automatic (fused while counter slots are free), 0 always the separate
// output kernel, 1 as -1.
std::atomic<int> g_finish_mode{-1};

// How a small-M call is launched.
struct GemvPlan {
  int load;        // kLoadLds / kLoadDword / kLoadHalf, from the trellis alignment
  int blocks;      // 128-input blocks per group
  int groups;      // groups of 4 wavefronts per workgroup (1 or 4)
  int64_t splits;  // K splits: padded_in / 128 / (blocks * groups)
};

GemvPlan plan_gemv(uintptr_t trellis, int64_t bits_x2, int64_t padded_in, int64_t padded_out,
                   bool automatic) {
  GemvPlan p;
  p.load = (trellis & 15) == 0 ? kLoadLds : ((trellis & 3) == 0 ? kLoadDword : kLoadHalf);
  const int64_t k_blocks = padded_in / 128;
  p.blocks = auto_blocks(padded_in, padded_out);
  p.groups = 1;
  if (!automatic) {
    const int forced = g_blocks_override.load();
    if (forced > 0 && k_blocks % forced == 0) p.blocks = forced;
    // groups of 4: LDS stream only, whole 4 * blocks ranges, two ring loads
    // per group range (can_group)
    if (g_groups_override.load() == 4 && p.load == kLoadLds && p.blocks <= 4 &&
        k_blocks % (4 * p.blocks) == 0 && can_group(bits_x2, p.blocks)) {
      p.groups = 4;
    }
  }
  p.splits = k_blocks / (p.blocks * p.groups);
  return p;
}

// FP32 elements of the small-M path's K-split partials for `rows` (<= 8) rows
// of `cols` columns under a plan.
int64_t partial_elements(const GemvPlan& p, int64_t rows, int64_t cols) { return p.splits * rows * cols; }

}  // namespace
}  // namespace exl3

extern "C" int64_t exl3_linear_workspace_size(int64_t max_rows, int64_t padded_in,
                                              int64_t padded_out) {
  if (max_rows < 0) {
    vq::fail("EXL3 max_rows must be nonnegative");
    return -1;
  }
  if (exl3::check_padded(padded_in) != vq::kOk || exl3::check_padded(padded_out) != vq::kOk) return -1;
  // The two paths never run in one call, so the larger need is enough.
  // Small-M (up to 32 rows, in chunks of 8): the K-split partials at the
  // automatic split count (a call whose plan needs more runs in column
  // ranges that fit).  Large-M: the FP16 high / low activations (rows *
  // padded_in floats) and one row exponent per row.
  const int64_t small_rows = std::min<int64_t>(max_rows, exl3::kMaxGemvRows);
  const exl3::GemvPlan plan = exl3::plan_gemv(0, 8, padded_in, padded_out, true);
  const int64_t small = exl3::partial_elements(plan, small_rows, padded_out);
  const int64_t large = max_rows > exl3::kGemvChunkedRows ? max_rows * (padded_in + 1) : 0;
  return std::max(small, large);
}

extern "C" int exl3_linear_prefill_rows(void) { return exl3::kGemvChunkedRows; }

extern "C" int exl3_decode(const void* trellis, int64_t tiles_k, int64_t tiles_n,
                           int64_t trellis_words, int64_t bits_x2, int64_t codebook, void* out,
                           void* stream) {
  if (!trellis || !out) return vq::fail("EXL3 decode needs trellis and out buffers");
  if (trellis_words != 8 * bits_x2) return vq::fail("EXL3 packed word stride mismatch");
  if (tiles_k <= 0 || tiles_n <= 0) return vq::fail("EXL3 decode needs a nonempty trellis");
  if (!exl3::known_format(bits_x2, codebook)) {
    return vq::fail("Unsupported EXL3 rate/codebook combination");
  }
  const bool aligned = (reinterpret_cast<uintptr_t>(trellis) & 3) == 0;
  return exl3::dispatch(bits_x2, codebook, aligned, 0, nullptr, 0, 1, dim3(),
                        static_cast<hipStream_t>(stream), static_cast<const uint8_t*>(trellis),
                        tiles_k, tiles_n, static_cast<uint16_t*>(out));
}

namespace exl3 {
namespace {

// Checks of exl3_linear_out in the reference's order and wording
// (csrc/exl3/dense.cu:85-113), shared with the entry point that brings its
// own scratch.  `workspace_numel` < 0: no workspace argument.
int check_linear(const void* x, int x_dtype, int64_t rows, int64_t x_cols, const void* trellis,
                 int64_t tiles_k, int64_t tiles_n, int64_t trellis_words, const void* suh,
                 int64_t suh_numel, const void* svh, int64_t svh_numel, int64_t bits_x2,
                 int64_t codebook, int64_t logical_in, int64_t logical_out, const void* out,
                 int out_dtype, int64_t out_rows, int64_t out_cols, const void* workspace,
                 int64_t workspace_numel) {
  using namespace vq;
  if (x_dtype != kBF16 && x_dtype != kFP16) return fail("x has incorrect dtype");
  if (out_dtype != kBF16 && out_dtype != kFP16 && out_dtype != kFP32) {
    return fail("EXL3 linear out must be BF16, FP16 or FP32");
  }
  if (trellis_words != 8 * bits_x2) return fail("EXL3 packed word stride mismatch");
  const int64_t padded_in = tiles_k * 16;
  const int64_t padded_out = tiles_n * 16;
  if (int rc = check_padded(padded_in)) return rc;
  if (int rc = check_padded(padded_out)) return rc;
  if (!(logical_in > 0 && logical_in <= padded_in && logical_out > 0 && logical_out <= padded_out)) {
    return fail("EXL3 logical dimensions must lie within the packed geometry");
  }
  if (!(x_cols == logical_in && out_rows == rows && out_cols == logical_out &&
        suh_numel == padded_in && svh_numel == padded_out)) {
    return fail("EXL3 linear input/output/scale geometry mismatch");
  }
  if (rows < 0 || rows > INT_MAX) return fail("EXL3 linear has too many rows");
  if (!known_format(bits_x2, codebook)) {
    return fail("Unsupported EXL3 rate/codebook combination");
  }
  int64_t ws_bytes = 0;
  if (workspace_numel >= 0) {
    const int64_t need = exl3_linear_workspace_size(rows, padded_in, padded_out);
    if (workspace_numel < need) return fail("EXL3 linear workspace is too small");
    if ((reinterpret_cast<uintptr_t>(workspace) & 15) != 0) {
      return fail("EXL3 linear workspace must be 16-byte aligned");
    }
    ws_bytes = workspace_numel * 4;
  }
  const int64_t x_bytes = rows * logical_in * dtype_bytes(x_dtype);
  const int64_t out_bytes = rows * logical_out * dtype_bytes(out_dtype);
  const int64_t tr_bytes = tiles_k * tiles_n * trellis_words * 2;
  const void* inputs[4] = {x, trellis, suh, svh};
  const int64_t input_bytes[4] = {x_bytes, tr_bytes, padded_in * 2, padded_out * 2};
  if (overlaps(out, out_bytes, workspace, ws_bytes)) {
    return fail("unsupported operation: some elements of the input tensor and the written-to "
                "tensor refer to a single memory location.");
  }
  for (int i = 0; i < 4; ++i) {
    if (overlaps(out, out_bytes, inputs[i], input_bytes[i]) ||
        overlaps(workspace, ws_bytes, inputs[i], input_bytes[i])) {
      return fail("unsupported operation: some elements of the input tensor and the written-to "
                  "tensor refer to a single memory location.");
    }
  }
  return kOk;
}

// The small-M path (rows <= 32, chunks of kMaxGemvRows rows) with `partial`
// holding `partial_numel` floats for the K-split partials.  A chunk whose
// partials do not fit runs in column ranges (whole 128-column blocks) that
// do; every range is its own launch on the stream.
int small_linear(const void* x, int x_dtype, int64_t rows, const uint8_t* trellis, int64_t tiles_k,
                 int64_t tiles_n, const uint16_t* suh, const uint16_t* svh, int64_t bits_x2,
                 int64_t codebook, int64_t logical_in, int64_t logical_out, void* out,
                 int out_dtype, float* partial, int64_t partial_numel, hipStream_t s) {
  const int64_t padded_in = tiles_k * 16;
  const int64_t padded_out = tiles_n * 16;
  const GemvPlan p = plan_gemv(reinterpret_cast<uintptr_t>(trellis), bits_x2, padded_in, padded_out,
                               false);
  if (p.splits > 65535) return vq::fail("EXL3 linear K is too large");
  const int64_t chunk_rows = std::min<int64_t>(rows, kMaxGemvRows);
  // columns per launch: every column block when the partials fit, else the
  // most whole blocks that do
  const int64_t per_block = partial_elements(p, chunk_rows, 128);
  const int64_t range_blocks = std::min<int64_t>(padded_out / 128, partial_numel / per_block);
  if (range_blocks < 1) return vq::fail("EXL3 linear workspace is too small");
  const int64_t range_cols = range_blocks * 128;
  // 32-bit buffer offsets: a workgroup's trellis rows and one split's partials
  if (8 * int64_t(p.blocks) * p.groups * tiles_n * 16 * bits_x2 > INT_MAX ||
      4 * partial_elements(p, kMaxGemvRows, range_cols) > INT_MAX) {
    return vq::fail("EXL3 linear N is too large for the small-M kernel");
  }
  const int mode = g_finish_mode.load();
  const int64_t tile_bytes = 16 * bits_x2;
  for (int64_t r0 = 0; r0 < rows; r0 += kMaxGemvRows) {
    const int chunk = int(std::min<int64_t>(rows - r0, kMaxGemvRows));
    for (int64_t c0 = 0; c0 < padded_out; c0 += range_cols) {
      const int64_t cols = std::min<int64_t>(range_cols, padded_out - c0);
      const CounterSlots slots = mode != 0 ? counter_slots(s, cols / 128) : CounterSlots{nullptr, -1};
      GemvArgs a{};
      a.x = static_cast<const uint8_t*>(x) + r0 * logical_in * vq::dtype_bytes(x_dtype);
      a.suh = suh;
      a.svh = svh + c0;
      a.trellis = trellis + (c0 / 16) * tile_bytes;
      a.partial = partial;
      a.out = static_cast<uint8_t*>(out) + (r0 * logical_out + c0) * vq::dtype_bytes(out_dtype);
      a.counters = slots.pool;
      a.counter_base = slots.base;
      a.logical_in = logical_in;
      a.logical_out = std::max<int64_t>(0, std::min<int64_t>(cols, logical_out - c0));
      a.out_stride = logical_out;
      a.tiles_n = tiles_n;
      a.np = cols;
      a.x_dtype = x_dtype;
      a.out_dtype = out_dtype;
      a.rows = chunk;
      a.splits = int(p.splits);
      const dim3 grid{unsigned(cols / 128), unsigned(p.splits), 1u};
      if (int rc = dispatch(bits_x2, codebook, p.load != kLoadHalf, p.load, &a, p.blocks, p.groups,
                            grid, s, nullptr, 0, 0, nullptr)) {
        return rc;
      }
      if (slots.base < 0) {
        if (int rc = launch_output(partial, int(p.splits), chunk, cols, a.svh, a.logical_out,
                                   a.out_stride, a.out, out_dtype, s)) {
          return rc;
        }
      }
    }
  }
  return vq::kOk;
}

}  // namespace
}  // namespace exl3

extern "C" int exl3_linear_out(const void* x, int x_dtype, int64_t rows, int64_t x_cols,
                               const void* trellis, int64_t tiles_k, int64_t tiles_n,
                               int64_t trellis_words, const void* suh, int64_t suh_numel,
                               const void* svh, int64_t svh_numel, int64_t bits_x2,
                               int64_t codebook, int64_t logical_in, int64_t logical_out,
                               void* out, int out_dtype, int64_t out_rows, int64_t out_cols,
                               float* workspace, int64_t workspace_numel, void* stream) {
  if (workspace_numel < 0) return vq::fail("EXL3 linear workspace is too small");
  if (int rc = exl3::check_linear(x, x_dtype, rows, x_cols, trellis, tiles_k, tiles_n, trellis_words,
                                  suh, suh_numel, svh, svh_numel, bits_x2, codebook, logical_in,
                                  logical_out, out, out_dtype, out_rows, out_cols, workspace,
                                  workspace_numel)) {
    return rc;
  }
  if (rows == 0) return vq::kOk;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (rows > exl3::kGemvChunkedRows) {
    return exl3::prefill_linear(x, x_dtype, rows, static_cast<const uint8_t*>(trellis), tiles_k,
                                tiles_n, static_cast<const uint16_t*>(suh),
                                static_cast<const uint16_t*>(svh), int(bits_x2), int(codebook),
                                logical_in, logical_out, out, out_dtype, workspace, s);
  }
  return exl3::small_linear(x, x_dtype, rows, static_cast<const uint8_t*>(trellis), tiles_k, tiles_n,
                            static_cast<const uint16_t*>(suh), static_cast<const uint16_t*>(svh),
                            bits_x2, codebook, logical_in, logical_out, out, out_dtype, workspace,
                            workspace_numel, s);
}

namespace exl3 {
namespace {

// The scratch of exl3_linear_out_scratch: the small-M path's K-split
// partials (in column ranges that fit) or the large-M path's activations.
// One copy per device, held until the process ends.
constexpr int64_t kScratchFloats = int64_t(4) << 20;  // 16 MiB
__device__ __align__(256) float scratch[kScratchFloats];

// The device address of `scratch` on the current device, looked up once per
// device (each device holds its own copy, at its own address); null on
// failure, with the error recorded.
float* scratch_address() {
  static std::mutex mutex;
  static std::map<int, float*> addresses;
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) {
    (void)hipGetLastError();
    vq::fail("EXL3 linear scratch: no current device");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mutex);
  const auto it = addresses.find(device);
  if (it != addresses.end()) return it->second;
  float* ptr = nullptr;
  if (hipGetSymbolAddress(reinterpret_cast<void**>(&ptr), HIP_SYMBOL(scratch)) != hipSuccess || !ptr) {
    (void)hipGetLastError();
    vq::fail("EXL3 linear scratch: hipGetSymbolAddress failed");
    return nullptr;
  }
  addresses[device] = ptr;
  return ptr;
}

}  // namespace
}  // namespace exl3

extern "C" int64_t exl3_linear_scratch_rows(int64_t padded_in, int64_t padded_out) {
  if (exl3::check_padded(padded_in) != vq::kOk || exl3::check_padded(padded_out) != vq::kOk) return -1;
  // small-M calls always fit (column ranges); large-M needs rows * (padded_in + 1)
  const int64_t large = exl3::kScratchFloats / (padded_in + 1);
  return std::max<int64_t>(exl3::kGemvChunkedRows, large);
}

extern "C" int exl3_linear_out_scratch(const void* x, int x_dtype, int64_t rows, int64_t x_cols,
                                       const void* trellis, int64_t tiles_k, int64_t tiles_n,
                                       int64_t trellis_words, const void* suh, int64_t suh_numel,
                                       const void* svh, int64_t svh_numel, int64_t bits_x2,
                                       int64_t codebook, int64_t logical_in, int64_t logical_out,
                                       void* out, int out_dtype, int64_t out_rows, int64_t out_cols,
                                       void* stream) {
  if (int rc = exl3::check_linear(x, x_dtype, rows, x_cols, trellis, tiles_k, tiles_n, trellis_words,
                                  suh, suh_numel, svh, svh_numel, bits_x2, codebook, logical_in,
                                  logical_out, out, out_dtype, out_rows, out_cols, nullptr, -1)) {
    return rc;
  }
  const int64_t padded_in = tiles_k * 16;
  if (rows > exl3::kGemvChunkedRows && rows * (padded_in + 1) > exl3::kScratchFloats) {
    return vq::fail("EXL3 linear: " + std::to_string(rows) + " rows of " + std::to_string(padded_in) +
                    " inputs exceed the 16 MiB static scratch (at most " +
                    std::to_string(exl3::kScratchFloats / (padded_in + 1)) +
                    " rows above 32 per call): split the rows or use exl3_linear_out");
  }
  if (rows == 0) return vq::kOk;
  float* scratch = exl3::scratch_address();
  if (!scratch) return vq::kHipFailure;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (rows > exl3::kGemvChunkedRows) {
    return exl3::prefill_linear(x, x_dtype, rows, static_cast<const uint8_t*>(trellis), tiles_k,
                                tiles_n, static_cast<const uint16_t*>(suh),
                                static_cast<const uint16_t*>(svh), int(bits_x2), int(codebook),
                                logical_in, logical_out, out, out_dtype, scratch, s);
  }
  return exl3::small_linear(x, x_dtype, rows, static_cast<const uint8_t*>(trellis), tiles_k, tiles_n,
                            static_cast<const uint16_t*>(suh), static_cast<const uint16_t*>(svh),
                            bits_x2, codebook, logical_in, logical_out, out, out_dtype, scratch,
                            exl3::kScratchFloats, s);
}

extern "C" int exl3_set_gemv_blocks(int blocks) {
  if (blocks != 0 && blocks != 1 && blocks != 2 && blocks != 4 && blocks != 8) {
    return vq::fail("EXL3 GEMV blocks per workgroup must be 0 (automatic), 1, 2, 4 or 8");
  }
  exl3::g_blocks_override.store(blocks);
  return vq::kOk;
}

extern "C" int exl3_set_gemv_groups(int groups) {
  if (groups != 0 && groups != 1 && groups != 4) {
    return vq::fail("EXL3 GEMV groups per workgroup must be 0 (automatic), 1 or 4");
  }
  exl3::g_groups_override.store(groups);
  return vq::kOk;
}

extern "C" int exl3_set_gemv_finish(int mode) {
  if (mode < -1 || mode > 1) return vq::fail("EXL3 GEMV finish mode must be -1, 0 or 1");
  exl3::g_finish_mode.store(mode);
  return vq::kOk;
}

extern "C" int64_t exl3_counter_fallbacks(void) { return exl3::g_counter_fallbacks.load(); }
