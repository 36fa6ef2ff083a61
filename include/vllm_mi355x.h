/*
 * C-ABI of the MI355X (gfx950) quantized-weight matmul library
 * (libvllm_mi355x.so): EXL3 trellis-coded linear layers and the
 * Marlin-layout int4 fused MoE.
 *
 * Every entry point takes plain device pointers, sizes, dtype codes and a
 * HIP stream (hipStream_t passed as void*; NULL = the default stream), runs
 * asynchronously on that stream, never allocates, never synchronizes, and
 * returns a status code.  On a nonzero status vllm_mi355x_last_error()
 * returns the message (thread-local), worded as the reference's TORCH_CHECK
 * messages are.  All buffers are caller-owned; only `out` and `workspace`
 * arguments are written.
 *
 * Reference interfaces replaced (paths relative to the reference repo):
 *   _exl3_C schema ..................... csrc/exl3/module.cpp:12-67
 *   _ampere_marlin_C schema ............ csrc/ampere_marlin/decode_orig.cu:403-411
 */
#ifndef VLLM_MI355X_H
#define VLLM_MI355X_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VLLM_MI355X_ABI_VERSION 1

/* Status codes. */
#define VQ_OK 0
#define VQ_INVALID_ARGUMENT 1 /* a check failed; see vllm_mi355x_last_error() */
#define VQ_HIP_FAILURE 2      /* a launch failed */

/* Element types of activations and outputs. */
#define VQ_BF16 0
#define VQ_FP16 1
#define VQ_FP32 2

/* Message of the last failed call on this thread ("" if none). */
const char* vllm_mi355x_last_error(void);
/* VLLM_MI355X_ABI_VERSION of the loaded library. */
int vllm_mi355x_abi_version(void);

/* ---- EXL3 ---------------------------------------------------------------- */

/*
 * FP32 workspace elements exl3_linear_out needs for calls of up to max_rows
 * rows of a padded_in x padded_out matrix: the larger of the small-M path's
 * K-split partial sums, min(max_rows, 8) * splits * padded_out (splits =
 * padded_in / 128 / blocks, with the automatic blocks per workgroup, at most
 * 32 where the shape allows), and, above exl3_linear_prefill_rows() rows,
 * the large-M path's max_rows * (padded_in + 1) (FP16 high/low activations,
 * one row exponent per row).  The two paths never run in one call.  Returns
 * -1 (with an error message) for a negative row count or padded sizes that
 * are not positive multiples of 128.
 * Replaces _exl3_C::linear_workspace_size (csrc/exl3/dense.cu:72-78).
 */
int64_t exl3_linear_workspace_size(int64_t max_rows, int64_t padded_in, int64_t padded_out);

/*
 * exl3_linear_out without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid allocation).  No counterpart in the
 * reference.  The same checks, kernels and results as exl3_linear_out; the
 * K-split partials (rows <= 32, in column ranges that fit) or the large-M
 * activations live in a static 16 MiB device array of the library (one per
 * device, held until the process ends; its address is looked up on the
 * first call on each device).  Calls of more than 32 rows need rows *
 * (padded_in + 1) floats of it: larger ones are rejected with an error
 * (exl3_linear_scratch_rows gives the limit).  Calls on one device share
 * the array: calls that overlap in time on one GPU (different streams)
 * race and must be ordered by the caller.  Allocates nothing.
 */
int exl3_linear_out_scratch(const void* x, int x_dtype, int64_t rows, int64_t x_cols,
                            const void* trellis, int64_t tiles_k, int64_t tiles_n,
                            int64_t trellis_words, const void* suh, int64_t suh_numel,
                            const void* svh, int64_t svh_numel, int64_t bits_x2, int64_t codebook,
                            int64_t logical_in, int64_t logical_out, void* out, int out_dtype,
                            int64_t out_rows, int64_t out_cols, void* stream);

/*
 * The most rows one exl3_linear_out_scratch call takes for a padded_in x
 * padded_out matrix (-1 for bad sizes).  No counterpart in the reference.
 */
int64_t exl3_linear_scratch_rows(int64_t padded_in, int64_t padded_out);

/*
 * The row count above which exl3_linear_out runs the large-M (prefill) GEMM;
 * up to it, the small-M kernel in chunks of 8 rows.  The reference's routing
 * question _exl3_C::linear_prefill_applies (vllm_sm80/kernels/exl3/
 * dense_prefill_tc.py:57-80) answers from it.
 */
int exl3_linear_prefill_rows(void);

/*
 * out[r][n] = RN_out( H128(C[r])[n] * svh[n] ),
 * C[r][n]   = sum_k t[r][k] * W[k][n],  t[r] = H128(x[r] * suh)  (FP32),
 * with W the exact FP16 weights decoded from the trellis, H128 the
 * normalized Sylvester Hadamard transform over 128-element blocks.
 *
 *   x        [rows][logical_in] of x_dtype (VQ_BF16 or VQ_FP16)
 *   trellis  int16 [tiles_k][tiles_n][trellis_words], trellis_words must be
 *            8 * bits_x2; padded_in = 16 * tiles_k, padded_out = 16 * tiles_n
 *   suh      fp16 [suh_numel == padded_in], svh fp16 [svh_numel == padded_out]
 *   bits_x2  2..16 with codebook 1 (mcg, even rates) or 2 (mul1, also 3/5/7)
 *   out      [rows][logical_out] of out_dtype (VQ_BF16, VQ_FP16 or VQ_FP32)
 *   workspace FP32, >= exl3_linear_workspace_size(rows, ...) elements,
 *            16-byte aligned, overlapping no other argument.
 * The weights are decoded bit-exactly; the products are summed in FP32 on
 * the matrix cores, with the activations split into FP16 high and low
 * parts (about 22 significant bits, the activation precision of the
 * reference's tensor-core kernels, csrc/exl3/dense_prefill_tc.h:5-12), so
 * the result agrees with the reference's sequential FP32 chain to FP32
 * rounding, not bit for bit.  Above 32 rows a 16-byte aligned trellis runs
 * on the many-row tile GEMM, any other on the decode-to-LDS prefill GEMM;
 * under exl3_set_tile_precision(1) the tile GEMM rounds each rotated input
 * once to FP16 instead (FP16-operand tolerance, an rms error of about
 * 2^-12 rms(result), half the matrix work).  A small-M call
 * whose K-split partials (under a forced exl3_set_gemv_blocks, or an
 * unaligned trellis) exceed the workspace runs in column ranges that fit.
 * Replaces _exl3_C::linear_out (csrc/exl3/dense.cu:80-149; schema
 * csrc/exl3/module.cpp:13-15).
 */
int exl3_linear_out(const void* x, int x_dtype, int64_t rows, int64_t x_cols,
                    const void* trellis, int64_t tiles_k, int64_t tiles_n,
                    int64_t trellis_words, const void* suh, int64_t suh_numel,
                    const void* svh, int64_t svh_numel, int64_t bits_x2,
                    int64_t codebook, int64_t logical_in, int64_t logical_out,
                    void* out, int out_dtype, int64_t out_rows, int64_t out_cols,
                    float* workspace, int64_t workspace_numel, void* stream);

/*
 * FP32 workspace elements exl3_moe_out needs: with A = max_rows * topk,
 * hpad / ipad the hidden / intermediate sizes rounded up to 128,
 * A * (hpad + 3 * ipad) (activations, gate, up and down-input rows) plus the int32
 * routing table (4 + A rounded up to 4 + 4 A) plus A * max(hpad, ipad) / 128
 * int32 scale exponents plus A int32 experts of the sorted rows; 0 when
 * local_experts is 0; -1 (with an error
 * message) for negative counts or nonpositive sizes.
 * Replaces _exl3_C::moe_workspace_size and moe_workspace_size_v2
 * (csrc/exl3/moe.cu:304-317, csrc/exl3/moe_v2.cu:2041-2061).
 */
int64_t exl3_moe_workspace_size(int64_t max_rows, int64_t hidden_size, int64_t intermediate_size,
                                int64_t topk, int64_t local_experts);

/*
 * Routed experts: out[t] = sum over the local routes k of token t, in route
 * order, of weights[t][k] * down_e(act(gate_e(x[t]), up_e(x[t]))), each
 * projection an EXL3 linear of the expert (H128(x * suh), trellis, H128,
 * svh), act = SiLU(min(g, L)) * clamp(u, -L, L) (L = swiglu_limit, 0 = no
 * clamp).  x / out [rows][hidden] of x_dtype (VQ_BF16 or VQ_FP16; out the
 * same), topk_ids [rows][topk] int32 (ids64 = 0) or int64 global expert ids
 * (negative or out of range = not routed here), topk_weights FP32,
 * expert_map [global_experts] int32 / int64 local ids (-1 = another rank),
 * packed_ptrs [local][3][3] device addresses {trellis, suh, svh} of gate,
 * up, down, packed_meta [local][3][4] {padded_in, padded_out, bits_x2,
 * codebook} (the caller keeps the matrices alive).  bits_x2 = 0 decodes
 * every expert's own format (moe_out); bits_x2 = 2..16 is the layer's one
 * mul1 rate (moe_out_v2; 2..8 run a decode specialized for the rate, 10..16
 * the run-time decode).  An expert whose matrices are not hpad x ipad /
 * ipad x hpad, or (bits_x2 > 0) not of that rate, yields NaN rows.  Every
 * argument check runs before the first launch.
 * Replaces _exl3_C::moe_out (csrc/exl3/moe.cu:450-458) and
 * _exl3_C::moe_out_v2 (csrc/exl3/moe_v2.h:19-30; schema module.cpp:19-26).
 */
int exl3_moe_out(const void* x, int x_dtype, int64_t rows, int64_t hidden, const void* topk_ids,
                 int ids64, const float* topk_weights, int64_t topk, const int64_t* packed_ptrs,
                 const int64_t* packed_meta, int64_t local_experts, const void* expert_map,
                 int map64, int64_t global_experts, int64_t intermediate_size, int64_t bits_x2,
                 void* out, int out_dtype, float* workspace, int64_t workspace_numel,
                 float swiglu_limit, void* stream);

/*
 * Test and tuning switch, process-wide: the routed-row count from which an
 * expert of a fixed-rate call (exl3_moe_out with bits_x2 > 0: moe_out_v2,
 * and moe_out_prefill at its bits_x2 10) runs on the many-row tile GEMM
 * (tasks of up to 128 rows) instead of the small-M GEMV; 0 = automatic (48
 * rows, and only when the call's tile tasks make at least 128 workgroups in
 * the narrower projection), any other value = that threshold with no
 * workgroup minimum (1: every expert with 16-byte aligned matrices).  Both
 * kernels keep FP16 high and low activation parts (unless
 * exl3_set_tile_precision(1)).  No counterpart in the reference (its
 * nearest is the prefill routing of moe_out_prefill, ops.py:1880-1910).
 */
int exl3_set_moe_tile_rows(int rows);

/*
 * Precision switch, process-wide: 0 (default) = the many-row tile GEMM
 * (exl3_linear_out above 32 rows, the MoE tile tasks) multiplies FP16 high
 * and low activation parts (~22 bits) against the exact FP16 weights, as
 * the reference's tensor-core kernels split them
 * (csrc/exl3/dense_prefill_tc.h:5-12); 1 = the high parts alone (each
 * rotated input rounded once to FP16: half the matrix work, an rms error of
 * about 2^-12 rms(result)), an explicit opt-in below the reference's
 * precision.  No counterpart in the reference.
 */
int exl3_set_tile_precision(int fp16_only);

/*
 * Test and tuning switch, process-wide: the kernel exl3_linear_out runs
 * above 32 rows: 0 = automatic (the tile GEMM for a 16-byte aligned
 * trellis, else the decode-to-LDS prefill GEMM), 1 = the prefill GEMM,
 * 2 = as 0.  Both keep the activations' high and low parts (the tile GEMM
 * unless exl3_set_tile_precision(1)).  No counterpart in the reference
 * (its nearest is set_gemm_shape_override, csrc/exl3/gemm.cu:400-409).
 */
int exl3_set_prefill_kernel(int kernel);

/*
 * Test and tuning switch, process-wide: how exl3_linear_out finishes its
 * small-M (<= 8 rows) launches.  -1 (default): the last workgroup of each
 * 128-column block sums the K-split partials and writes the outputs, using
 * arrival counters from a static pool of 128 ranges per device: one range
 * per stream for its eager launches and one per stream for every graph
 * captured on it (graphs captured on one stream must not be replayed
 * concurrently with each other; once the ranges are spent, launches on
 * further streams use the separate kernel, counted by
 * exl3_counter_fallbacks); 0: always a separate output kernel; 1: as -1.
 * Both finishes add in the same order, so results are bitwise equal.
 * No counterpart in the reference (its nearest is the test-only
 * set_gemm_shape_override, csrc/exl3/gemm.cu:400-409).
 */
int exl3_set_gemv_finish(int mode);

/*
 * Launches since the library loaded that found no arrival-counter range
 * and took the separate finish (a performance fallback, never a wrong
 * result).  No counterpart in the reference.
 */
int64_t exl3_counter_fallbacks(void);

/*
 * Test and tuning switch, process-wide: 128-input blocks per workgroup of
 * the small-M kernel (0 = automatic, 1, 2, 4 or 8; more blocks = fewer K
 * splits; a value that does not divide padded_in / 128 is ignored for that
 * call).  Changes the FP32 summation grouping, not the weights.  No
 * counterpart in the reference (its nearest is set_gemm_shape_override,
 * csrc/exl3/gemm.cu:400-409).
 */
int exl3_set_gemv_blocks(int blocks);

/*
 * Test and tuning switch, process-wide: groups of 4 wavefronts per
 * workgroup of the small-M kernel (0 = automatic, 1 or 4).  A group count of
 * 4 applies when the input blocks divide into whole 4 * blocks ranges (else
 * 1 is used).  Changes the FP32 summation grouping, not the weights.  No
 * counterpart in the reference (its nearest is set_gemm_shape_override,
 * csrc/exl3/gemm.cu:400-409).
 */
int exl3_set_gemv_groups(int groups);

/*
 * Decodes every tile of a trellis into its exact FP16 weights,
 * out[k][n] (k < 16 * tiles_k, n < 16 * tiles_n, row-major, FP16 bits).
 * The inspection form of the decode exl3_linear_out fuses; it has no
 * operator of its own in the reference, whose decode is
 * csrc/exl3/reference.cu:62-103 (core_value) / csrc/exl3/codec.cuh:45-180.
 */
int exl3_decode(const void* trellis, int64_t tiles_k, int64_t tiles_n, int64_t trellis_words,
                int64_t bits_x2, int64_t codebook, void* out, void* stream);

/*
 * Selected rows of an EXL3 PLE table (trellis-compressed embeddings), BF16:
 * packed_rows int16 [rows][words], words = 1 + dim * bits / 16 (an FP16
 * scale, then a little-endian ring of dim * bits bits); channel c's state
 * takes bit m from ring bit ((c - m / bits) mod dim) * bits + m % bits; the
 * value is RN_bf16(RN32(RN16(RN32(RN32(1024 + bytesum(state * 0x83DCD12D)) *
 * fp16(0x1EEE)) + fp16(0xC931))) * scale) + head_bias[head][c]) for a row
 * whose global id lies in [owner_lo, owner_hi) and inside the vocabulary of
 * the last head starting at or before it (head_offsets ascending, as the
 * reference's search also assumes; head_offsets / head_vocab_sizes int64
 * [heads], head_bias fp16 [heads][dim]); every other row is zero.
 * Replaces _exl3_C::ple_decode_out (csrc/exl3/ple.cu:167-234; schema
 * csrc/exl3/module.cpp:30-32).
 */
int exl3_ple_decode_out(const void* packed_rows, int64_t rows, int64_t words,
                        const int64_t* global_ids, const void* head_bias, int64_t heads,
                        const int64_t* head_offsets, const int64_t* head_vocab_sizes, int64_t dim,
                        int64_t owner_lo, int64_t owner_hi, int64_t bits, void* out, void* stream);

/* ---- Marlin-format int4 fused MoE ------------------------------------------
 *
 * Weights in vLLM's Marlin packing (csrc/ampere_marlin/decode_orig.cu:10-19):
 * uint4b8 nibbles, int32 [E][K/16][2N]; group-128 scales [E][K/128][N] of
 * the activation dtype (VQ_BF16 or VQ_FP16) with the in-chunk column
 * permutation.  Dequant w = RN((q - 8) * s), one rounding, as the reference.
 */

/* Modes of marlin_moe_gemm. */
#define VQ_MARLIN_PARTIAL 0 /* FP32 k-split partials part[ks][slot][N] */
#define VQ_MARLIN_STORE 1   /* out[slot][n] = RN(sum) */
#define VQ_MARLIN_TOPK 2    /* out[slot][n] = RN(RN(sum) * RN(topk_w[slot])) */
#define VQ_MARLIN_SWIGLU 3  /* marlin_moe_gemm_direct only: h = SwiGLU(gate, up) */

/*
 * Grouped expert GEMM over aligned blocks: for every block b < ntpp[0] /
 * block_size with expert e = expert_ids[b] in [0, experts), every routed
 * slot sid = sorted[b * block_size + t] < n_slots, and every column n < N:
 * sum over k < K (K-split into ksplit equal ranges of whole 128-k groups)
 * of a[sid / top_k][k] * w_e[k][n], FP32 on the matrix cores.  a: rows of
 * a_stride elements (a_stride % 8 == 0), at least ceil(n_slots / top_k)
 * rows; block_size a multiple of 8 up to 64.  part needs ksplit * n_slots *
 * N floats (mode PARTIAL); out rows of out_stride elements (STORE / TOPK,
 * ksplit 1).  Rows of unrouted slots are left untouched.  sorted == NULL
 * (and ntpp NULL): identity routing, block b is slot b alone and
 * expert_ids[b] its local expert (expert_ids_numel >= n_slots): one token's
 * slots need no alignment launch.
 * Replaces _ampere_marlin_C::decode_gemm_orig / decode_gemm_v2
 * (csrc/ampere_marlin/decode_orig.cu:361-390, decode_v2.cu:395-399) and
 * prefill_tile_gemm (csrc/ampere_marlin/prefill_tiles.cu:12-26, upstream
 * moe_wna16_marlin_gemm).
 */
int marlin_moe_gemm(const void* a, int act_dtype, int64_t a_rows, int64_t a_stride,
                    const int32_t* w, const void* scales, int64_t experts, const int32_t* sorted,
                    int64_t sorted_numel, const int32_t* expert_ids, int64_t expert_ids_numel,
                    const int32_t* ntpp, const float* topk_w, int64_t top_k, int64_t n_slots,
                    int64_t K, int64_t N, int64_t block_size, int mode, int64_t ksplit,
                    float* part, int64_t part_numel, void* out, int64_t out_stride,
                    int64_t out_rows, void* stream);

/*
 * marlin_moe_gemm (same arguments, checks and sums, bitwise) on k-permuted
 * activations: a's rows hold, in every 32-k step, element 8q + 2s + t = k
 * 8s + 2q + t (marlin_permute_act); weights stream through LDS and each
 * lane loads its matrix operand directly, with no staging barrier.  Eight
 * 64-column tiles per workgroup (SWIGLU: two gate tiles and their up
 * tiles), ksplit 1 for STORE / TOPK / SWIGLU.  Mode
 * SWIGLU (ksplit 1, N % 256 == 0): N = 2 Nh columns of gate | up, out =
 * h[slot] (rows of out_stride elements, out_stride % 32 == 0) in the
 * permuted layout, h = RN(RN(SiLU(min(G, L))) * clamp(U, -L, L)) of the
 * activation-dtype roundings G, U of the sums (marlin_moe_act's arithmetic).
 * No counterpart in the reference: the fused path's layout of
 * decode_gemm_orig / decode_act_orig (csrc/ampere_marlin/decode_orig.cu:
 * 272-305, 361-390).
 */
int marlin_moe_gemm_direct(const void* a_perm, int act_dtype, int64_t a_rows, int64_t a_stride,
                           const int32_t* w, const void* scales, int64_t experts,
                           const int32_t* sorted, int64_t sorted_numel, const int32_t* expert_ids,
                           int64_t expert_ids_numel, const int32_t* ntpp, const float* topk_w,
                           int64_t top_k, int64_t n_slots, int64_t K, int64_t N,
                           int64_t block_size, int mode, int64_t ksplit, float limit, float* part,
                           int64_t part_numel, void* out, int64_t out_stride, int64_t out_rows,
                           void* stream);

/*
 * out[r][p(k)] = a[r][k] for r < rows, k < cols (cols % 32 == 0), p the
 * permutation marlin_moe_gemm_direct reads (inside each 32-k step, k = 8s +
 * 2q + t goes to 8q + 2s + t).  No counterpart in the reference.
 */
int marlin_permute_act(const void* a, int act_dtype, int64_t rows, int64_t cols, int64_t a_stride,
                       void* out, int64_t out_stride, void* stream);

/*
 * SwiGLU of the w13 partials: G / U = RN(sum over ks in order of
 * part[ks][slot][n] / [..][Nh + n]), h[slot][n] = RN(RN(SiLU(min(G, L))) *
 * clamp(U, -L, L)) (limit = +inf: no clamp); slots with ids[slot] < 0 are
 * skipped.  Replaces _ampere_marlin_C::decode_act_orig
 * (csrc/ampere_marlin/decode_orig.cu:272-305, :392-401).
 */
int marlin_moe_act(const float* part, const int32_t* ids, int64_t ksplit, int64_t n_slots,
                   int64_t nh, float limit, void* h, int act_dtype, void* stream);

/*
 * marlin_moe_gemm in mode PARTIAL (same arguments, checks and sums; N % 128
 * == 0, partials below 2 GiB) followed by marlin_moe_act on its partials
 * (ids, limit; h rows of N / 2 elements, h_rows >= n_slots), bitwise equal
 * to the two calls, in one launch: the last of the 2 * ksplit wavefronts
 * that produce a (block, 64 gate columns) pair of tiles to finish forms
 * that pair's h from every split's partials, counted by the library's
 * arrival counters (one per block and 64 gate columns; when none are free
 * it makes the two calls).  The partials are still written.  Calls that
 * overlap on one stream's counters race, as on the split-K GEMV's.
 * The reference's decode_gemm_orig + decode_act_orig pair
 * (csrc/ampere_marlin/decode_orig.cu:272-305, :361-401) in one call.
 */
int marlin_moe_w13_act(const void* a, int act_dtype, int64_t a_rows, int64_t a_stride,
                       const int32_t* w, const void* scales, int64_t experts, const int32_t* sorted,
                       int64_t sorted_numel, const int32_t* expert_ids, int64_t expert_ids_numel,
                       const int32_t* ntpp, const int32_t* ids, int64_t top_k, int64_t n_slots,
                       int64_t K, int64_t N, int64_t block_size, int64_t ksplit, float limit,
                       float* part, int64_t part_numel, void* h, int64_t h_stride, int64_t h_rows,
                       void* stream);

/*
 * marlin_moe_gemm in mode TOPK with identity routing (sorted and ntpp NULL,
 * ksplit 1, a: one row per slot, so the GEMM's own top_k is 1; top_k here:
 * slots per token, n_slots a multiple of it; out rows of exactly N
 * elements, below 2 GiB) followed by moe_sum of its rows with expert_ids as the
 * routed ids (sum_out[t][n] = RN(FP32 sum over the slots of token t, in slot
 * order, whose id is in [0, experts))), bitwise equal to the two calls, in
 * one launch: the last wavefront of a token's routed slots to finish a
 * 64-column tile sums that tile, counted by the library's arrival counters
 * (one per token and 64 columns; when none are free, or top_k > 64, it
 * makes the two calls).  The slot rows are still written.  Calls that overlap on one
 * stream's counters race.  The reference's one-token decode_gemm_orig (w2)
 * + moe_sum pair (csrc/ampere_marlin/decode_orig.cu:361-390,
 * vllm_sm80/kernels/moe/routing.py:579-600) in one call.
 */
int marlin_moe_w2_sum(const void* a, int act_dtype, int64_t a_rows, int64_t a_stride, const int32_t* w,
                      const void* scales, int64_t experts, const int32_t* expert_ids,
                      int64_t expert_ids_numel, const float* topk_w, int64_t top_k, int64_t n_slots,
                      int64_t K, int64_t N, int64_t block_size, void* out, int64_t out_stride,
                      int64_t out_rows, void* sum_out, void* stream);

/*
 * The dequantized weights of one packed matrix, out[k][n] (K x N, the
 * activation dtype), through the GEMM's own fragment and dequant path.
 * The inspection form of the decode marlin_moe_gemm fuses; the reference's
 * is csrc/ampere_marlin/decode_orig.cu:56-67 (upstream dequant.h).
 */
int marlin_dequant(const int32_t* w, const void* scales, int act_dtype, int64_t K, int64_t N,
                   void* out, void* stream);

/*
 * out[t][c] = RN(FP32 sum over slots k = 0..topk-1, in order, of
 * in[t][k][c]); with ids, slots whose id is outside [0, experts) add
 * nothing.  Replaces moe_sum (vllm_sm80/kernels/moe/routing.py:579-600,
 * upstream _moe_C::moe_sum).
 */
int moe_sum(const void* in, int act_dtype, int64_t tokens, int64_t topk, int64_t hidden,
            const int32_t* ids, int64_t experts, void* out, void* stream);

/*
 * The routed sum with the shared expert's output folded in, one launch:
 * out[t][c] = RN(f32(RN(FP32 sum over slots in order of in[t][k][c])) +
 * f32(shared[t * shared_stride0 + c * shared_stride1])) (element strides).
 * Replaces moe_sum_add (vllm_sm80/kernels/moe/sum.py:18-56).
 */
int moe_sum_add(const void* in, int act_dtype, int64_t tokens, int64_t topk, int64_t hidden,
                const void* shared, int64_t shared_stride0, int64_t shared_stride1, void* out,
                void* stream);

/*
 * Deterministic block alignment of routed rows: rows grouped by (mapped)
 * expert in ascending expert order, ascending flat index inside an expert,
 * each expert padded to a multiple of block_size with the sentinel numel;
 * expert_ids[b] = expert of block b (-1 past the padded total); ntpp[0] =
 * padded total.  Ids outside [0, num_experts) and experts mapped to -1 are
 * dropped.  sorted needs numel + num_experts * (block_size - 1) entries
 * (min(numel * block_size, that) when numel < num_experts).
 * Replaces moe_align_block_size (vllm_sm80/kernels/moe/align.py:233-273,
 * spec tests/kernels/moe_align_reference.py:18-70).
 */
int moe_align_block_size(const int32_t* topk_ids, int64_t numel, int64_t num_experts,
                         int64_t block_size, const int32_t* expert_map, int32_t* sorted,
                         int64_t sorted_numel, int32_t* expert_ids, int64_t expert_ids_numel,
                         int32_t* ntpp, void* stream);

/*
 * moe_align_block_size and marlin_permute_act (the same arguments, checks
 * and results) in one launch: the permutation runs beside the
 * single-workgroup alignment.  The output rows must be 16-byte aligned
 * (out_stride % 8 == 0).  No counterpart in the reference: the direct fused
 * path's first step (align, then the w13 GEMM's k-permuted input).
 */
int marlin_moe_align_permute(const int32_t* topk_ids, int64_t numel, int64_t num_experts,
                             int64_t block_size, const int32_t* expert_map, int32_t* sorted,
                             int64_t sorted_numel, int32_t* expert_ids, int64_t expert_ids_numel,
                             int32_t* ntpp, const void* a, int act_dtype, int64_t rows,
                             int64_t cols, int64_t a_stride, void* out, int64_t out_stride,
                             void* stream);

/*
 * MoE router with the block alignment: logits = x W^T in FP32 (bf16 or fp16
 * x [M][K] with row stride x_stride, weight [E][K] contiguous; products
 * exact, summed in one fixed order on the matrix cores), then per row the
 * top-k experts by key, ties to the lower expert: scoring 1 = sigmoid +
 * bias (score 0.5 tanh(0.5 l) + 0.5, key score + bias[e]), 0 = softmax
 * (key = score = exp(l - max) / sum); weights = the selected scores,
 * divided by (their sum + 1e-20) when renormalize, times scale; rows with
 * is_padding[m] != 0 (optional uint8 [M]) route to -1.  Then the
 * moe_align_block_size alignment of the ids (same outputs and sizes).
 * logits fp32 [M][E], topk_weights fp32 / topk_ids int32 [M][topk].  Two
 * launches; K % 128 == 0, E <= 1024, topk <= 64.  Replaces moe_route
 * (vllm_sm80/kernels/moe/route.py:994-1084: router GEMV, sigmoid/bias
 * top-k, alignment), with softmax scoring added for routers that use it.
 */
int moe_route(const void* x, int x_dtype, int64_t M, int64_t K, int64_t x_stride,
              const void* weight, const float* bias, int64_t num_experts, int64_t topk,
              int scoring, int renormalize, float scale, int64_t block_size,
              const uint8_t* is_padding, float* logits, float* topk_weights, int32_t* topk_ids,
              int32_t* sorted, int64_t sorted_numel, int32_t* expert_ids,
              int64_t expert_ids_numel, int32_t* ntpp, void* stream);

/*
 * Split-cover MoE alignment: the routed rows sorted by expert (stable, by
 * flat index) into four block lists of sizes 64, 48, 32 and 16, an expert
 * with r rows getting cover[r][k] blocks of size k (cover: int32
 * [cover_rows + 1][4] on the device, the cheapest cover by the caller's cost
 * model; cover_rows >= numel).  Its rows fill its list-0 blocks, then its
 * list-1 blocks, and so on; only its last block is padded (sentinel numel).
 * List k: sorted ids (sorted_numel[k] >= numel + size_k * E entries), expert
 * per block (eids_numel[k] >= (numel + size_k * E) / size_k; -1 past the
 * list), ntpp[k] = its padded row count.  Deterministic (no atomic decides a
 * position).  One workgroup; at most 1820 experts.  Replaces split_align
 * (vllm_sm80/kernels/marlin_moe/split_align.py:173-224 and its five Triton
 * kernels, split_align.py:45-170).
 */
int moe_split_align(const int32_t* topk_ids, int64_t numel, int64_t num_experts,
                    const int32_t* expert_map, const int32_t* cover, int64_t cover_rows,
                    int32_t* sorted64, int32_t* sorted48, int32_t* sorted32, int32_t* sorted16,
                    const int64_t* sorted_numel, int32_t* eids64, int32_t* eids48,
                    int32_t* eids32, int32_t* eids16, const int64_t* eids_numel, int32_t* ntpp,
                    void* stream);

#ifdef __cplusplus
}
#endif

#endif /* VLLM_MI355X_H */
