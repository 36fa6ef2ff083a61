/*
 * CPU oracle for the Marlin-format int4 fused MoE.  TEST INFRASTRUCTURE ONLY:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker.  The product path never calls
 * it and has no CPU fallback.
 *
 * A plain-C restatement of the reference's W4A16 MoE path:
 *   layout      csrc/ampere_marlin/decode_orig.cu:10-19 (uint4b8 nibbles in
 *               the mma A-fragment order, int32 [E][K/16][2N]; group-128
 *               scales [E][K/128][N] with the in-chunk column permutation)
 *   dequant     decode_orig.cu:56-67 and csrc/quantization/marlin/dequant.h:
 *               w = RN_act((q - 8) * s), one rounding ((q - 8) * s is exact
 *               in FP32)
 *   w13 / w2    decode_orig.cu:188-229 and marlin_moe_template.h:1798-1830:
 *               RN_act(FP32 sum) per output; the down projection then
 *               RN_act(RN_act(sum) * RN_act(router weight))
 *   activation  decode_orig.cu:275-305: h = RN(RN(SiLU(min(G, L))) *
 *               clamp(U, -L, L)), G / U already rounded to the activation
 *               dtype
 *   moe_sum     vllm_sm80/kernels/moe/routing.py:579-600: FP32 sum over the
 *               top-k slots in slot order, rounded once
 *   align       tests/kernels/moe_align_reference.py:18-70: routed rows
 *               grouped by expert, ranked by ascending flat index, each
 *               expert padded to the block size with the sentinel numel
 * The FP32 sums here are sequential (k ascending, fmaf); the reference's
 * kernels sum in other orders, so sums are pinned to tolerance, as is the
 * SiLU (the C library's expf, not CUDA's).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

enum { DT_BF16 = 0, DT_FP16 = 1 };

static uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

static float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1f;
  const uint32_t man = h & 0x3ff;
  if (exp == 0) {
    const float v = (float)man * 5.9604644775390625e-08f; /* man * 2^-24, exact */
    return sign ? -v : v;
  }
  if (exp == 31) return bits_f32(sign | 0x7f800000u | (man << 13));
  return bits_f32(sign | ((exp + 112) << 23) | (man << 13));
}

static uint16_t f32_to_f16(float f) {
  const uint32_t u = f32_bits(f);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  const uint32_t exp = (u >> 23) & 0xff;
  uint32_t man = u & 0x7fffffu;
  if (exp == 0xff) return sign | 0x7c00u | (man ? 0x200u : 0u);
  const int e = (int)exp - 127;
  if (e > 15) return sign | 0x7c00u;
  if (e >= -14) {
    uint32_t h = ((uint32_t)(e + 15) << 10) | (man >> 13);
    const uint32_t rest = man & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h += 1;
    return sign | (uint16_t)h;
  }
  if (e < -25) return sign;
  man |= 0x800000u;
  const int shift = -e - 1;
  uint32_t h = man >> shift;
  const uint32_t rest = man & ((1u << shift) - 1u);
  const uint32_t half = 1u << (shift - 1);
  if (rest > half || (rest == half && (h & 1u))) h += 1;
  return sign | (uint16_t)h;
}

static float bf16_to_f32(uint16_t b) { return bits_f32((uint32_t)b << 16); }

static uint16_t f32_to_bf16(float f) {
  const uint32_t u = f32_bits(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu)) return (uint16_t)((u >> 16) | 0x40u);
  const uint32_t lsb = (u >> 16) & 1u;
  return (uint16_t)((u + 0x7fffu + lsb) >> 16);
}

static float act_f32(uint16_t v, int dt) { return dt == DT_BF16 ? bf16_to_f32(v) : f16_to_f32(v); }
static uint16_t to_act(float f, int dt) { return dt == DT_BF16 ? f32_to_bf16(f) : f32_to_f16(f); }
static float round_act(float f, int dt) { return act_f32(to_act(f, dt), dt); }

/* ---- layout (decode_orig.cu:10-19) ---------------------------------------- */

/* Nibble i of NVIDIA lane l's word: k offset 2c + kk[i], n offset g + nn[i]
 * (c = l % 4, g = l / 4) inside a 16-row, 16-column block. */
static const int kk[8] = {0, 8, 0, 8, 1, 9, 1, 9};
static const int nn[8] = {0, 0, 8, 8, 0, 0, 8, 8};

/* q [K][N] (values 0..15) from packed int32 [K/16][2N]. */
void oracle_marlin_unpack(const int32_t* w, int64_t K, int64_t N, uint8_t* q) {
  for (int64_t r = 0; r < K / 16; ++r)
    for (int64_t t = 0; t < N / 64; ++t)
      for (int l = 0; l < 32; ++l)
        for (int j = 0; j < 4; ++j) {
          const uint32_t word = (uint32_t)w[r * 2 * N + (t * 32 + l) * 4 + j];
          for (int i = 0; i < 8; ++i) {
            const int64_t k = 16 * r + 2 * (l & 3) + kk[i];
            const int64_t n = 64 * t + 16 * j + (l >> 2) + nn[i];
            q[k * N + n] = (uint8_t)((word >> (4 * i)) & 15u);
          }
        }
}

/* The inverse: packs q [K][N] (values 0..15) into int32 [K/16][2N]. */
void oracle_marlin_pack(const uint8_t* q, int64_t K, int64_t N, int32_t* w) {
  for (int64_t r = 0; r < K / 16; ++r)
    for (int64_t t = 0; t < N / 64; ++t)
      for (int l = 0; l < 32; ++l)
        for (int j = 0; j < 4; ++j) {
          uint32_t word = 0;
          for (int i = 0; i < 8; ++i) {
            const int64_t k = 16 * r + 2 * (l & 3) + kk[i];
            const int64_t n = 64 * t + 16 * j + (l >> 2) + nn[i];
            word |= (uint32_t)(q[k * N + n] & 15u) << (4 * i);
          }
          w[r * 2 * N + (t * 32 + l) * 4 + j] = (int32_t)word;
        }
}

/* Stored position of logical column c of a scale row: inside each 64-column
 * chunk, column c sits at 8 (c % 8) + c / 8. */
int64_t oracle_marlin_scale_pos(int64_t c) { return (c / 64) * 64 + 8 * (c % 8) + (c % 64) / 8; }

/* W [K][N] in the activation dtype: RN((q - 8) * s[k / 128][n]). */
void oracle_marlin_dequant(const int32_t* w, const uint16_t* s, int64_t K, int64_t N, int dt,
                           uint16_t* out) {
  uint8_t* q = (uint8_t*)malloc((size_t)(K * N));
  if (!q) return;
  oracle_marlin_unpack(w, K, N, q);
  for (int64_t k = 0; k < K; ++k)
    for (int64_t n = 0; n < N; ++n) {
      const float sc = act_f32(s[(k / 128) * N + oracle_marlin_scale_pos(n)], dt);
      out[k * N + n] = to_act((float)((int)q[k * N + n] - 8) * sc, dt);
    }
  free(q);
}

static float* dequant_f32(const int32_t* w, const uint16_t* s, int64_t K, int64_t N, int dt) {
  uint16_t* h = (uint16_t*)malloc((size_t)(K * N) * 2);
  float* f = (float*)malloc((size_t)(K * N) * 4);
  if (!h || !f) { free(h); free(f); return NULL; }
  oracle_marlin_dequant(w, s, K, N, dt, h);
  for (int64_t i = 0; i < K * N; ++i) f[i] = act_f32(h[i], dt);
  free(h);
  return f;
}

/* ---- fused MoE --------------------------------------------------------------- */

/* x [M][K] act dtype; ids int32 [M][topk] (an id outside [0, E) routes
 * nowhere: its slot contributes 0); weights fp32 [M][topk];
 * w13 int32 [E][K/16][4N], s13 [E][K/128][2N] (gate columns 0..N-1, up
 * N..2N-1); w2 int32 [E][N/16][2K], s2 [E][N/128][K]; limit: SwiGLU clamp
 * (+inf: none).  out [M][K] act dtype.  Optional h1 [M*topk][2N] and
 * h [M*topk][N] (act dtype) receive the intermediate rows of routed slots.
 * Returns 0, or -1 when out of memory. */
int oracle_marlin_moe(const uint16_t* x, int dt, int64_t M, int64_t K, int64_t N,
                      const int32_t* ids, const float* weights, int64_t topk, int64_t E,
                      const int32_t* w13, const uint16_t* s13, const int32_t* w2,
                      const uint16_t* s2, float limit, uint16_t* out, uint16_t* h1_out,
                      uint16_t* h_out) {
  float** d13 = (float**)calloc((size_t)(E + 1), sizeof(float*));
  float** d2 = (float**)calloc((size_t)(E + 1), sizeof(float*));
  float* xr = (float*)malloc((size_t)K * 4);
  float* h1 = (float*)malloc((size_t)(2 * N) * 4);
  float* h = (float*)malloc((size_t)N * 4);
  float* acc = (float*)malloc((size_t)K * 4);
  float* z = (float*)malloc((size_t)K * 4);
  int rc = -1;
  if (!d13 || !d2 || !xr || !h1 || !h || !acc || !z) goto done;
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t c = 0; c < K; ++c) { xr[c] = act_f32(x[m * K + c], dt); acc[c] = 0.0f; }
    for (int64_t k = 0; k < topk; ++k) {
      const int64_t slot = m * topk + k;
      const int64_t e = ids[slot];
      if (e < 0 || e >= E) continue; /* contributes 0 (acc + 0 == acc) */
      if (!d13[e]) {
        d13[e] = dequant_f32(w13 + e * (K / 16) * 4 * N, s13 + e * (K / 128) * 2 * N, K, 2 * N, dt);
        d2[e] = dequant_f32(w2 + e * (N / 16) * 2 * K, s2 + e * (N / 128) * K, N, K, dt);
        if (!d13[e] || !d2[e]) goto done;
      }
      /* w13: RN(sequential FP32 sum) */
      for (int64_t n = 0; n < 2 * N; ++n) {
        float s = 0.0f;
        for (int64_t c = 0; c < K; ++c) s = fmaf(xr[c], d13[e][c * 2 * N + n], s);
        h1[n] = round_act(s, dt);
        if (h1_out) h1_out[slot * 2 * N + n] = to_act(h1[n], dt);
      }
      /* activation */
      for (int64_t n = 0; n < N; ++n) {
        const float g = fminf(h1[n], limit);
        const float u = fmaxf(fminf(h1[N + n], limit), -limit);
        const float sl = round_act(g / (1.0f + expf(-g)), dt);
        h[n] = round_act(sl * u, dt);
        if (h_out) h_out[slot * N + n] = to_act(h[n], dt);
      }
      /* w2 with the router weight, then the slot-order FP32 sum */
      const float rw = round_act(weights[slot], dt);
      for (int64_t c = 0; c < K; ++c) {
        float s = 0.0f;
        for (int64_t n = 0; n < N; ++n) s = fmaf(h[n], d2[e][n * K + c], s);
        z[c] = round_act(round_act(s, dt) * rw, dt);
        acc[c] = acc[c] + z[c];
      }
    }
    for (int64_t c = 0; c < K; ++c) out[m * K + c] = to_act(acc[c], dt);
  }
  rc = 0;
done:
  if (d13) for (int64_t e = 0; e < E; ++e) free(d13[e]);
  if (d2) for (int64_t e = 0; e < E; ++e) free(d2[e]);
  free(d13); free(d2); free(xr); free(h1); free(h); free(acc); free(z);
  return rc;
}

/* ---- alignment (moe_align_reference.py:18-70) -------------------------------- */

/* ids int32 [numel]; expert_map (NULL: identity) int32 [E]: local id or -1.
 * sorted [sorted_size] (sentinel numel), expert_ids [blocks] (-1 past the
 * padded total), ntpp[0] = padded total.  Returns 0, or -1 if the padded
 * total does not fit sorted_size. */
int oracle_moe_align(const int32_t* ids, int64_t numel, int64_t E, int64_t bs,
                     const int32_t* expert_map, int32_t* sorted, int64_t sorted_size,
                     int32_t* expert_ids, int64_t blocks, int32_t* ntpp) {
  int64_t* count = (int64_t*)calloc((size_t)(E + 1), sizeof(int64_t));
  int64_t* start = (int64_t*)calloc((size_t)(E + 1), sizeof(int64_t));
  if (!count || !start) { free(count); free(start); return -1; }
  for (int64_t i = 0; i < numel; ++i) {
    int64_t e = ids[i];
    if (e < 0 || e >= E) continue;
    if (expert_map) { e = expert_map[e]; if (e < 0) continue; }
    count[e]++;
  }
  int64_t total = 0;
  for (int64_t e = 0; e < E; ++e) {
    start[e] = total;
    total += (count[e] + bs - 1) / bs * bs;
  }
  if (total > sorted_size) { free(count); free(start); return -1; }
  for (int64_t i = 0; i < sorted_size; ++i) sorted[i] = (int32_t)numel;
  for (int64_t e = 0; e < E; ++e) count[e] = 0;
  for (int64_t i = 0; i < numel; ++i) {
    int64_t e = ids[i];
    if (e < 0 || e >= E) continue;
    if (expert_map) { e = expert_map[e]; if (e < 0) continue; }
    sorted[start[e] + count[e]++] = (int32_t)i;
  }
  for (int64_t b = 0; b < blocks; ++b) {
    int32_t owner = -1;
    if (b < total / bs)
      for (int64_t e = 0; e < E; ++e)
        if (start[e] / bs <= b) owner = (int32_t)e;
    expert_ids[b] = owner;
  }
  ntpp[0] = (int32_t)total;
  free(count);
  free(start);
  return 0;
}
