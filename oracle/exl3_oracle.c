/*
 * CPU oracle for the EXL3 quantized-weight path.  TEST INFRASTRUCTURE ONLY:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker.  The product path never calls
 * it and has no CPU fallback.
 *
 * A plain-C restatement of the reference's scalar, bit-exact EXL3 operators.
 * Every arithmetic step is IEEE: FP16 round-to-nearest add/FMA for the
 * codebooks, FP32 round-to-nearest mul/add/fma for the transforms and the
 * sequential k-ordered FMA chain, BF16/FP16 round-to-nearest-even on store.
 * Build flags keep the compiler from contracting or reassociating
 * (-ffp-contract=off, no -ffast-math), so the C operators reproduce those
 * steps exactly.  The one non-IEEE step of the reference is CUDA's expf in
 * the MoE SiLU; this file uses the C library's expf, so MoE outputs are
 * pinned to tolerance only.
 *
 * Reference files followed (paths relative to the reference repository):
 *   csrc/exl3/reference.cu:62-75    codebook_value (mcg / mul1)
 *   csrc/exl3/reference.cu:77-103   core_value (tile ring, window, lane map)
 *   csrc/exl3/reference.cu:107-122  hadamard128 (Sylvester, distances 1..64)
 *   csrc/exl3/reference.cu:124-171  linear_input / linear_core / linear_output
 *   csrc/exl3/reference.cu:173-310  Routing, expert_* kernels, activate, combine
 *   csrc/exl3/reference.cu:315-448  linear_out_reference / moe_out_reference
 *   csrc/exl3/common.h:85-97        swiglu_clamp
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define H128_SCALE 0.08838834764831845f

enum { DT_BF16 = 0, DT_FP16 = 1, DT_FP32 = 2 };

/* ---- scalar conversions (round to nearest even) ------------------------ */

static uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float oracle_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1f;
  const uint32_t man = h & 0x3ff;
  if (exp == 0) {
    /* zero or subnormal: man * 2^-24, exact in FP32 */
    const float v = (float)man * 5.9604644775390625e-08f;
    return sign ? -v : v;
  }
  if (exp == 31) return bits_f32(sign | 0x7f800000u | (man << 13));
  return bits_f32(sign | ((exp + 112) << 23) | (man << 13));
}

uint16_t oracle_f32_to_f16(float f) {
  const uint32_t u = f32_bits(f);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  const uint32_t exp = (u >> 23) & 0xff;
  uint32_t man = u & 0x7fffffu;
  if (exp == 0xff) return sign | 0x7c00u | (man ? 0x200u : 0u);
  const int e = (int)exp - 127;
  if (e > 15) return sign | 0x7c00u;
  if (e >= -14) {
    /* normal half: keep 10 mantissa bits, round the 13 dropped ones */
    uint32_t h = ((uint32_t)(e + 15) << 10) | (man >> 13);
    const uint32_t rest = man & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h += 1; /* may carry to inf */
    return sign | (uint16_t)h;
  }
  if (e < -25) return sign; /* below half the smallest subnormal */
  /* subnormal half: value = m * 2^-24 with m = full_mantissa >> shift */
  man |= 0x800000u;
  const int shift = -e - 1; /* 14 .. 24 */
  uint32_t h = man >> shift;
  const uint32_t rest = man & ((1u << shift) - 1u);
  const uint32_t half = 1u << (shift - 1);
  if (rest > half || (rest == half && (h & 1u))) h += 1;
  return sign | (uint16_t)h;
}

float oracle_bf16_to_f32(uint16_t b) { return bits_f32((uint32_t)b << 16); }

uint16_t oracle_f32_to_bf16(float f) {
  const uint32_t u = f32_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  const uint32_t lsb = (u >> 16) & 1u;
  return (uint16_t)((u + 0x7fffu + lsb) >> 16);
}

static float load_act(const void* p, int dtype, int64_t i) {
  if (dtype == DT_BF16) return oracle_bf16_to_f32(((const uint16_t*)p)[i]);
  if (dtype == DT_FP16) return oracle_f16_to_f32(((const uint16_t*)p)[i]);
  return ((const float*)p)[i];
}
static void store_act(void* p, int dtype, int64_t i, float v) {
  if (dtype == DT_BF16) ((uint16_t*)p)[i] = oracle_f32_to_bf16(v);
  else if (dtype == DT_FP16) ((uint16_t*)p)[i] = oracle_f32_to_f16(v);
  else ((float*)p)[i] = v;
}

/* ---- format ------------------------------------------------------------- */

/* 16-bit trellis state of encoder-order value `index` (0..255) of one tile.
 * The tile is a ring of 128*bits_x2 bits held as 4*bits_x2 uint32 words,
 * word w = halfword 2w (low) | halfword 2w+1 (high), read MSB first.  Value
 * i ends at bit (i+1)*floor(bits_x2/2) (+ floor((i+1)/2) for odd bits_x2);
 * its state is the 16 ring bits before that end, wrapping around the ring.
 * Follows reference.cu:84-101. */
uint32_t oracle_exl3_state(const uint16_t* tile, int bits_x2, int index) {
  const int whole = bits_x2 / 2;
  const int end = (index + 1) * whole + ((bits_x2 & 1) ? (index + 1) / 2 : 0);
  const int ring_bits = 128 * bits_x2;
  const int start = (end - 16 + ring_bits) % ring_bits;
  const int words = ring_bits / 32;
  const int w0 = start / 32;
  const int w1 = (w0 + 1) % words;
  const uint64_t a = (uint64_t)tile[2 * w0] | ((uint64_t)tile[2 * w0 + 1] << 16);
  const uint64_t b = (uint64_t)tile[2 * w1] | ((uint64_t)tile[2 * w1 + 1] << 16);
  const uint64_t window = (a << 32) | b;
  return (uint32_t)((window >> (48 - (start & 31))) & 0xffffu);
}

/* Codebook value of a state as FP16 bits (reference.cu:62-75).
 * codebook 1 (mcg): p = s*0xCBAC1FED; m = (p & 0x8fff8fff) ^ 0x3b603b60;
 *   value = RN16(half(m.lo) + half(m.hi)).
 * codebook 2 (mul1): p = s*0x83DCD12D; t = sum of the 4 bytes of p;
 *   value = RN16(half(0x6400 + t) * half(0x1eee) + half(0xc931)).
 * Both exact sums/products fit FP32 (operands are FP16 with bounded
 * exponents), so one FP32 evaluation followed by one RN16 is the FP16 op. */
uint16_t oracle_exl3_codebook(uint32_t state, int codebook) {
  if (codebook == 1) {
    uint32_t p = state * 0xCBAC1FEDu;
    p = (p & 0x8fff8fffu) ^ 0x3b603b60u;
    const float lo = oracle_f16_to_f32((uint16_t)(p & 0xffffu));
    const float hi = oracle_f16_to_f32((uint16_t)(p >> 16));
    return oracle_f32_to_f16(lo + hi);
  }
  const uint32_t p = state * 0x83DCD12Du;
  const uint32_t t = (p & 255u) + ((p >> 8) & 255u) + ((p >> 16) & 255u) + (p >> 24);
  const float base = oracle_f16_to_f32((uint16_t)(0x6400u + t));
  const float scale = oracle_f16_to_f32(0x1eeeu);
  const float bias = oracle_f16_to_f32(0xc931u);
  return oracle_f32_to_f16(fmaf(base, scale, bias));
}

/* Tile row / column of encoder-order value i = 8*L + j (reference.cu:79-83
 * inverted; codec.cuh:175-180). */
static int lane_row(int i) { const int L = i >> 3, j = i & 7; return 2 * (L & 3) + (j & 1) + 8 * ((j >> 1) & 1); }
static int lane_col(int i) { const int L = i >> 3, j = i & 7; return (L >> 2) + 8 * (j >> 2); }

int oracle_exl3_lane_row(int i) { return lane_row(i); }
int oracle_exl3_lane_col(int i) { return lane_col(i); }

/* Decodes every tile: w[k][n] (FP16 bits), k < 16*tiles_k, n < 16*tiles_n.
 * Tile (tr, tc) is trellis element tr*tiles_n + tc, 8*bits_x2 halfwords. */
void oracle_exl3_decode(const uint16_t* trellis, int64_t tiles_k, int64_t tiles_n,
                        int bits_x2, int codebook, uint16_t* w) {
  const int64_t n_cols = 16 * tiles_n;
  for (int64_t tr = 0; tr < tiles_k; ++tr) {
    for (int64_t tc = 0; tc < tiles_n; ++tc) {
      const uint16_t* tile = trellis + (tr * tiles_n + tc) * (8 * bits_x2);
      for (int i = 0; i < 256; ++i) {
        const uint16_t v = oracle_exl3_codebook(oracle_exl3_state(tile, bits_x2, i), codebook);
        w[(tr * 16 + lane_row(i)) * n_cols + tc * 16 + lane_col(i)] = v;
      }
    }
  }
}

/* H128 over 128 consecutive floats (reference.cu:107-122): for distance
 * 1, 2, ..., 64 in order, lower <- lo + hi, upper <- lo - hi (FP32 RN), then
 * every element times 1/sqrt(128) rounded to FP32. */
void oracle_exl3_h128(float* v) {
  for (int d = 1; d < 128; d <<= 1) {
    for (int i = 0; i < 128; ++i) {
      if (i & d) continue;
      const float lo = v[i], hi = v[i + d];
      v[i] = lo + hi;
      v[i + d] = lo - hi;
    }
  }
  for (int i = 0; i < 128; ++i) v[i] = v[i] * H128_SCALE;
}

/* ---- dense linear (reference.cu:124-171, :315-367) --------------------- */

static float* decode_f32(const uint16_t* trellis, int64_t pin, int64_t pout, int bits_x2,
                         int codebook) {
  const int64_t n = pin * pout;
  uint16_t* h = (uint16_t*)malloc((size_t)n * 2);
  float* w = (float*)malloc((size_t)n * 4);
  if (!h || !w) { free(h); free(w); return NULL; }
  oracle_exl3_decode(trellis, pin / 16, pout / 16, bits_x2, codebook, h);
  for (int64_t i = 0; i < n; ++i) w[i] = oracle_f16_to_f32(h[i]);
  free(h);
  return w;
}

/* core[n] = chain over k = 0..K-1 of fmaf(t[k], W[k][n], sum) from 0.0f */
static void core_rows(const float* t, const float* w, int64_t pin, int64_t pout, float* out) {
  for (int64_t n = 0; n < pout; ++n) out[n] = 0.0f;
  for (int64_t k = 0; k < pin; ++k) {
    const float a = t[k];
    const float* row = w + k * pout;
    for (int64_t n = 0; n < pout; ++n) out[n] = fmaf(a, row[n], out[n]);
  }
}

/* The reference linear: out[r][n] = RN_out(H128(core)[n] * svh[n]) with
 * core = chain(H128(x * suh)).  x_dtype/out_dtype: 0 bf16, 1 fp16, 2 fp32.
 * core_out (optional): the FP32 core rows [rows][pout].  Returns 0 or -1. */
int oracle_exl3_linear_out(const void* x, int x_dtype, int64_t rows, int64_t logical_in,
                           const uint16_t* trellis, const uint16_t* suh, const uint16_t* svh,
                           int64_t pin, int64_t pout, int bits_x2, int codebook,
                           int64_t logical_out, void* out, int out_dtype, float* core_out) {
  float* w = decode_f32(trellis, pin, pout, bits_x2, codebook);
  float* t = (float*)malloc((size_t)pin * 4);
  float* c = (float*)malloc((size_t)pout * 4);
  if (!w || !t || !c) { free(w); free(t); free(c); return -1; }
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t k = 0; k < pin; ++k) {
      t[k] = k < logical_in ? load_act(x, x_dtype, r * logical_in + k) * oracle_f16_to_f32(suh[k])
                            : 0.0f;
    }
    for (int64_t b = 0; b < pin; b += 128) oracle_exl3_h128(t + b);
    core_rows(t, w, pin, pout, c);
    if (core_out) memcpy(core_out + r * pout, c, (size_t)pout * 4);
    for (int64_t b = 0; b < pout; b += 128) oracle_exl3_h128(c + b);
    for (int64_t n = 0; n < logical_out; ++n) {
      store_act(out, out_dtype, r * logical_out + n, c[n] * oracle_f16_to_f32(svh[n]));
    }
  }
  free(w); free(t); free(c);
  return 0;
}

/* ---- routed-expert MoE (reference.cu:173-310, :371-448) ---------------- */

/* One projection of one local expert, as packed_ptrs/packed_meta hold it:
 * ptrs [E][3][3] = {trellis, suh, svh} host addresses, meta [E][3][4] =
 * {padded_in, padded_out, bits_x2, codebook}. */
typedef struct {
  const uint16_t* trellis;
  const uint16_t* suh;
  const uint16_t* svh;
  int64_t pin, pout;
  int bits_x2, codebook;
} proj_t;

static proj_t expert_proj(const int64_t* ptrs, const int64_t* meta, int64_t e, int p) {
  proj_t m;
  const int64_t* pp = ptrs + e * 9 + p * 3;
  const int64_t* mm = meta + e * 12 + p * 4;
  m.trellis = (const uint16_t*)(intptr_t)pp[0];
  m.suh = (const uint16_t*)(intptr_t)pp[1];
  m.svh = (const uint16_t*)(intptr_t)pp[2];
  m.pin = mm[0]; m.pout = mm[1];
  m.bits_x2 = (int)mm[2]; m.codebook = (int)mm[3];
  return m;
}

static int64_t local_of(const int64_t* ids, int64_t a, const int64_t* map, int64_t global,
                        int64_t local) {
  const int64_t g = ids[a];
  if (g < 0 || g >= global) return -1;
  const int64_t l = map[g];
  return (l >= 0 && l < local) ? l : -1;
}

/* Core of one assignment against a projection, reducing over kpad inputs
 * and producing npad outputs, decoding with the projection's own geometry
 * (reference.cu:213-238: "use actual metadata strides"). */
static void expert_core_row(const float* in, const float* w, const proj_t* m, int64_t kpad,
                            int64_t npad, float* out) {
  for (int64_t n = 0; n < npad; ++n) out[n] = 0.0f;
  for (int64_t k = 0; k < kpad; ++k) {
    const float a = in[k];
    const float* row = w + k * m->pout;
    for (int64_t n = 0; n < npad; ++n) out[n] = fmaf(a, row[n], out[n]);
  }
}

/* moe_out_reference.  ids int64 [rows][topk] (global ids, -1 masked),
 * weights fp32 [rows][topk], expert_map int64 [global] (-1: not local).
 * x/out dtype as in linear.  limit: swiglu clamp (0 = none).
 * Returns 0 or -1 on allocation failure. */
int oracle_exl3_moe_out(const void* x, int x_dtype, int64_t rows, int64_t hidden,
                        const int64_t* ids, const float* weights, int64_t topk,
                        const int64_t* ptrs, const int64_t* meta, int64_t local_experts,
                        const int64_t* expert_map, int64_t global_experts,
                        int64_t intermediate, float limit, void* out, int out_dtype) {
  const int64_t hpad = (hidden + 127) / 128 * 128;
  const int64_t ipad = (intermediate + 127) / 128 * 128;
  const int64_t assignments = rows * topk;
  float** wdec = (float**)calloc((size_t)(local_experts * 3 + 1), sizeof(float*));
  /* in holds an expert input (hpad) and later the down input (ipad) */
  float* in = (float*)malloc((size_t)(hpad > ipad ? hpad : ipad) * 4);
  float* gate = (float*)malloc((size_t)ipad * 4);
  float* up = (float*)malloc((size_t)ipad * 4);
  float* down = (float*)malloc((size_t)(assignments ? assignments : 1) * hpad * 4);
  int rc = -1;
  if (!wdec || !in || !gate || !up || !down) goto done;
  for (int64_t a = 0; a < assignments; ++a) {
    float* dn = down + a * hpad;
    const int64_t e = local_experts > 0
        ? local_of(ids, a, expert_map, global_experts, local_experts) : -1;
    if (e < 0) { for (int64_t c = 0; c < hpad; ++c) dn[c] = 0.0f; continue; }
    for (int p = 0; p < 3; ++p) {
      if (!wdec[e * 3 + p]) {
        const proj_t m = expert_proj(ptrs, meta, e, p);
        wdec[e * 3 + p] = decode_f32(m.trellis, m.pin, m.pout, m.bits_x2, m.codebook);
        if (!wdec[e * 3 + p]) goto done;
      }
    }
    const int64_t r = a / topk;
    float* res[2] = {gate, up};
    for (int p = 0; p < 2; ++p) {
      const proj_t m = expert_proj(ptrs, meta, e, p);
      /* expert_input: H128(x * suh) over hpad */
      for (int64_t c = 0; c < hpad; ++c)
        in[c] = c < hidden ? load_act(x, x_dtype, r * hidden + c) * oracle_f16_to_f32(m.suh[c]) : 0.0f;
      for (int64_t b = 0; b < hpad; b += 128) oracle_exl3_h128(in + b);
      /* expert_core + expert_output: H128(core) * svh */
      expert_core_row(in, wdec[e * 3 + p], &m, hpad, ipad, res[p]);
      for (int64_t b = 0; b < ipad; b += 128) oracle_exl3_h128(res[p] + b);
      for (int64_t c = 0; c < ipad; ++c) res[p][c] = res[p][c] * oracle_f16_to_f32(m.svh[c]);
    }
    /* activate_down_input: clamp, SiLU(g) * u * suh_down, H128 */
    const proj_t md = expert_proj(ptrs, meta, e, 2);
    for (int64_t c = 0; c < ipad; ++c) {
      float v = 0.0f;
      if (c < intermediate) {
        float g = gate[c], u = up[c];
        if (limit > 0.0f) { g = fminf(g, limit); u = fminf(fmaxf(u, -limit), limit); }
        const float silu = g / (1.0f + expf(-g));
        v = (silu * u) * oracle_f16_to_f32(md.suh[c]);
      }
      in[c] = v;
    }
    for (int64_t b = 0; b < ipad; b += 128) oracle_exl3_h128(in + b);
    expert_core_row(in, wdec[e * 3 + 2], &md, ipad, hpad, dn);
    for (int64_t b = 0; b < hpad; b += 128) oracle_exl3_h128(dn + b);
    for (int64_t c = 0; c < hpad; ++c) dn[c] = dn[c] * oracle_f16_to_f32(md.svh[c]);
  }
  /* combine_routes: one FMA per local route, route order */
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t c = 0; c < hidden; ++c) {
      float sum = 0.0f;
      for (int64_t k = 0; k < topk; ++k) {
        const int64_t a = r * topk + k;
        if (local_experts > 0 && local_of(ids, a, expert_map, global_experts, local_experts) >= 0)
          sum = fmaf(down[a * hpad + c], weights[a], sum);
      }
      store_act(out, out_dtype, r * hidden + c, sum);
    }
  }
  rc = 0;
done:
  if (wdec) { for (int64_t i = 0; i < local_experts * 3; ++i) free(wdec[i]); }
  free(wdec); free(in); free(gate); free(up); free(down);
  return rc;
}
