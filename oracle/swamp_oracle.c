/*
 * swamp_oracle.c -- CPU oracle for the quantized-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY (see swamp_oracle.h).  A plain-C restatement of
 * the reference's scalar Rust code; every function cites what it follows.
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, no fast-math).
 */
#include "swamp_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#if defined(__x86_64__)
#include <immintrin.h>
#endif

/* ---------------------------------------------------------------------- */
/* GgmlDType table: swamp-gguf/src/dtype.rs:79-139                         */
/* ---------------------------------------------------------------------- */

size_t or_block_size(uint32_t dt) {
  switch (dt) {
  case 0: case 1: case 30: case 24: case 25: case 26: case 27: case 28:
    return 1; /* F32 F16 BF16 I8 I16 I32 I64 F64, dtype.rs:81 */
  case 2: case 3: case 6: case 7: case 8: case 9:
    return 32; /* Q4_0 Q4_1 Q5_0 Q5_1 Q8_0 Q8_1, dtype.rs:82 */
  case 10: case 11: case 12: case 13: case 14: case 15:
    return 256; /* K-quants, dtype.rs:83 */
  case 16: case 17: case 22: case 18: case 21: case 19: case 29:
    return 256; /* IQ2_*, IQ3_*, IQ1_*, dtype.rs:84-87 */
  case 20: case 23:
    return 32; /* IQ4_NL, IQ4_XS, dtype.rs:86 */
  default:
    return 0;
  }
}

size_t or_type_size(uint32_t dt) {
  switch (dt) { /* dtype.rs:92-132 */
  case 0: return 4;   case 1: return 2;   case 30: return 2;  case 28: return 8;
  case 24: return 1;  case 25: return 2;  case 26: return 4;  case 27: return 8;
  case 2: return 18;  case 3: return 20;  case 6: return 22;  case 7: return 24;
  case 8: return 34;  case 9: return 40;  case 10: return 84; case 11: return 110;
  case 12: return 144; case 13: return 176; case 14: return 210; case 15: return 292;
  case 16: return 66; case 17: return 74; case 22: return 82; case 18: return 98;
  case 21: return 110; case 20: return 18; case 23: return 136; case 19: return 50;
  case 29: return 56;
  default: return 0;
  }
}

size_t or_nbytes_for(uint32_t dt, size_t n) { /* dtype.rs:135-139 */
  size_t bs = or_block_size(dt);
  if (bs == 0) return 0;
  return (n + bs - 1) / bs * or_type_size(dt);
}

/* ---------------------------------------------------------------------- */
/* half 2.7.1 conversions                                                  */
/* ---------------------------------------------------------------------- */

static float bits_f32(uint32_t b) {
  float f;
  memcpy(&f, &b, 4);
  return f;
}

/* binary16 -> binary32, exact.  Subnormals are renormalised; inf keeps its
 * sign; NaN keeps sign and payload and gets the quiet bit (half's software
 * path and the x86 F16C instruction agree on this). */
float or_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1Fu;
  uint32_t man = h & 0x3FFu;
  if (exp == 0) {
    if (man == 0) return bits_f32(sign);
    int e = -1;
    do {
      e++;
      man <<= 1;
    } while (!(man & 0x400u));
    return bits_f32(sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3FFu) << 13));
  }
  if (exp == 31) {
    if (man == 0) return bits_f32(sign | 0x7F800000u);
    return bits_f32(sign | 0x7FC00000u | (man << 13));
  }
  return bits_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

void or_f16_to_f32_array(const uint16_t *h, float *out, size_t n) {
  for (size_t i = 0; i < n; i++) out[i] = or_f16_to_f32(h[i]);
}

#if defined(__x86_64__)
__attribute__((target("f16c"))) static void f16c_convert(const uint16_t *h,
                                                         float *out, size_t n) {
  for (size_t i = 0; i < n; i++) out[i] = _cvtsh_ss(h[i]);
}
#endif

int or_f16_to_f32_hw_array(const uint16_t *h, float *out, size_t n) {
#if defined(__x86_64__)
  __builtin_cpu_init();
  if (!__builtin_cpu_supports("f16c")) return -1;
  f16c_convert(h, out, n);
  return 0;
#else
  (void)h; (void)out; (void)n;
  return -1;
#endif
}

float or_bf16_to_f32(uint16_t h) { return bits_f32((uint32_t)h << 16); }

static inline float f16_le(const uint8_t *p) {
  return or_f16_to_f32((uint16_t)(p[0] | ((uint16_t)p[1] << 8)));
}

/* ---------------------------------------------------------------------- */
/* Dequantizers                                                            */
/* ---------------------------------------------------------------------- */

/* q4_0::dequant, swamp-gguf/src/quant/q4_0.rs:11-39.  Element i of a block
 * is byte i/2 of the 16 nibble bytes, LOW nibble when i is even (:30-35). */
int or_dequant_q4_0(const uint8_t *raw, size_t raw_len, float *dst, size_t n) {
  size_t n_blocks = (n + 31) / 32;
  if (raw_len < n_blocks * 18) return -1; /* BufferTooSmall, :15-20 */
  for (size_t b = 0; b < n_blocks; b++) {
    const uint8_t *base = raw + b * 18;
    float scale = f16_le(base);
    const uint8_t *nib = base + 2;
    size_t s = b * 32, e = s + 32 < n ? s + 32 : n;
    for (size_t i = 0; i < e - s; i++) {
      uint8_t byte = nib[i / 2];
      uint8_t q = (i % 2 == 0) ? (byte & 0x0F) : (byte >> 4);
      int32_t v = (int32_t)q - 8;
      dst[s + i] = (float)v * scale;
    }
  }
  return 0;
}

/* q8_0::dequant scalar arm, q8_0.rs:15-40 + :127-139 (the AVX arms at
 * :48-125 compute the same single product per element). */
int or_dequant_q8_0(const uint8_t *raw, size_t raw_len, float *dst, size_t n) {
  size_t n_blocks = (n + 31) / 32;
  if (raw_len < n_blocks * 34) return -1; /* :19-24 */
  for (size_t b = 0; b < n_blocks; b++) {
    const uint8_t *base = raw + b * 34;
    float scale = f16_le(base);
    const int8_t *qs = (const int8_t *)(base + 2);
    size_t s = b * 32, e = s + 32 < n ? s + 32 : n;
    for (size_t i = 0; i < e - s; i++) dst[s + i] = (float)qs[i] * scale;
  }
  return 0;
}

/* q4_k::unpack_scales, q4_k.rs:37-53 (identical to fused_gemv_q4k.rs:30-43) */
void or_unpack_scales_q4k(const uint8_t sc[12], uint8_t scales[8],
                          uint8_t mins[8]) {
  for (int j = 0; j < 4; j++) {
    scales[j] = sc[j] & 63;
    mins[j] = sc[j + 4] & 63;
  }
  for (int j = 4; j < 8; j++) {
    scales[j] = (uint8_t)((sc[j + 4] & 0xF) | ((sc[j - 4] >> 6) << 4));
    mins[j] = (uint8_t)((sc[j + 4] >> 4) | ((sc[j] >> 6) << 4));
  }
}

/* q4_k::dequant_q4k -> dequant_scalar, q4_k.rs:21-33 + :278-321 (layout A:
 * pair p uses qs[32p..32p+32]; low nibble -> sub-block 2p, high nibble ->
 * sub-block 2p+1).  w = (d*sc)*q - (dmin*m), each product and the
 * difference rounded separately (no FMA contraction). */
int or_dequant_q4_k(const uint8_t *raw, size_t raw_len, float *dst, size_t n) {
  size_t n_blocks = (n + 255) / 256;
  if (raw_len < n_blocks * 144) return -1; /* :25-30 */
  for (size_t b = 0; b < n_blocks; b++) {
    const uint8_t *base = raw + b * 144;
    float d = f16_le(base);
    float dmin = f16_le(base + 2);
    uint8_t scales[8], mins[8];
    or_unpack_scales_q4k(base + 4, scales, mins);
    const uint8_t *qs = base + 16;
    size_t out_start = b * 256;
    size_t out_end = out_start + 256 < n ? out_start + 256 : n;
    for (int pair = 0; pair < 4; pair++) {
      const uint8_t *q = qs + pair * 32;
      int se = pair * 2, so = pair * 2 + 1;
      float scale_e = d * (float)(scales[se] & 0x3F);
      float min_e = dmin * (float)(mins[se] & 0x3F);
      for (int i = 0; i < 32; i++) {
        size_t g = out_start + (size_t)se * 32 + i;
        if (g < out_end) {
          float t = scale_e * (float)(q[i] & 0x0F);
          dst[g] = t - min_e;
        }
      }
      float scale_o = d * (float)(scales[so] & 0x3F);
      float min_o = dmin * (float)(mins[so] & 0x3F);
      for (int i = 0; i < 32; i++) {
        size_t g = out_start + (size_t)so * 32 + i;
        if (g < out_end) {
          float t = scale_o * (float)(q[i] >> 4);
          dst[g] = t - min_o;
        }
      }
    }
  }
  return 0;
}

/* q6_k::dequant_q6k, swamp-gguf/src/quant/q6_k.rs:7-56.  A 256-weight
 * block is 210 bytes: ql[128], qh[64], int8 sc[16], f16 d (:25-28).  Two
 * halves of 128 outputs; in a half, l < 32 gives outputs l, l+32, l+64,
 * l+96 from the low nibble of ql[l], the low nibble of ql[l+32], the high
 * nibble of ql[l], the high nibble of ql[l+32], each with the next 2-bit
 * field of qh[l] as bits 4-5 (:36-39); value (d * sc[l/16 + 2j]) * (q - 32)
 * (:41-44), then ql += 64, qh += 32, sc += 8 (:47-49).  The last block may
 * be partial (:52-54). */
int or_dequant_q6_k(const uint8_t *raw, size_t raw_len, float *dst, size_t n) {
  size_t n_blocks = (n + 255) / 256;
  if (raw_len < n_blocks * 210) return -1; /* BufferTooSmall, :11-16 */
  for (size_t b = 0; b < n_blocks; b++) {
    const uint8_t *ql = raw + b * 210;
    const uint8_t *qh = ql + 128;
    const int8_t *sc = (const int8_t *)(ql + 192);
    float d = f16_le(ql + 208);
    float y[256];
    for (int h = 0; h < 2; h++) {
      for (int l = 0; l < 32; l++) {
        int is = l / 16;
        int q1 = (int)((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32;
        int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
        int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
        int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
        y[128 * h + l] = d * (float)sc[is] * (float)q1;
        y[128 * h + l + 32] = d * (float)sc[is + 2] * (float)q2;
        y[128 * h + l + 64] = d * (float)sc[is + 4] * (float)q3;
        y[128 * h + l + 96] = d * (float)sc[is + 6] * (float)q4;
      }
      ql += 64;
      qh += 32;
      sc += 8;
    }
    size_t start = b * 256;
    size_t count = n - start < 256 ? n - start : 256;
    memcpy(dst + start, y, count * sizeof(float));
  }
  return 0;
}

/* swamp-gguf/src/quant/mod.rs:18-33 (+ dequant_f32 :35-44, f16.rs:6-28) */
int or_dequantize(uint32_t dtype, const uint8_t *raw, size_t raw_len,
                  float *dst, size_t n) {
  switch (dtype) {
  case 0:
    if (raw_len < n * 4) return -1;
    memcpy(dst, raw, n * 4);
    return 0;
  case 1:
    if (raw_len < n * 2) return -1;
    for (size_t i = 0; i < n; i++) dst[i] = f16_le(raw + 2 * i);
    return 0;
  case 30:
    if (raw_len < n * 2) return -1;
    for (size_t i = 0; i < n; i++)
      dst[i] = or_bf16_to_f32((uint16_t)(raw[2 * i] | ((uint16_t)raw[2 * i + 1] << 8)));
    return 0;
  case 2: return or_dequant_q4_0(raw, raw_len, dst, n);
  case 8: return or_dequant_q8_0(raw, raw_len, dst, n);
  case 12: return or_dequant_q4_k(raw, raw_len, dst, n);
  case 14: return or_dequant_q6_k(raw, raw_len, dst, n);
  default: return -2; /* other dtypes are off this path */
  }
}

/* ---------------------------------------------------------------------- */
/* Q4_K fused GEMV (scalar), batched, multi                                */
/* ---------------------------------------------------------------------- */

/* One Q4_K block against 256 x values, accumulating into acc in the exact
 * order of fused_gemv_q4k.rs:484-504: pairs 0..3, even sub-block (low
 * nibbles) then odd sub-block (high nibbles), i = 0..31 each. */
static float q4k_block_dot(const uint8_t *base, const float *x_blk, float acc) {
  float d = f16_le(base);
  float dmin = f16_le(base + 2);
  uint8_t scales[8], mins[8];
  or_unpack_scales_q4k(base + 4, scales, mins);
  const uint8_t *qs = base + 16;
  for (int pair = 0; pair < 4; pair++) {
    const uint8_t *q = qs + pair * 32;
    int se = pair * 2, so = pair * 2 + 1;
    float sv_e = d * (float)(scales[se] & 0x3F);
    float mv_e = dmin * (float)(mins[se] & 0x3F);
    for (int i = 0; i < 32; i++) {
      float t = sv_e * (float)(q[i] & 0x0F);
      float w = t - mv_e;
      float p = w * x_blk[se * 32 + i];
      acc = acc + p;
    }
    float sv_o = d * (float)(scales[so] & 0x3F);
    float mv_o = dmin * (float)(mins[so] & 0x3F);
    for (int i = 0; i < 32; i++) {
      float t = sv_o * (float)(q[i] >> 4);
      float w = t - mv_o;
      float p = w * x_blk[so * 32 + i];
      acc = acc + p;
    }
  }
  return acc;
}

/* fused_gemv_q4k_scalar, fused_gemv_q4k.rs:466-508 */
static void q4k_scalar(const uint8_t *w, const float *x, float *out,
                       size_t n_rows, size_t n_blocks) {
  for (size_t row = 0; row < n_rows; row++) {
    float acc = 0.0f;
    for (size_t blk = 0; blk < n_blocks; blk++)
      acc = q4k_block_dot(w + (row * n_blocks + blk) * 144, x + blk * 256, acc);
    out[row] = acc;
  }
}

/* fused_gemv_q4k asserts (:66-70) then the scalar arm (:81) */
int or_fused_gemv_q4k(const uint8_t *w_raw, size_t w_len, const float *x,
                      size_t x_len, float *out, size_t out_len, size_t n_rows,
                      size_t n_cols) {
  if (n_cols % 256 != 0) return -1;
  size_t nb = n_cols / 256;
  if (w_len != n_rows * nb * 144) return -1;
  if (x_len != n_cols) return -1;
  if (out_len < n_rows) return -1;
  q4k_scalar(w_raw, x, out, n_rows, nb);
  return 0;
}

/* batched_scalar, fused_gemv_q4k.rs:650-698 (block -> row -> token, each
 * (row, token) partial starts at 0 and is ADDED to out, :694). */
int or_fused_gemv_q4k_batched(const uint8_t *w_raw, const float *const *x_ptrs,
                              float *const *out_ptrs, size_t n_rows,
                              size_t n_cols, size_t batch) {
  if (n_cols % 256 != 0) return -1;
  size_t nb = n_cols / 256;
  for (size_t blk = 0; blk < nb; blk++) {
    for (size_t row = 0; row < n_rows; row++) {
      const uint8_t *base = w_raw + (row * nb + blk) * 144;
      for (size_t t = 0; t < batch; t++) {
        float acc = q4k_block_dot(base, x_ptrs[t] + blk * 256, 0.0f);
        out_ptrs[t][row] += acc;
      }
    }
  }
  return 0;
}

/* fused_gemv_q4k_multi, fused_gemv_q4k.rs:401-460: zero every output, then
 * block-outer; acc starts from out[row] so each row sums block after block
 * in the same order as the scalar GEMV. */
int or_fused_gemv_q4k_multi(const uint8_t *const *raws, const float *x,
                            float *const *outputs, const size_t *row_counts,
                            size_t n_mats, size_t n_cols) {
  if (n_cols % 256 != 0) return -1;
  size_t nb = n_cols / 256;
  for (size_t m = 0; m < n_mats; m++)
    memset(outputs[m], 0, row_counts[m] * sizeof(float));
  for (size_t blk = 0; blk < nb; blk++)
    for (size_t m = 0; m < n_mats; m++)
      for (size_t row = 0; row < row_counts[m]; row++) {
        float acc = outputs[m][row];
        acc = q4k_block_dot(raws[m] + (row * nb + blk) * 144, x + blk * 256, acc);
        outputs[m][row] = acc;
      }
  return 0;
}

/* ---------------------------------------------------------------------- */
/* Q6_K fused GEMV (scalar)                                                */
/* ---------------------------------------------------------------------- */

/* f16_to_f32_raw, swamp-kernels/src/fused_gemv_q6k.rs:11-21: the fused Q6_K
 * kernels' private decode of d.  It equals or_f16_to_f32 for exponent
 * fields 1..30.  Exponent 0 (zero and subnormal codes) gives
 * sign | ((1023 - 14) << 23 wrapped to 32 bits = 0xF8800000) | man << 13, a
 * negative value near -2^114; exponent 31 (inf, NaN) decodes as the finite
 * 2^16 * (1 + man/1024). */
float or_q6k_f16_raw(uint16_t v) {
  uint32_t sign = (uint32_t)(v >> 15) << 31;
  uint32_t exp = (v >> 10) & 0x1Fu;
  uint32_t man = v & 0x3FFu;
  if (exp == 0) return bits_f32(sign | (1009u << 23) | (man << 13));
  return bits_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

/* One Q6_K block against 256 x values in the order of the scalar kernel,
 * fused_gemv_q6k.rs:253-286: half 0..1, l = 0..31, then the four terms
 * ((d * sc) * q) * x[l + 32j] for j = 0..3, each added to acc.  Scales are
 * int8 (:277-280).  d is decoded exactly (half::f16, as the dequantizer
 * q6_k.rs:28 does), not with f16_to_f32_raw: the two agree on every code
 * with exponent field 1..30. */
static float q6k_block_dot(const uint8_t *base, const float *x_blk, float acc) {
  float d = f16_le(base + 208);
  const uint8_t *ql = base, *qh = base + 128;
  const int8_t *sc = (const int8_t *)(base + 192);
  for (int h = 0; h < 2; h++) {
    const uint8_t *ql_h = ql + 64 * h, *qh_h = qh + 32 * h;
    const int8_t *sc_h = sc + 8 * h;
    const float *xh = x_blk + 128 * h;
    for (int l = 0; l < 32; l++) {
      int is = l / 16;
      float q1 = (float)((int)((ql_h[l] & 0x0F) | ((qh_h[l] & 3) << 4)) - 32);
      float q2 = (float)((int)((ql_h[l + 32] & 0x0F) | (((qh_h[l] >> 2) & 3) << 4)) - 32);
      float q3 = (float)((int)((ql_h[l] >> 4) | (((qh_h[l] >> 4) & 3) << 4)) - 32);
      float q4 = (float)((int)((ql_h[l + 32] >> 4) | (((qh_h[l] >> 6) & 3) << 4)) - 32);
      acc = acc + d * (float)sc_h[is] * q1 * xh[l];
      acc = acc + d * (float)sc_h[is + 2] * q2 * xh[l + 32];
      acc = acc + d * (float)sc_h[is + 4] * q3 * xh[l + 64];
      acc = acc + d * (float)sc_h[is + 6] * q4 * xh[l + 96];
    }
  }
  return acc;
}

/* fused_gemv_q6k_scalar, fused_gemv_q6k.rs:248-291 (one f32 accumulator per
 * row, block after block; overwrites out[row]). */
static void q6k_scalar(const uint8_t *w, const float *x, float *out,
                       size_t n_rows, size_t n_blocks) {
  for (size_t row = 0; row < n_rows; row++) {
    float acc = 0.0f;
    for (size_t blk = 0; blk < n_blocks; blk++)
      acc = q6k_block_dot(w + (row * n_blocks + blk) * 210, x + blk * 256, acc);
    out[row] = acc;
  }
}

int or_fused_gemv_q6k(const uint8_t *w_raw, size_t w_len, const float *x,
                      size_t x_len, float *out, size_t out_len, size_t n_rows,
                      size_t n_cols) {
  if (n_cols % 256 != 0) return -1;
  size_t nb = n_cols / 256;
  if (w_len < n_rows * nb * 210) return -1;
  if (x_len < n_cols) return -1;
  if (out_len < n_rows) return -1;
  q6k_scalar(w_raw, x, out, n_rows, nb);
  return 0;
}

/* ---------------------------------------------------------------------- */
/* forward_linear and friends (row-partitioned worker threads)             */
/* ---------------------------------------------------------------------- */

typedef struct {
  int kind; /* 0 = Q4_K fused, 1 = dense f32 dot over deq, 2 = Q6_K fused,
               3 = Q4_K batched (bs tokens) */
  const uint8_t *raw;
  const float *deq;
  const float *x;
  float *out;
  size_t nc, rs, re;
  const float *const *xp; /* kind 3: token inputs */
  float *const *op;       /* kind 3: token outputs (whole rows) */
  size_t bs;
} slice_job;

static void run_slice(const slice_job *j) {
  if (j->rs >= j->re) return;
  size_t rc = j->re - j->rs;
  if (j->kind == 0) {
    size_t nb = j->nc / 256;
    q4k_scalar(j->raw + j->rs * nb * 144, j->x, j->out + j->rs, rc, nb);
  } else if (j->kind == 2) {
    size_t nb = j->nc / 256;
    q6k_scalar(j->raw + j->rs * nb * 210, j->x, j->out + j->rs, rc, nb);
  } else if (j->kind == 3) {
    /* linear.rs:215-233: the slice's rows of every token output */
    size_t nb = j->nc / 256;
    float **op = (float **)malloc(j->bs * sizeof(float *));
    if (!op) return;
    for (size_t t = 0; t < j->bs; t++) op[t] = j->op[t] + j->rs;
    or_fused_gemv_q4k_batched(j->raw + j->rs * nb * 144, j->xp, op, rc, j->nc, j->bs);
    free(op);
  } else {
    /* linear.rs:81-85: s += deq[i*nc+j] * x[j], sequential f32 */
    for (size_t i = 0; i < rc; i++) {
      const float *row = j->deq + (j->rs + i) * j->nc;
      float s = 0.0f;
      for (size_t k = 0; k < j->nc; k++) {
        float p = row[k] * j->x[k];
        s = s + p;
      }
      j->out[j->rs + i] = s;
    }
  }
}

static void *slice_thread(void *arg) {
  run_slice((const slice_job *)arg);
  return NULL;
}

/* rayon partition of linear.rs:31-45 / :73-87: thread t owns rows
 * [t*rpt, min(t*rpt+rpt, nr)) with rpt = ceil(nr/nt). */
static int run_partitioned(slice_job proto, size_t nr, int n_threads) {
  if (n_threads < 1) n_threads = 1;
  size_t nt = (size_t)n_threads;
  size_t rpt = (nr + nt - 1) / nt;
  slice_job *jobs = (slice_job *)calloc(nt, sizeof(slice_job));
  pthread_t *th = (pthread_t *)calloc(nt, sizeof(pthread_t));
  int *started = (int *)calloc(nt, sizeof(int));
  if (!jobs || !th || !started) {
    free(jobs); free(th); free(started);
    return -3;
  }
  for (size_t t = 0; t < nt; t++) {
    jobs[t] = proto;
    jobs[t].rs = t * rpt < nr ? t * rpt : nr;
    jobs[t].re = t * rpt + rpt < nr ? t * rpt + rpt : nr;
  }
  for (size_t t = 1; t < nt; t++)
    started[t] = pthread_create(&th[t], NULL, slice_thread, &jobs[t]) == 0;
  run_slice(&jobs[0]);
  for (size_t t = 1; t < nt; t++) {
    if (started[t]) pthread_join(th[t], NULL);
    else run_slice(&jobs[t]);
  }
  free(jobs); free(th); free(started);
  return 0;
}

int or_forward_linear(uint32_t dtype, const uint8_t *raw, size_t raw_len,
                      const float *x, size_t x_len, float *out, size_t out_len,
                      size_t nr, size_t nc, int n_threads) {
  if (x_len < nc || out_len < nr) return -1; /* linear.rs:23-25 bail! */
  if (raw_len < or_nbytes_for(dtype, nr * nc)) return -1; /* tensor_raw_bytes */
  slice_job proto;
  memset(&proto, 0, sizeof proto);
  proto.raw = raw;
  proto.x = x;
  proto.out = out;
  proto.nc = nc;
  if (dtype == 12) { /* Q4_K arm, :28-47 */
    if (nc % 256 != 0) return -1; /* fused_gemv_q4k assert :66 */
    proto.kind = 0;
    return run_partitioned(proto, nr, n_threads);
  }
  if (dtype == 14) { /* Q6_K arm, :48-66 */
    /* the reference takes nc / 256 blocks without a check; a row that is
     * not whole blocks is rejected here */
    if (nc % 256 != 0) return -1;
    proto.kind = 2;
    return run_partitioned(proto, nr, n_threads);
  }
  /* `_` arm, :68-88: whole-tensor dequant on the calling thread first */
  float *deq = (float *)calloc(nr * nc ? nr * nc : 1, sizeof(float));
  if (!deq) return -3;
  int rc = or_dequantize(dtype, raw, raw_len, deq, nr * nc);
  if (rc != 0) {
    free(deq);
    return rc;
  }
  proto.kind = 1;
  proto.deq = deq;
  rc = run_partitioned(proto, nr, n_threads);
  free(deq);
  return rc;
}

int or_forward_linear_batch(uint32_t dtype, const uint8_t *raw, size_t raw_len,
                            const float *xs, float *outs, size_t bs, size_t nr,
                            size_t nc, int n_threads) {
  if (bs == 0) return 0; /* linear.rs:184 */
  if (dtype == 12) {
    if (nc % 256 != 0) return -1;
    if (raw_len < or_nbytes_for(12, nr * nc)) return -1;
    memset(outs, 0, bs * nr * sizeof(float)); /* :205-207 */
    /* :209-236: rows partitioned over n_threads threads (rpt = ceil(nr /
     * nt)); inside a slice the batched scalar kernel runs block -> row ->
     * token.  Each (row, token) value is a sum of per-block partials added
     * in block order, so the result does not depend on the partition. */
    const float **xp = (const float **)malloc(bs * sizeof(float *));
    float **op = (float **)malloc(bs * sizeof(float *));
    if (!xp || !op) {
      free(xp); free(op);
      return -3;
    }
    for (size_t t = 0; t < bs; t++) {
      xp[t] = xs + t * nc;
      op[t] = outs + t * nr;
    }
    slice_job proto;
    memset(&proto, 0, sizeof proto);
    proto.kind = 3;
    proto.raw = raw;
    proto.nc = nc;
    proto.xp = xp;
    proto.op = op;
    proto.bs = bs;
    int rc = run_partitioned(proto, nr, n_threads);
    free(xp); free(op);
    return rc;
  }
  for (size_t t = 0; t < bs; t++) {
    int rc = or_forward_linear(dtype, raw, raw_len, xs + t * nc, nc,
                               outs + t * nr, nr, nr, nc, n_threads);
    if (rc != 0) return rc;
  }
  return 0;
}

/* ---------------------------------------------------------------------- */
/* f32 steps either side of the path, swamp-engine/src/ops.rs:188-220      */
/* ---------------------------------------------------------------------- */

/* rmsnorm, ops.rs:188-201: ss = sum x*x in order, ss /= n, ss += eps,
 * inv = 1 / sqrt(ss), out = x * inv * w (left to right). */
void or_rmsnorm(float *out, const float *x, const float *w, size_t n, float eps) {
  float ss = 0.0f;
  for (size_t i = 0; i < n; i++) {
    float p = x[i] * x[i];
    ss = ss + p;
  }
  ss = ss / (float)n;
  ss = ss + eps;
  float inv = 1.0f / sqrtf(ss);
  for (size_t i = 0; i < n; i++) out[i] = x[i] * inv * w[i];
}

/* silu, ops.rs:203-208: x = x / (1 + exp(-x)), with the C library's expf
 * (what f32::exp calls on Linux). */
void or_silu(float *x, size_t n) {
  for (size_t i = 0; i < n; i++) {
    float v = x[i];
    x[i] = v / (1.0f + expf(-v));
  }
}

/* mul_in_place, ops.rs:210-214; add_in_place, ops.rs:216-220 */
void or_mul_in_place(float *a, const float *b, size_t n) {
  for (size_t i = 0; i < n; i++) a[i] = a[i] * b[i];
}
void or_add_in_place(float *a, const float *b, size_t n) {
  for (size_t i = 0; i < n; i++) a[i] = a[i] + b[i];
}

/* ---------------------------------------------------------------------- */
/* int8 dot, swamp-kernels/src/lib.rs:452-482 (scalar arm :477-481)        */
/* ---------------------------------------------------------------------- */

float or_gemv_q8_dot(const int8_t *w, const int8_t *a, int k, float scale) {
  if (!w || !a || k <= 0) return 0.0f;
  int32_t dot = 0;
  for (int i = 0; i < k; i++) dot += (int32_t)w[i] * (int32_t)a[i];
  return (float)dot * scale;
}

void or_xorshift64_i8(uint64_t *s, int8_t *out, size_t n) {
  for (size_t i = 0; i < n; i++) {
    *s ^= *s << 13;
    *s ^= *s >> 7;
    *s ^= *s << 17;
    out[i] = (int8_t)(uint8_t)(*s & 0xFF);
  }
}
