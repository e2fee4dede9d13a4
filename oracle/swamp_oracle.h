/*
 * swamp_oracle.h -- CPU oracle for the quantized-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the
 * reference's scalar CPU matmul path (llamanyon.rs, Rust).  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and
 * only as the checker (or as the timed CPU baseline).  The product library
 * (libswamp_gpu.so) never links or calls it.
 *
 * Every function cites the reference file:line it restates.  Compiled with
 * -ffp-contract=off and no fast-math: Rust never contracts a*b-c into an
 * FMA, so the sequence of roundings here is the reference's.
 *
 * Return codes follow the reference's error behaviour:
 *   0  ok
 *  -1  BufferTooSmall / shape assert (the reference panics or bails)
 *  -2  dtype not implemented on this path
 */
#ifndef SWAMP_ORACLE_H
#define SWAMP_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GgmlDType table: swamp-gguf/src/dtype.rs:10-40 (codes), :79-89 (block
 * size), :92-132 (type size), :135-139 (nbytes_for).  0 = unknown code. */
size_t or_block_size(uint32_t dtype);
size_t or_type_size(uint32_t dtype);
size_t or_nbytes_for(uint32_t dtype, size_t n_elems);

/* half 2.7.1 f16::to_f32 (exact binary16 -> binary32; NaN keeps its payload
 * and gets the quiet bit).  Call sites: q4_0.rs:24, q8_0.rs:130,
 * q4_k.rs:281-282, fused_gemv_q4k.rs:475-476. */
float or_f16_to_f32(uint16_t h);
void or_f16_to_f32_array(const uint16_t *h, float *out, size_t n);
/* Same conversion done by the host's F16C unit (vcvtph2ps); returns -1 when
 * the CPU has no F16C.  Used only to pin or_f16_to_f32. */
int or_f16_to_f32_hw_array(const uint16_t *h, float *out, size_t n);
/* half 2.7.1 bf16::to_f32 (swamp-gguf/src/quant/f16.rs:18-28). */
float or_bf16_to_f32(uint16_t h);

/* quant::dequantize dispatcher, swamp-gguf/src/quant/mod.rs:18-33, for the
 * dtypes of this path: F32 (:35-44), F16/BF16 (f16.rs:6-28), Q4_0
 * (q4_0.rs:11-39), Q8_0 (q8_0.rs:127-139), Q4_K (q4_k.rs:21-33, 278-321). */
int or_dequantize(uint32_t dtype, const uint8_t *raw, size_t raw_len,
                  float *dst, size_t n);
int or_dequant_q4_0(const uint8_t *raw, size_t raw_len, float *dst, size_t n);
int or_dequant_q8_0(const uint8_t *raw, size_t raw_len, float *dst, size_t n);
int or_dequant_q4_k(const uint8_t *raw, size_t raw_len, float *dst, size_t n);
/* q6_k::dequant_q6k, swamp-gguf/src/quant/q6_k.rs:7-56 */
int or_dequant_q6_k(const uint8_t *raw, size_t raw_len, float *dst, size_t n);

/* unpack_scales, q4_k.rs:37-53 == unpack_scales_q4k fused_gemv_q4k.rs:30-43 */
void or_unpack_scales_q4k(const uint8_t sc[12], uint8_t scales[8],
                          uint8_t mins[8]);

/* fused_gemv_q4k with the scalar body, fused_gemv_q4k.rs:59-82 asserts +
 * :466-508 body (layout A, sequential f32 accumulation, overwrites out). */
int or_fused_gemv_q4k(const uint8_t *w_raw, size_t w_len, const float *x,
                      size_t x_len, float *out, size_t out_len, size_t n_rows,
                      size_t n_cols);

/* fused_gemv_q6k with the scalar body, swamp-kernels/src/fused_gemv_q6k.rs:
 * 248-291 (int8 scales, sequential f32 accumulation, overwrites out), d
 * decoded exactly like the dequantizer (q6_k.rs:28).  The reference's own
 * decode of d, f16_to_f32_raw (:11-21), is restated as or_q6k_f16_raw; it
 * agrees on every code with exponent field 1..30 and mis-decodes zero,
 * subnormal, inf and NaN codes.  n_cols % 256 != 0 -> -1. */
int or_fused_gemv_q6k(const uint8_t *w_raw, size_t w_len, const float *x,
                      size_t x_len, float *out, size_t out_len, size_t n_rows,
                      size_t n_cols);
float or_q6k_f16_raw(uint16_t v);

/* fused_gemv_q4k_batched with the scalar body, :527-554 + :650-698.
 * Loop order block -> row -> token; ACCUMULATES into out (out[t][row] +=). */
int or_fused_gemv_q4k_batched(const uint8_t *w_raw, const float *const *x_ptrs,
                              float *const *out_ptrs, size_t n_rows,
                              size_t n_cols, size_t batch);

/* fused_gemv_q4k_multi, :401-460 (zero-fill, block-outer, x shared). */
int or_fused_gemv_q4k_multi(const uint8_t *const *raws, const float *x,
                            float *const *outputs, const size_t *row_counts,
                            size_t n_mats, size_t n_cols);

/* forward_linear, swamp-engine/src/linear.rs:14-90.  Q4_K -> row slices of
 * rpt = ceil(nr/nt) through or_fused_gemv_q4k (:28-47); every other dtype of
 * this path -> allocate nr*nc f32, dequantize the whole tensor on one
 * thread, then per row a sequential f32 dot (:68-88).  n_threads worker
 * threads partition rows exactly like the rayon closure; the result does
 * not depend on n_threads.  Q6_K -> row slices through or_fused_gemv_q6k
 * (:48-66; n_cols % 256 != 0 -> -1). */
int or_forward_linear(uint32_t dtype, const uint8_t *raw, size_t raw_len,
                      const float *x, size_t x_len, float *out, size_t out_len,
                      size_t n_rows, size_t n_cols, int n_threads);

/* forward_linear_batch, linear.rs:176-239.  Q4_K: zero outs (:205-207) then
 * row slices through the batched scalar kernel.  Other dtypes: the
 * reference's fallback_gemv (:336-364) decodes non-Q4_K bytes as Q4_K
 * (:358), which is a bug; this restatement applies forward_linear per token
 * instead (the semantics the engine's decode path gives each token).  For
 * Q6_K that is exactly fallback_gemv's Q6_K arm (:357): fused_gemv_q6k per
 * token, written over the output.
 * xs is [bs][n_cols] contiguous, outs is [bs][n_rows] contiguous. */
int or_forward_linear_batch(uint32_t dtype, const uint8_t *raw, size_t raw_len,
                            const float *xs, float *outs, size_t bs,
                            size_t n_rows, size_t n_cols, int n_threads);

/* The f32 steps the engine runs either side of the path
 * (swamp-engine/src/ops.rs): rmsnorm (:188-201, sequential sum of squares,
 * out = x * inv * w), silu in place (:203-208, libm expf), mul_in_place
 * (:210-214), add_in_place (:216-220). */
void or_rmsnorm(float *out, const float *x, const float *w, size_t n, float eps);
void or_silu(float *x, size_t n);
void or_mul_in_place(float *a, const float *b, size_t n);
void or_add_in_place(float *a, const float *b, size_t n);

/* swamp_gemv_q8_vnni scalar arm, swamp-kernels/src/lib.rs:452-482:
 * exact int32 dot of two int8 vectors times scale; null or k<=0 -> 0. */
float or_gemv_q8_dot(const int8_t *w, const int8_t *a, int k, float scale);

/* xorshift64 byte stream of the int8-dot test, lib.rs:600-606:
 * s ^= s<<13; s ^= s>>7; s ^= s<<17; value = (int8)s. */
void or_xorshift64_i8(uint64_t *state, int8_t *out, size_t n);

#ifdef __cplusplus
}
#endif
#endif
