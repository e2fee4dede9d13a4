/*
 * swamp_quant.h -- host-side weight and activation preparation.
 *
 * The reference (llamanyon.rs) only DEquantizes GGUF blocks; it has no
 * quantizer.  These functions produce the block bytes that the device
 * kernels in swamp_qmm.h consume, plus the seeded synthetic data used by
 * the tests and the benchmark.  They run on the host, once, before any
 * timed work; nothing in the matmul path calls them.
 *
 * Byte layouts are the ones the reference's dequantizers read:
 *   Q4_0  18 B / 32 weights: f16 d, then 16 bytes; element i is in byte
 *         i/2, LOW nibble for even i (swamp-gguf/src/quant/q4_0.rs:30-35),
 *         value (q - 8) * d.
 *   Q8_0  34 B / 32 weights: f16 d, 32 int8; value q * d (q8_0.rs:127-139).
 *   Q4_K  144 B / 256 weights: f16 d, f16 dmin, 12 packed 6-bit scale/min
 *         bytes (q4_k.rs:37-53), 128 nibble bytes in "layout A"
 *         (q4_k.rs:290-319): byte 32p+i holds sub-block 2p element i (low)
 *         and sub-block 2p+1 element i (high); value (d*sc)*q - dmin*m.
 *   Q6_K  210 B / 256 weights: ql[128], qh[64], int8 sc[16], f16 d
 *         (q6_k.rs:25-28); element 128h + 32k + l (k < 4, l < 32) has its
 *         low 4 bits in ql[64h + l + 32(k&1)] (low nibble for k < 2, high
 *         for k >= 2) and bits 4-5 in qh[32h + l] bits 2k..2k+1; value
 *         (d * sc[e/16]) * (q - 32) for element e (q6_k.rs:36-44).
 *
 * All functions return 0 on success, -1 on a bad argument, -2 on an
 * unsupported dtype.  n_threads <= 0 means "use the hardware threads";
 * results never depend on n_threads.
 */
#ifndef SWAMP_QUANT_H
#define SWAMP_QUANT_H

#ifndef SWAMP_API
#define SWAMP_API __attribute__((visibility("default")))
#endif

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* IEEE conversions with round-to-nearest-even (what half::f16::from_f32 and
 * half::bf16::from_f32 do). */
SWAMP_API uint16_t swamp_f32_to_f16(float f);
SWAMP_API uint16_t swamp_f32_to_bf16(float f);
SWAMP_API void swamp_f32_to_bf16_array(const float *src, uint16_t *dst, size_t n);

/* rows x cols i.i.d. N(0, sigma^2) floats.  Row r draws from its own
 * splitmix64 stream seeded with seed ^ ((r + 1) * 0xD1B54A32D192ED03), and
 * Box-Muller in double precision turns pairs of draws into two normals. */
SWAMP_API int swamp_fill_normal(uint64_t seed, float sigma, float *dst, size_t rows,
                      size_t cols, int n_threads);

/* Quantize rows x cols floats (row-major, cols a multiple of the block
 * size) into dtype blocks, row after row.  dtype: 2 = Q4_0, 8 = Q8_0,
 * 12 = Q4_K, 14 = Q6_K.  dst holds rows * cols / block * type_size bytes. */
SWAMP_API int swamp_quantize(uint32_t dtype, const float *src, uint8_t *dst, size_t rows,
                   size_t cols, int n_threads);

/* swamp_fill_normal followed by swamp_quantize, one row at a time, so a
 * 128256 x 8192 matrix never needs its f32 copy in memory.  Produces the
 * same bytes as the two-step call with the same seed. */
SWAMP_API int swamp_synth_quantized(uint32_t dtype, uint64_t seed, float sigma,
                          uint8_t *dst, size_t rows, size_t cols,
                          int n_threads);

#ifdef __cplusplus
}
#endif
#endif
