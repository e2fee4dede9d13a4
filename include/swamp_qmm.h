/*
 * swamp_qmm.h -- C ABI of libswamp_gpu.so, the MI355X (gfx950) quantized
 * matmul library for GGUF Q4_0 / Q8_0 / Q4_K / Q6_K weights.
 *
 * Conventions (all entry points):
 *  - dtype codes are GGML's (swamp-gguf/src/dtype.rs:10-40):
 *      SWAMP_F32 = 0, SWAMP_F16 = 1, SWAMP_Q4_0 = 2, SWAMP_Q8_0 = 8,
 *      SWAMP_Q4_K = 12, SWAMP_Q6_K = 14, SWAMP_BF16 = 30.
 *  - W is row-major by output row, raw GGUF block bytes exactly as
 *    GgufFile::tensor_raw_bytes returns them (swamp-gguf/src/mmap.rs:110-117):
 *    row r starts at byte r * (n_cols / block) * type_size.
 *    n_cols = tensor.shape[0] = K, n_rows = tensor.shape[1]
 *    (swamp-engine/src/linear.rs:21-22).
 *  - y[r] = sum_k W[r,k] * x[k] in fp32.
 *  - Pointers named d_* are DEVICE pointers; the caller owns every buffer.
 *  - stream is a hipStream_t passed as void* (NULL = default stream); every
 *    device entry point is asynchronous on it.  None allocates, except that
 *    swamp_qgemv_batched and swamp_qgemm take scratch memory for split
 *    reductions from a buffer the library keeps per (device, stream): see
 *    "Scratch" below.
 *  - Return 0 on success, a negative SWAMP_E* code on error; on error no
 *    output is written and nothing is launched.
 */
#ifndef SWAMP_QMM_H
#define SWAMP_QMM_H

#ifndef SWAMP_API
#define SWAMP_API __attribute__((visibility("default")))
#endif

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  SWAMP_F32 = 0,
  SWAMP_F16 = 1,
  SWAMP_Q4_0 = 2,
  SWAMP_Q8_0 = 8,
  SWAMP_Q4_K = 12,
  SWAMP_Q6_K = 14,
  SWAMP_BF16 = 30
};

enum {
  SWAMP_OK = 0,
  SWAMP_EINVAL = -1,    /* null pointer, negative size, misaligned pointer */
  SWAMP_EDTYPE = -2,    /* dtype not supported by this entry point */
  SWAMP_ESHAPE = -3,    /* n_cols not a multiple of the block, buffer too small */
  SWAMP_ELAUNCH = -4,   /* HIP launch or copy failed */
  SWAMP_ENODEVICE = -5, /* no HIP device */
  SWAMP_EWORKSPACE = -6 /* workspace missing or too small */
};

/* Replaces gpu_init (swamp-gpu/src/lib.rs:62-71 -> fused_attention.cu:133-143)
 * for the matmul library: selects the current device, creates its context
 * and caches its CU count.  Idempotent; optional (every entry point calls
 * it on first use). */
SWAMP_API int swamp_gpu_init(void);

/* Text for a return code (static storage). */
SWAMP_API const char *swamp_strerror(int code);

/* GgmlDType::block_size / type_size / nbytes_for (swamp-gguf/src/dtype.rs:
 * 79-89, 92-132, 135-139).  0 for an unknown code. */
SWAMP_API size_t swamp_block_size(uint32_t dtype);
SWAMP_API size_t swamp_type_size(uint32_t dtype);
SWAMP_API size_t swamp_nbytes_for(uint32_t dtype, size_t n_elems);

/* quant::dequantize (swamp-gguf/src/quant/mod.rs:18-33) on the device, for
 * F32, F16, BF16, Q4_0 (q4_0.rs:11-39), Q8_0 (q8_0.rs:15-40), Q4_K
 * (q4_k.rs:21-33, 278-321) and Q6_K (q6_k.rs:7-56; d_raw 2-byte aligned).  Writes n floats to d_dst, bit-identical to the
 * reference's scalar CPU dequantizer (NaN inputs give NaN outputs).
 * raw_len < nbytes_for(dtype, n) -> SWAMP_ESHAPE (the reference's
 * BufferTooSmall, q4_0.rs:15-20). */
SWAMP_API int swamp_qdequant(uint32_t dtype, const void *d_raw, size_t raw_len,
                   float *d_dst, size_t n, void *stream);

/* No counterpart in the reference: the bf16 form of swamp_qdequant, the
 * pass the prefill GEMM's dequantize-once route runs before its plain bf16
 * GEMM, exported so that its output can be checked bit for bit and
 * for callers that feed their own bf16 GEMM.  Writes n bf16 values (raw
 * bits, uint16) to d_dst: each the swamp_qdequant value rounded to nearest
 * even (NaN stays NaN).  dtype Q4_0, Q8_0 (n a multiple of 32, d_raw 4-byte
 * aligned), Q4_K (n a multiple of 256, d_raw 16-byte aligned) or Q6_K (n a
 * multiple of 256, d_raw 2-byte aligned); d_dst 16-byte aligned.
 * raw_len < nbytes_for(dtype, n) -> SWAMP_ESHAPE. */
SWAMP_API int swamp_qdequant_bf16(uint32_t dtype, const void *d_raw, size_t raw_len,
                                  void *d_dst, size_t n, void *stream);

/* Decode GEMV, y = W x, OVERWRITING y[0..n_rows).
 * Replaces forward_linear (swamp-engine/src/linear.rs:14-90) and the
 * kernels it reaches, fused_gemv_q4k (swamp-kernels/src/fused_gemv_q4k.rs:
 * 59-82) and fused_gemv_q6k (fused_gemv_q6k.rs:22-41).
 * Arithmetic in the reference's precision: the exact weight codes times
 * unrounded fp32 x, summed in fp32 (one rounding per multiply-add), with
 * each block's scale and offset applied to the block's sums rather than
 * to every weight -- d (sum q x - 8 sum x) for Q4_0, (d sc) sum q x -
 * (dmin m) sum x per Q4_K sub-block -- a regrouping of the reference's
 * per-weight products whose rounding differs from it; the normalized error
 * against the reference's arithmetic measures 1.0-1.4e-7 (Q4_0, Q8_0) and
 * 2e-8 (Q4_K) on the Llama shapes, against a 1e-6 gate.
 * dtype Q4_0, Q8_0, Q4_K or Q6_K; n_cols a multiple of the block size (32,
 * or 256 for Q4_K and Q6_K); w_len >= nbytes_for(dtype, n_rows * n_cols);
 * d_w 4-byte aligned (16 for Q4_K), d_x 16-byte aligned.  n_cols == 0
 * gives y = 0.
 * Q6_K follows the dequantizer's arithmetic (int8 scales, exact f16 d,
 * q6_k.rs:28-44), as the reference's scalar GEMV does for every d whose
 * exponent field is 1..30; the reference's private f16 decode
 * (fused_gemv_q6k.rs:11-21) mis-decodes zero and subnormal d, and its SIMD
 * arms read the int8 scales as unsigned (:71-74, :164-167). */
SWAMP_API int swamp_qgemv(uint32_t dtype, const void *d_w, size_t w_len,
                const float *d_x, float *d_y, int n_rows, int n_cols,
                void *stream);

/* The decode GEMV at reduced x precision, for callers that accept it:
 * arguments, shapes and y as swamp_qgemv, but each 64-weight run of x is
 * scaled by a power of two (exact) and rounded to fp16 (2^-11 relative)
 * inside the kernel, and weight pairs meet x pairs in fp16 dot products
 * with fp32 accumulation.  That halves the kernel's arithmetic per weight
 * against swamp_qgemv's fp32 x; the results differ from the reference's
 * fp32 arithmetic by about 1e-5 of ||W_r|| ||x|| (swamp_qgemv: about
 * 1e-7).  No counterpart in the reference. */
SWAMP_API int swamp_qgemv_f16x(uint32_t dtype, const void *d_w, size_t w_len,
                               const float *d_x, float *d_y, int n_rows, int n_cols,
                               void *stream);

/* Several matrices that share one x (the engine's fused QKV and gate+up):
 * y_m = W_m x for m < n_mats, each OVERWRITTEN, one launch.
 * Replaces forward_linear_multi (linear.rs:96-170) and fused_gemv_q4k_multi
 * (fused_gemv_q4k.rs:401-460).  All matrices share n_cols; dtypes may differ
 * per matrix.  At most SWAMP_MULTI_MAX matrices. */
#define SWAMP_MULTI_MAX 8
SWAMP_API int swamp_qgemv_multi(int n_mats, const uint32_t *dtypes,
                      const void *const *d_ws, const size_t *w_lens,
                      const int *row_counts, const float *d_x,
                      float *const *d_ys, int n_cols, void *stream);

/* Several GEMVs, each with its own weights, shape, x and y, in one call:
 * y_i = W_i x_i, each OVERWRITTEN, i < n.  Replaces forward_gemvs
 * (swamp-engine/src/linear.rs:278-333), which zeroes each output and runs
 * the specs' row slices in one parallel section.  Arguments per GEMV as
 * swamp_qgemv (any of its dtypes; the reference sends every non-Q4_K spec
 * to the Q6_K kernel, here each dtype gets its own); every GEMV is
 * validated before any is launched; the GEMVs run in order on the stream. */
SWAMP_API int swamp_qgemv_many(int n, const uint32_t *dtypes, const void *const *d_ws,
                               const size_t *w_lens, const int *n_rows, const int *n_cols,
                               const float *const *d_xs, float *const *d_ys, void *stream);

/* RMSNorm fused into the GEMV's x prologue: y_m = W_m x_norm with
 * x_norm = (x * inv_rms) * norm_w, inv_rms = 1 / sqrt(sum(x^2) / n_cols +
 * eps), each y_m OVERWRITTEN; x_norm is not written.  Replaces the
 * engine's rmsnorm (swamp-engine/src/ops.rs:188-201) followed by
 * forward_linear_multi / forward_linear on its output (executor.rs:433-445
 * QKV, :488-499 gate+up, :530-533 logits).  Arguments as swamp_qgemv_multi
 * plus d_norm_w (n_cols floats, 16-byte aligned) and eps.  The sum of
 * squares is reduced in a different order than the reference's sequential
 * loop.  n_cols <= 32768 and a whole number of 64-weight items (multiple of
 * 64; 256 for Q4_K; 512 for Q6_K), else SWAMP_ESHAPE. */
SWAMP_API int swamp_qgemv_rmsnorm(int n_mats, const uint32_t *dtypes,
                        const void *const *d_ws, const size_t *w_lens,
                        const int *row_counts, const float *d_x,
                        const float *d_norm_w, float eps, float *const *d_ys,
                        int n_cols, void *stream);

/* SiLU(gate) * up fused into the GEMV's x prologue (the FFN down
 * projection): h = gate / (1 + exp(-gate)) * up, then y = W h
 * (accumulate = 0) or y += W h (accumulate = 1, the residual add).
 * Replaces silu + mul_in_place (swamp-engine/src/ops.rs:203-214) +
 * forward_linear + add_in_place (:216-220) at executor.rs:501-506.
 * d_gate, d_up: n_cols floats each, 16-byte aligned.  Shape rules as
 * swamp_qgemv_rmsnorm. */
SWAMP_API int swamp_qgemv_swiglu(uint32_t dtype, const void *d_w, size_t w_len,
                       const float *d_gate, const float *d_up, float *d_y,
                       int n_rows, int n_cols, int accumulate, void *stream);

/* Small-batch GEMV/GEMM for speculative verify and continuous batching:
 * n_tok tokens, d_x is [n_tok][n_cols] fp32, d_y is [n_tok][n_rows] fp32.
 * accumulate = 0: y = W x (forward_linear_batch zeroes its outputs first,
 * linear.rs:205-207); accumulate = 1: y += W x (the kernel contract of
 * fused_gemv_q4k_batched, fused_gemv_q4k.rs:527-554, :694).
 * Replaces forward_linear_batch (linear.rs:176-239) and
 * fused_gemv_q4k_batched.  Any n_tok >= 1; weights are read once per
 * pass of up to 64 tokens (Q4_0, Q8_0, Q4_K; Q6_K 32).  With accumulate = 0, a pass
 * of one token runs the decode GEMV, a pass of two the GEMV over both
 * tokens (x rounded to fp16 like the passes of 3..64, rows of up to 32768
 * weights), and n_tok > 64 runs swamp_qgemm's
 * kernels on x rounded to bf16 (in scratch; without scratch, passes of 64
 * instead).  Passes of 2..64 tokens round x to fp16 on the matrix cores
 * (about 3e-5 of ||W_r|| ||x|| against the fp32 reference; more than 64
 * tokens, bf16: about 1e-4): entries must lie within fp16 range
 * (|x| < 65504), also for accumulate = 1 and when no scratch is available.  Q6_K
 * (forward_linear_batch's fallback_gemv, linear.rs:336-364, is written over
 * y): accumulate = 1 is SWAMP_EDTYPE; rows of a multiple of 512 weights
 * run passes of up to 32 tokens on the matrix cores, at any n_tok, with
 * the weights d * sc * (q - 32) rounded once to fp16 (the same precision
 * class as the other formats' passes); other rows run swamp_qgemv per
 * token. */
SWAMP_API int swamp_qgemv_batched(uint32_t dtype, const void *d_w, size_t w_len,
                        const float *d_x, float *d_y, int n_tok, int n_rows,
                        int n_cols, int accumulate, void *stream);

/* Prefill GEMM on the matrix cores: y[m][r] = sum_k W[r,k] x[m][k], fp32
 * out [m][n_rows], OVERWRITTEN.  Replaces the prefill use of
 * forward_linear_batch (swamp-engine/src/executor.rs:106-110 ->
 * linear.rs:176-239).
 *   x_type SWAMP_BF16: d_x is bf16 [m][n_cols]; W is dequantized in
 *     registers to bf16 and fed to bf16 MFMA (fp32 accumulate).
 *   x_type SWAMP_Q8_0: d_x is Q8_0 blocks [m][n_cols/32] (as produced by
 *     swamp_quantize_q8_0); int8 MFMA (one 32x32x32 instruction per
 *     32-weight block) against W's int8 codes (Q4_0: nibble - 8; Q4_K:
 *     the nibble, with d * sc as the block scale and dmin * m * d_x *
 *     sum(q_x) subtracted per block), each block's int32 result scaled by
 *     d_w * d_x into fp32.  Q4_0, Q8_0 and Q4_K weights; n_cols a multiple
 *     of 128.
 * dtype Q4_0, Q8_0, Q4_K or Q6_K (Q6_K with bf16 x only); bf16 x needs
 * n_cols a multiple of 64.
 * With bf16 x the fused kernel dequantizes weight tiles in registers to
 * bf16 (every tile reads the quantized blocks: 0.56-1.06 bytes per
 * weight); when the tiles do not fill the GPU, K is split across
 * workgroups whose partial tiles go to scratch and are summed in piece
 * order by a second kernel (deterministic).  For Q6_K at any length, and
 * from 1024 tokens when 256 x 256 tiles would fill more than half but not
 * all of the CUs (e.g. 2048 tokens x 6144 rows), the weights are instead
 * dequantized once per call to bf16 in scratch (row chunks of at most
 * 512 MB; the same bf16 values) and each chunk runs through this library's
 * plain bf16 x bf16 -> fp32 MFMA GEMM, whose 192- and 128-row tiles fill
 * the CUs; when that scratch cannot be had the fused kernel runs (Q6_K:
 * SWAMP_EWORKSPACE).  Both routes sum in a fixed order: repeated calls
 * give the same bits. */
SWAMP_API int swamp_qgemm(uint32_t dtype, const void *d_w, size_t w_len,
                const void *d_x, uint32_t x_type, float *d_y, int m,
                int n_rows, int n_cols, void *stream);

/* Scratch.  swamp_qgemv_batched and swamp_qgemm need scratch memory for
 * some shapes (the partial sums of K split across workgroups, the bf16
 * copy of x of a batch of more than 64 tokens, and the bf16 weight chunk
 * of the GEMM's dequantize-once route).  The library keeps one buffer per
 * (device, stream) for it (hipStreamPerThread: per host thread too),
 * allocated on first use and replaced when a call needs more, both
 * stream-ordered on that stream (hipMallocAsync / hipFreeAsync): no call
 * synchronizes the host.  A buffer that a call under graph capture used is
 * never freed (the graph's replays write it): when a later call needs
 * more, it is kept until the process ends and a new one replaces it for
 * the stream's eager calls.  While the stream is being captured into a graph
 * nothing is allocated: a call that needs more than the stream's buffer
 * holds takes the path without scratch (split pieces added with float
 * atomics into y cleared by a kernel, which is not bit-reproducible; more
 * than 64 tokens in passes of 64).  Calls on one stream must be issued from
 * one host thread at a time: two threads calling on the same stream (the
 * null stream included) at once race on its buffer.
 *   swamp_qgemv_batched_workspace / swamp_qgemm_workspace: the scratch
 *     bytes such a call takes (0: none);
 *   swamp_workspace_reserve: make the stream's buffer at least `bytes`
 *     long now (for example before capturing calls into a graph); 0, or
 *     SWAMP_EWORKSPACE when it cannot be allocated or the stream is being
 *     captured. */
SWAMP_API size_t swamp_qgemv_batched_workspace(uint32_t dtype, int n_tok, int n_rows,
                                               int n_cols, int accumulate);
SWAMP_API size_t swamp_qgemm_workspace(uint32_t dtype, uint32_t x_type, int m, int n_rows,
                                       int n_cols);
SWAMP_API int swamp_workspace_reserve(void *stream, size_t bytes);

/* swamp_qgemv_batched with every argument, result and error as there, but
 * allocating nothing: no hipMalloc / hipMallocAsync / hipFree and no
 * allocating library routine, on any path.  No counterpart in the
 * reference; it is for callers that cannot allocate (code under graph
 * capture, tight serving loops, harnesses that forbid allocation).  Its
 * scratch is a fixed array of SWAMP_NOALLOC_SCRATCH_BYTES (32 MiB) in
 * device memory that each GPU the library runs on holds until the process
 * ends; a call whose scratch exceeds it (swamp_qgemv_batched_workspace)
 * returns SWAMP_EWORKSPACE before launching anything.  Every call on one
 * GPU shares that GPU's array: calls that overlap on one GPU (on two
 * streams, or from two host threads) race on it and must be ordered by the
 * caller. */
#define SWAMP_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
SWAMP_API int swamp_qgemv_batched_noalloc(uint32_t dtype, const void *d_w, size_t w_len,
                                          const float *d_x, float *d_y, int n_tok,
                                          int n_rows, int n_cols, int accumulate,
                                          void *stream);

/* Activation producers for the small batch (out_type SWAMP_F32) and the
 * prefill GEMM (SWAMP_BF16: its bf16 x, rounded to nearest even), over
 * n_tok tokens in one pass.
 * swamp_rmsnorm_rows: out[t] = (x[t] * inv) * w with inv = 1 /
 *   sqrt(sum(x[t]^2) / n_cols + eps), d_x [n_tok][n_cols].  Replaces
 *   rmsnorm (swamp-engine/src/ops.rs:188-201) before the QKV and FFN
 *   projections (executor.rs:433, :488) for a whole batch or prompt.
 * swamp_swiglu: out = silu(gate) * up = gate / (1 + exp(-gate)) * up over
 *   n elements.  Replaces silu + mul_in_place (ops.rs:203-214) before the
 *   down projection (executor.rs:501-502).
 * Inputs 16-byte aligned, d_out 16-byte (fp32) or 8-byte (bf16) aligned;
 * n_cols and n multiples of 4 (SWAMP_ESHAPE); out_type other than F32 /
 * BF16: SWAMP_EDTYPE. */
SWAMP_API int swamp_rmsnorm_rows(const float *d_x, const float *d_norm_w, float eps,
                       void *d_out, uint32_t out_type, int n_tok, int n_cols,
                       void *stream);
SWAMP_API int swamp_swiglu(const float *d_gate, const float *d_up, void *d_out,
                 uint32_t out_type, size_t n, void *stream);

/* Activations to Q8_0 blocks on the device (the int8 GEMM's input):
 * x_type SWAMP_F32 or SWAMP_BF16, n a multiple of 32, d_q receives
 * n / 32 * 34 bytes.  Per block d = amax / 127 rounded to f16,
 * q = round-half-away(x / d_unrounded) -- the block formula of the host
 * quantizer swamp_quantize (swamp_quant.h). */
SWAMP_API int swamp_quantize_q8_0(const void *d_x, uint32_t x_type, void *d_q, size_t n,
                        void *stream);

/* ---- the reference's two existing C exports, host-pointer semantics ---- */

/* swamp_fused_gemv_q4k (fused_gemv_q4k.rs:799-823): HOST pointers, Q4_K,
 * zeroes out and writes W x.  Null pointer or n_cols % 256 != 0 -> silent
 * return, like the reference.  Stages through device memory on the current
 * device and synchronizes before returning. */
SWAMP_API void swamp_fused_gemv_q4k(const uint8_t *w_raw, const float *x, float *out,
                          int n_rows, int n_cols);

/* swamp_gemv_q8_vnni (swamp-kernels/src/lib.rs:452-482): HOST pointers,
 * exact int32 dot of two int8 vectors times scale; null or k <= 0 -> 0.0f.
 * Computed on the device (staged), synchronizes before returning; returns
 * NaN if the device step fails. */
SWAMP_API float swamp_gemv_q8_vnni(const int8_t *weights, const int8_t *activations,
                         int k, float scale);

#ifdef __cplusplus
}
#endif
#endif
