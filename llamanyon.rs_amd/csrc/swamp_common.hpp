// swamp_common.hpp -- shared device/host helpers for libswamp_gpu.so (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "swamp_qmm.h"

namespace swamp {

// Block geometry of the three weight formats (swamp-gguf/src/dtype.rs:79-132).
constexpr int kQ4_0Block = 32, kQ4_0Bytes = 18;
constexpr int kQ8_0Block = 32, kQ8_0Bytes = 34;
constexpr int kQ4_KBlock = 256, kQ4_KBytes = 144;
constexpr int kQ6_KBlock = 256, kQ6_KBytes = 210;

// One "item" is 64 weights of one row: two Q4_0 blocks (36 B), two Q8_0
// blocks (68 B), one quarter of a Q4_K super-block (32 nibble bytes plus
// the block's 16-byte header) or one quarter of a Q6_K block (48 bytes of
// ql/qh plus 4 scales and d; its 64 weights are four runs of 16).  Every
// kernel that streams rows hands out whole items to lanes.
constexpr int kItem = 64;

__host__ __device__ constexpr int item_bytes(int dt) {
  return dt == SWAMP_Q4_0 ? 36 : dt == SWAMP_Q8_0 ? 68 : 36 /* Q4_K: 144/4 */;
}

__host__ __device__ constexpr size_t row_bytes(int dt, size_t n_cols) {
  return dt == SWAMP_Q4_0   ? n_cols / 32 * 18
         : dt == SWAMP_Q8_0 ? n_cols / 32 * 34
         : dt == SWAMP_Q4_K ? n_cols / 256 * 144
         : dt == SWAMP_Q6_K ? n_cols / 256 * 210
                            : 0;
}

// 16-byte load with 4-byte alignment (gfx950 global loads accept dword
// alignment for multi-dword accesses).
struct __attribute__((aligned(4))) u32x4 {
  uint32_t v[4];
};

__device__ __forceinline__ u32x4 ld4(const uint8_t *p) {
  return *reinterpret_cast<const u32x4 *>(p);
}
__device__ __forceinline__ uint32_t ld1(const uint8_t *p) {
  return *reinterpret_cast<const uint32_t *>(p);
}

// Exact binary16 -> binary32 in integer arithmetic (same rules as
// half::f16::to_f32: subnormals renormalised, NaN payload kept + quiet bit).
__device__ __forceinline__ float f16_bits_to_f32_exact(uint32_t h) {
  const uint32_t sign = (h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1Fu;
  uint32_t man = h & 0x3FFu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {
      // man has its leading one at bit p (0..9); value = man * 2^-24.
      const int p = 31 - __builtin_clz(man);
      bits = sign | (uint32_t(p + 103) << 23) | ((man << (23 - p)) & 0x7FFFFFu);
    }
  } else if (exp == 31) {
    bits = sign | 0x7F800000u | (man ? (0x400000u | (man << 13)) : 0u);
  } else {
    bits = sign | ((exp + 112u) << 23) | (man << 13);
  }
  return __uint_as_float(bits);
}

// Hardware conversion (v_cvt_f32_f16); exact for every finite input.
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  _Float16 v = __builtin_bit_cast(_Float16, uint16_t(h & 0xFFFFu));
  return float(v);
}

// Wavefront (64-lane) sum; result valid in every lane.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// silu(g) * u = g / (1 + e^-g) * u with the hardware exp2 and reciprocal
// (about 1 ulp each): g * rcp(1 + 2^(-g log2 e)) * u.
__device__ __forceinline__ float silu_mul(float g, float u) {
  const float e = __builtin_amdgcn_exp2f(g * -1.44269504088896341f);
  return g * __builtin_amdgcn_rcpf(1.0f + e) * u;
}

// Per-device properties cached by the host side.
struct DeviceInfo {
  int device = -1;
  int num_cus = 256;
};
const DeviceInfo &device_info();  // current device (initialises it)

// Scratch memory of one entry-point call: partial sums of split reductions
// and converted activations, carved from one region by a bump allocator
// (256-byte aligned pieces).  The region is either the per-(device,
// stream) buffer of stream_workspace or a fixed region the caller names.
// get() returns nullptr once the region is exhausted; every caller then
// takes its path without scratch.
struct Scratch {
  uint8_t *base = nullptr;
  size_t cap = 0, used = 0;
  void *get(size_t bytes) {
    const size_t n = (bytes + 255) & ~size_t(255);
    if (!base || n > cap - used) return nullptr;
    void *p = base + used;
    used += n;
    return p;
  }
};

// The per-(device, stream) buffer, at least `bytes` long, for work queued
// on stream s of the current device; calls on one stream run in order and
// share it, calls on different streams never do (hipStreamPerThread is
// also told apart by host thread).  It is allocated on first use and
// replaced by a larger one when a call needs more, both stream-ordered on
// s (hipMallocAsync, the old one released by hipFreeAsync), so no call
// blocks the host.  While s is being captured into a graph nothing is
// allocated: nullptr when the buffer is missing or too small.  nullptr also
// when the allocation fails.
void *stream_workspace(hipStream_t s, size_t bytes);

// Scratch over the stream's buffer, sized for `bytes` (empty when bytes is
// 0 or the buffer is not available).
inline Scratch stream_scratch(hipStream_t s, size_t bytes) {
  Scratch sc;
  if (bytes) {
    sc.base = static_cast<uint8_t *>(stream_workspace(s, bytes));
    sc.cap = sc.base ? bytes : 0;
  }
  return sc;
}

}  // namespace swamp

// Internal launchers (defined in dequant.hip, gemv.hip, gemv_fused.hip,
// gemv_tokens.hip, gemv_batched.hip, gemm.hip, gemm_i8.hip, producers.hip).  They
// assume the arguments have been validated by api.cpp.
int swamp_launch_dequant(uint32_t dtype, const void *d_raw, float *d_dst,
                         size_t n, hipStream_t s);
int swamp_launch_dequant_bf16(uint32_t dtype, const void *d_raw, void *d_dst, size_t n,
                              hipStream_t s);
int swamp_launch_gemv(uint32_t dtype, const void *d_w, const float *d_x,
                      float *d_y, int n_rows, int n_cols, hipStream_t s);
int swamp_launch_gemv_f16x(uint32_t dtype, const void *d_w, const float *d_x,
                           float *d_y, int n_rows, int n_cols, hipStream_t s);
// 2 tokens at once through the fp16-x GEMV (gemv_tokens.hip), y written
// [n_tok][n_rows]; SWAMP_ESHAPE (nothing launched) outside the shapes
// swamp_gemv_tokens_ok accepts.
bool swamp_gemv_tokens_ok(uint32_t dtype, int n_tok, int n_cols);
int swamp_launch_gemv_tokens(uint32_t dtype, const void *d_w, const float *d_x, float *d_y,
                             int n_tok, int n_rows, int n_cols, hipStream_t s);
int swamp_launch_gemv_multi(int n_mats, const uint32_t *dtypes,
                            const void *const *d_ws, const int *row_counts,
                            const float *d_x, float *const *d_ys, int n_cols,
                            hipStream_t s);
int swamp_launch_gemv_rmsnorm(int n_mats, const uint32_t *dtypes,
                              const void *const *d_ws, const int *row_counts,
                              const float *d_x, const float *d_norm_w, float eps,
                              float *const *d_ys, int n_cols, hipStream_t s);
int swamp_launch_gemv_swiglu(uint32_t dtype, const void *d_w,
                             const float *d_gate, const float *d_up, float *d_y,
                             int n_rows, int n_cols, int accumulate,
                             hipStream_t s);
// Scratch bytes a call will take from its region (0: none), from the same
// plans the launchers follow.
size_t swamp_batched_scratch_bytes(uint32_t dtype, int n_tok, int n_rows, int n_cols,
                                   int accumulate, size_t limit = SIZE_MAX);
// limit: scratch the caller can offer; a route that needs more is not taken.
size_t swamp_gemm_scratch_bytes(uint32_t dtype, uint32_t x_type, int m, int n_rows, int n_cols,
                                size_t limit = SIZE_MAX);
// The bf16 GEMM's dequantize-once route (gemm_dq.hip, gemm_bb.hip): whether
// a shape takes it, its scratch, and the launcher, which returns
// kDqUnavailable, having launched nothing, when the scratch is missing (the
// caller then runs the fused kernel).
constexpr int kDqUnavailable = 1;
bool swamp_gemm_dq_route(uint32_t dtype, int m, int n_rows, int n_cols);
size_t swamp_gemm_dq_scratch_bytes(int m, int n_rows, int n_cols);
int swamp_launch_gemm_dq(uint32_t dtype, const void *d_w, const void *d_x, float *d_y, int m,
                         int n_rows, int n_cols, swamp::Scratch &sc, hipStream_t s);
int swamp_launch_gemv_batched(uint32_t dtype, const void *d_w,
                              const float *d_x, float *d_y, int n_tok,
                              int n_rows, int n_cols, int accumulate,
                              swamp::Scratch &sc, hipStream_t s);
int swamp_launch_gemm(uint32_t dtype, const void *d_w, const void *d_x,
                      uint32_t x_type, float *d_y, int m, int n_rows,
                      int n_cols, swamp::Scratch &sc, hipStream_t s);
int swamp_launch_gemm_i8(uint32_t dtype, const void *d_w, const void *d_xq8, float *d_y, int m,
                         int n_rows, int n_cols, swamp::Scratch &sc, hipStream_t s);
size_t swamp_gemm_i8_scratch_bytes(uint32_t dtype, int m, int n_rows, int n_cols);
int swamp_launch_split_reduce(const float *d_part, float *d_y, int pieces, size_t n,
                              hipStream_t s);
int swamp_launch_rmsnorm_rows(const float *d_x, const float *d_norm_w, float eps, void *d_out,
                              uint32_t out_type, int n_tok, int n_cols, hipStream_t s);
int swamp_launch_swiglu(const float *d_gate, const float *d_up, void *d_out, uint32_t out_type,
                        size_t n, hipStream_t s);
int swamp_launch_f32_to_bf16(const float *d_x, void *d_out, size_t n, hipStream_t s);
int swamp_launch_quantize_q8_0(const void *d_x, uint32_t x_type, void *d_q,
                               size_t n, hipStream_t s);
int swamp_launch_i8dot(const int8_t *d_w, const int8_t *d_a, int k,
                       int *d_out, hipStream_t s);
