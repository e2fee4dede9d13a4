// producers.hip -- the activation producers on either side of the small
// batch and the prefill GEMM: RMSNorm of every token row (ops.rs:188-201)
// and SiLU(gate) * up (ops.rs:203-214), for n_tok tokens at once, written
// as fp32 (the small batch's input) or as the bf16 the prefill GEMM reads.
//
// Replaces, for a whole prompt or batch, the per-token rmsnorm before the
// QKV and FFN projections (swamp-engine/src/executor.rs:433, :488) and the
// silu + mul_in_place before the down projection (:501-502).  HBM-bound
// single passes: RMSNorm reads x (kept in registers between the sum of
// squares and the scaling) and w, SwiGLU reads gate and up once; each
// writes its output once, so the GEMM gets its bf16 input without a
// separate cast.
//
// Arithmetic: inv_rms = rsq(sum(x^2) / n + eps) and out = (x * inv_rms) * w
// as in the fused decode GEMV's prologue; silu(g) * u = g * rcp(1 + 2^(-g
// log2 e)) * u (swamp::silu_mul).  The sum of squares runs in a different
// order than the reference's sequential loop, so results agree to rounding.
// bf16 output is the fp32 result rounded to nearest even.
#include "swamp_common.hpp"

#include <algorithm>

namespace {

typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void store4(float *o, size_t i, float4 v) {
  *reinterpret_cast<float4 *>(o + i) = v;
}
__device__ __forceinline__ void store4(__bf16 *o, size_t i, float4 v) {
  bf16x4_t b;
  b[0] = (__bf16)v.x;
  b[1] = (__bf16)v.y;
  b[2] = (__bf16)v.z;
  b[3] = (__bf16)v.w;
  *reinterpret_cast<bf16x4_t *>(o + i) = b;
}

constexpr int kThreads = 256;

// One workgroup per token row; n_cols % 4 == 0, rows 16-byte aligned.  The
// first kKeep float4 of each thread (rows up to 8192 floats) stay in
// registers between the sum of squares and the scaling; longer rows read
// the rest again.
constexpr int kKeep = 8;
template <typename OutT>
__global__ void __launch_bounds__(kThreads) rmsnorm_rows_kernel(const float *__restrict__ x,
                                                                const float *__restrict__ w,
                                                                float eps, OutT *__restrict__ out,
                                                                int n_cols) {
  const size_t row = size_t(blockIdx.x) * size_t(n_cols);
  const float *xr = x + row;
  const int i0 = 4 * int(threadIdx.x);
  float4 keep[kKeep];
#pragma unroll
  for (int j = 0; j < kKeep; j++) {
    const int i = i0 + 4 * kThreads * j;
    keep[j] = i < n_cols ? *reinterpret_cast<const float4 *>(xr + i) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < kKeep; j++)
    ss += keep[j].x * keep[j].x + keep[j].y * keep[j].y + keep[j].z * keep[j].z +
          keep[j].w * keep[j].w;
  for (int i = i0 + 4 * kThreads * kKeep; i < n_cols; i += 4 * kThreads) {
    const float4 v = *reinterpret_cast<const float4 *>(xr + i);
    ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
  }
  __shared__ float part[kThreads / 64];
  ss = swamp::wave_sum(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int k = 0; k < kThreads / 64; k++) tot += part[k];
  const float inv = __builtin_amdgcn_rsqf(tot / float(n_cols) + eps);
  auto put = [&](int i, float4 v) {
    const float4 g = *reinterpret_cast<const float4 *>(w + i);
    store4(out, row + size_t(i),
           make_float4(v.x * inv * g.x, v.y * inv * g.y, v.z * inv * g.z, v.w * inv * g.w));
  };
#pragma unroll
  for (int j = 0; j < kKeep; j++) {
    const int i = i0 + 4 * kThreads * j;
    if (i < n_cols) put(i, keep[j]);
  }
  for (int i = i0 + 4 * kThreads * kKeep; i < n_cols; i += 4 * kThreads)
    put(i, *reinterpret_cast<const float4 *>(xr + i));
}

// Grid-stride over n4 groups of 4 elements.
template <typename OutT>
__global__ void __launch_bounds__(kThreads) swiglu_kernel(const float *__restrict__ gate,
                                                          const float *__restrict__ up,
                                                          OutT *__restrict__ out, size_t n4) {
  for (size_t i = size_t(blockIdx.x) * kThreads + threadIdx.x; i < n4;
       i += size_t(gridDim.x) * kThreads) {
    const float4 g = reinterpret_cast<const float4 *>(gate)[i];
    const float4 u = reinterpret_cast<const float4 *>(up)[i];
    store4(out, 4 * i,
           make_float4(swamp::silu_mul(g.x, u.x), swamp::silu_mul(g.y, u.y),
                       swamp::silu_mul(g.z, u.z), swamp::silu_mul(g.w, u.w)));
  }
}

// fp32 -> bf16 (round to nearest even), grid-stride over n4 groups of 4.
__global__ void __launch_bounds__(kThreads) f32_to_bf16_kernel(const float *__restrict__ x,
                                                               __bf16 *__restrict__ out,
                                                               size_t n4) {
  for (size_t i = size_t(blockIdx.x) * kThreads + threadIdx.x; i < n4;
       i += size_t(gridDim.x) * kThreads)
    store4(out, 4 * i, reinterpret_cast<const float4 *>(x)[i]);
}

unsigned stream_grid(size_t n4) {
  const size_t want = (n4 + kThreads - 1) / kThreads;
  return unsigned(std::min<size_t>(want, size_t(swamp::device_info().num_cus) * 16));
}

}  // namespace

int swamp_launch_f32_to_bf16(const float *d_x, void *d_out, size_t n, hipStream_t s) {
  f32_to_bf16_kernel<<<stream_grid(n / 4), kThreads, 0, s>>>(d_x, static_cast<__bf16 *>(d_out),
                                                             n / 4);
  return hipGetLastError() == hipSuccess ? SWAMP_OK : SWAMP_ELAUNCH;
}

int swamp_launch_rmsnorm_rows(const float *d_x, const float *d_norm_w, float eps, void *d_out,
                              uint32_t out_type, int n_tok, int n_cols, hipStream_t s) {
  if (out_type == SWAMP_BF16)
    rmsnorm_rows_kernel<__bf16><<<unsigned(n_tok), kThreads, 0, s>>>(
        d_x, d_norm_w, eps, static_cast<__bf16 *>(d_out), n_cols);
  else
    rmsnorm_rows_kernel<float><<<unsigned(n_tok), kThreads, 0, s>>>(
        d_x, d_norm_w, eps, static_cast<float *>(d_out), n_cols);
  return hipGetLastError() == hipSuccess ? SWAMP_OK : SWAMP_ELAUNCH;
}

int swamp_launch_swiglu(const float *d_gate, const float *d_up, void *d_out, uint32_t out_type,
                        size_t n, hipStream_t s) {
  const size_t n4 = n / 4;
  const unsigned grid = stream_grid(n4);
  if (out_type == SWAMP_BF16)
    swiglu_kernel<__bf16><<<grid, kThreads, 0, s>>>(d_gate, d_up, static_cast<__bf16 *>(d_out), n4);
  else
    swiglu_kernel<float><<<grid, kThreads, 0, s>>>(d_gate, d_up, static_cast<float *>(d_out), n4);
  return hipGetLastError() == hipSuccess ? SWAMP_OK : SWAMP_ELAUNCH;
}
