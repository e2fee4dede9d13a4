// gemm.hip -- prefill GEMM on the matrix cores, and on-device Q8_0
// activation quantization.
//
// Replaces the prefill use of forward_linear_batch
// (swamp-engine/src/executor.rs:106-110 -> linear.rs:176-239): the reference
// runs the batched CPU GEMV token block by token block; here one launch
// computes y[m][r] = sum_k W[r,k] x[m][k] for the whole prompt.
//
// bf16 path (MFMA-bound: 2*M*N*K flops over ~0.56 B/weight + 2 B/act):
//  * Workgroup tile 256 tokens x 256 weight rows, K step 64, 4 waves in a
//    2 x 2 arrangement; each wave owns 128 x 128 outputs = 4 x 4
//    V_MFMA_F32_32X32X16_BF16 tiles (256 fp32 accumulators per lane).
//  * Per K step the activation tile (256 x 64 bf16, 32 KB) is copied into
//    LDS and the weight tile is dequantized ONCE into LDS as bf16 (32 KB):
//    lane t dequantizes row t's 64-weight item.  Two LDS stages (128 KB of
//    gfx950's 160 KB) let the next tile's global loads fly during the
//    current tile's MFMAs; one barrier per K step.
//  * LDS rows are 128 B; 16-byte chunks are XOR-swizzled by (row & 7) so
//    the 32-row fragment reads hit distinct banks.
//  * Workgroup ids are remapped so each XCD (ids i, i+8, ...) walks a
//    contiguous run of tiles that share weight columns in its L2.
#include "swamp_common.hpp"
#include "swamp_items.hpp"

namespace {

using swamp::Raw;
using swamp::load_raw;
using swamp::q4k_scales;
using swamp::shr16;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4v_t __attribute__((ext_vector_type(4)));

constexpr int kBM = 256, kBN = 256, kBK = 64;
constexpr int kThreads = 256;
constexpr int kStageBytes = (kBM + kBN) * kBK * 2;  // 64 KB
constexpr int kSmemBytes = 2 * kStageBytes;         // 128 KB

__device__ __forceinline__ int swz(int row, int chunk) {
  return row * 128 + ((chunk ^ (row & 7)) << 4);
}

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  bf16x2_t v;
  v[0] = (__bf16)a;
  v[1] = (__bf16)b;
  return __builtin_bit_cast(uint32_t, v);
}

// Dequantize the 64 weights of one item (natural k order) into 8 chunks of
// 8 bf16 (4 dwords each).
template <int DT>
__device__ __forceinline__ void dequant_item_bf16(const Raw<DT> &r, int item, uint32_t (&o)[8][4]) {
  if constexpr (DT == SWAMP_Q4_0) {
#pragma unroll
    for (int blk = 0; blk < 2; blk++) {
      const float d = swamp::f16_bits_to_f32(blk == 0 ? (r.d[0] & 0xFFFFu) : (r.d[4] >> 16));
      const float nd = -8.0f * d;
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const uint32_t w = blk == 0 ? shr16(r.d[t + 1], r.d[t]) : r.d[5 + t];
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = __builtin_fmaf(float((w >> (4 * e)) & 0xFu), d, nd);
#pragma unroll
        for (int q = 0; q < 4; q++) o[4 * blk + t][q] = pack_bf16(v[2 * q], v[2 * q + 1]);
      }
    }
  } else if constexpr (DT == SWAMP_Q8_0) {
#pragma unroll
    for (int blk = 0; blk < 2; blk++) {
      const float d = swamp::f16_bits_to_f32(blk == 0 ? (r.d[0] & 0xFFFFu) : (r.d[8] >> 16));
#pragma unroll
      for (int t = 0; t < 4; t++) {
        uint32_t w0, w1;
        if (blk == 0) {
          w0 = shr16(r.d[2 * t + 1], r.d[2 * t]);
          w1 = shr16(r.d[2 * t + 2], r.d[2 * t + 1]);
        } else {
          w0 = r.d[9 + 2 * t];
          w1 = r.d[10 + 2 * t];
        }
        float v[8];
#pragma unroll
        for (int b = 0; b < 4; b++) {
          v[b] = float(int8_t(uint8_t(w0 >> (8 * b)))) * d;
          v[4 + b] = float(int8_t(uint8_t(w1 >> (8 * b)))) * d;
        }
#pragma unroll
        for (int q = 0; q < 4; q++) o[4 * blk + t][q] = pack_bf16(v[2 * q], v[2 * q + 1]);
      }
    }
  } else {
    const float d = swamp::f16_bits_to_f32(r.h[0] & 0xFFFFu);
    const float dmin = swamp::f16_bits_to_f32(r.h[0] >> 16);
    uint32_t sc0, m0, sc1, m1;
    q4k_scales(r.h, 2 * (item & 3), sc0, m0, sc1, m1);
    const float sa = d * float(sc0), ma = dmin * float(m0);
    const float sb = d * float(sc1), mb = dmin * float(m1);
#pragma unroll
    for (int c = 0; c < 8; c++) {
      // chunk c < 4: sub-block A elements 8c..8c+7 = low nibbles of bytes
      // 8c..8c+7; chunk c >= 4: sub-block B, high nibbles of 8(c-4)..
      const int cc = c & 3;
      const bool hi = c >= 4;
      const uint32_t w0 = r.q[2 * cc], w1 = r.q[2 * cc + 1];
      const float s = hi ? sb : sa, m = hi ? mb : ma;
      float v[8];
#pragma unroll
      for (int b = 0; b < 4; b++) {
        const uint32_t q0 = (w0 >> (8 * b + (hi ? 4 : 0))) & 0xFu;
        const uint32_t q1 = (w1 >> (8 * b + (hi ? 4 : 0))) & 0xFu;
        v[b] = __builtin_fmaf(float(q0), s, -m);
        v[4 + b] = __builtin_fmaf(float(q1), s, -m);
      }
#pragma unroll
      for (int q = 0; q < 4; q++) o[c][q] = pack_bf16(v[2 * q], v[2 * q + 1]);
    }
  }
}

// Global loads of K step kt: 8 activation chunks (16 B) and this lane's
// weight item (row tid of the tile).
template <int DT>
__device__ __forceinline__ void tile_gload(u32x4v_t (&xreg)[8], Raw<DT> &raw,
                                           const uint16_t *const (&xsrc)[8], const uint8_t *wrow,
                                           int kt) {
#pragma unroll
  for (int i = 0; i < 8; i++) xreg[i] = *reinterpret_cast<const u32x4v_t *>(xsrc[i] + kt * kBK);
  load_raw<DT>(raw, wrow, kt);
}

// Registers -> one LDS stage: activations as loaded, weights dequantized.
template <int DT>
__device__ __forceinline__ void tile_lstore(uint8_t *xs, const u32x4v_t (&xreg)[8], const Raw<DT> &raw,
                                            const int (&xoff)[8], int tid, int kt) {
  uint8_t *ws = xs + kBM * kBK * 2;
#pragma unroll
  for (int i = 0; i < 8; i++) *reinterpret_cast<u32x4v_t *>(xs + xoff[i]) = xreg[i];
  uint32_t o[8][4];
  dequant_item_bf16<DT>(raw, kt, o);
#pragma unroll
  for (int c = 0; c < 8; c++)
    *reinterpret_cast<u32x4v_t *>(ws + swz(tid, c)) = u32x4v_t{o[c][0], o[c][1], o[c][2], o[c][3]};
}

template <int DT>
__global__ void __launch_bounds__(kThreads, 1) gemm_bf16_kernel(
    const uint8_t *__restrict__ w, const uint16_t *__restrict__ x, float *__restrict__ y, int M,
    int N, int K, size_t row_bytes, int tiles_m, int tiles_n) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave & 1, wn = wave >> 1;

  // XCD-aware tile order: hardware ids i, i+8, ... run on one XCD; give
  // each XCD a contiguous slice of the (n-major) tile sequence.
  const int total = tiles_m * tiles_n;
  int L = blockIdx.x;
  if (total % 8 == 0) L = (blockIdx.x % 8) * (total / 8) + blockIdx.x / 8;
  const int mt = L % tiles_m, nt = L / tiles_m;
  const int m0 = mt * kBM, n0 = nt * kBN;

  // global -> register assignments
  const uint16_t *xsrc[8];
  int xoff[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const int id = i * kThreads + tid;
    const int xr = id >> 3, xc = id & 7;
    const int grow = min(m0 + xr, M - 1);
    xsrc[i] = x + size_t(grow) * K + 8 * xc;
    xoff[i] = swz(xr, xc);
  }
  const uint8_t *wrow = w + size_t(min(n0 + tid, N - 1)) * row_bytes;

  const int KT = K / kBK;
  u32x4v_t xreg[8];
  Raw<DT> raw;
  tile_gload<DT>(xreg, raw, xsrc, wrow, 0);
  tile_lstore<DT>(smem, xreg, raw, xoff, tid, 0);

  f32x16_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;

  __syncthreads();

  const int fr = lane & 31, fc = lane >> 5;
  for (int kt = 0; kt < KT; kt++) {
    const int stage = kt & 1;
    if (kt + 1 < KT) tile_gload<DT>(xreg, raw, xsrc, wrow, kt + 1);
    const uint8_t *xs = smem + stage * kStageBytes;
    const uint8_t *ws = xs + kBM * kBK * 2;
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ks++) {
      bf16x8_t a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int r = wm * 128 + i * 32 + fr;
        a[i] = *reinterpret_cast<const bf16x8_t *>(xs + swz(r, 2 * ks + fc));
      }
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int r = wn * 128 + j * 32 + fr;
        b[j] = *reinterpret_cast<const bf16x8_t *>(ws + swz(r, 2 * ks + fc));
      }
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < KT) tile_lstore<DT>(smem + (stage ^ 1) * kStageBytes, xreg, raw, xoff, tid, kt + 1);
    __syncthreads();
  }

  // C layout of a 32x32 tile: lane holds column (lane & 31), rows
  // 8*(e/4) + 4*(lane/32) + (e%4) for e = 0..15.
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int n = n0 + wn * 128 + j * 32 + fr;
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const int m = m0 + wm * 128 + i * 32 + 8 * (e >> 2) + 4 * fc + (e & 3);
        if (m < M && n < N) y[size_t(m) * N + n] = acc[i][j][e];
      }
    }
}

// ---- Q8_0 activation quantization ------------------------------------------
// One wavefront quantizes two 32-element blocks (lanes 0-31, 32-63).
template <bool kBf16>
__global__ void quantize_q8_0_kernel(const void *__restrict__ src, uint8_t *__restrict__ dst,
                                     size_t n_blocks) {
  const size_t gid = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const size_t blk = gid >> 5;
  const int i = int(gid & 31);
  const bool ok = blk < n_blocks;
  float v = 0.f;
  if (ok) {
    if (kBf16) v = __uint_as_float(uint32_t(static_cast<const uint16_t *>(src)[gid]) << 16);
    else v = static_cast<const float *>(src)[gid];
  }
  float a = fabsf(v);
#pragma unroll
  for (int off = 16; off >= 1; off >>= 1) a = fmaxf(a, __shfl_xor(a, off, 32));
  const float d = a / 127.0f;
  const float id = d != 0.f ? 1.0f / d : 0.f;
  float q = roundf(v * id);
  q = fminf(127.f, fmaxf(-127.f, q));
  if (ok) {
    uint8_t *b = dst + blk * 34;
    b[2 + i] = uint8_t(int8_t(q));
    if (i == 0) {
      const uint16_t h = __builtin_bit_cast(uint16_t, _Float16(d));
      b[0] = uint8_t(h & 0xFF);
      b[1] = uint8_t(h >> 8);
    }
  }
}

}  // namespace

int swamp_launch_gemm(uint32_t dtype, const void *d_w, const void *d_x, uint32_t x_type,
                      float *d_y, int m, int n_rows, int n_cols, hipStream_t s) {
  if (m == 0 || n_rows == 0) return SWAMP_OK;
  if (x_type != SWAMP_BF16) return SWAMP_EDTYPE;  // int8 path: not built yet
  if (n_cols % kBK != 0) return SWAMP_ESHAPE;
  const int tiles_m = (m + kBM - 1) / kBM, tiles_n = (n_rows + kBN - 1) / kBN;
  const dim3 grid(unsigned(tiles_m * tiles_n));
  const uint8_t *w = static_cast<const uint8_t *>(d_w);
  const uint16_t *x = static_cast<const uint16_t *>(d_x);
  const size_t rb = swamp::row_bytes(int(dtype), size_t(n_cols));
  switch (dtype) {
#define SWAMP_GEMM_CASE(DT)                                                                   \
  case DT: {                                                                                  \
    static bool attr = false;                                                                 \
    if (!attr) {                                                                              \
      if (hipFuncSetAttribute(reinterpret_cast<const void *>(&gemm_bf16_kernel<DT>),         \
                              hipFuncAttributeMaxDynamicSharedMemorySize,                     \
                              kSmemBytes) != hipSuccess)                                      \
        return SWAMP_ELAUNCH;                                                                 \
      attr = true;                                                                            \
    }                                                                                         \
    gemm_bf16_kernel<DT><<<grid, kThreads, kSmemBytes, s>>>(w, x, d_y, m, n_rows, n_cols, rb, \
                                                            tiles_m, tiles_n);                \
    break;                                                                                    \
  }
    SWAMP_GEMM_CASE(SWAMP_Q4_0)
    SWAMP_GEMM_CASE(SWAMP_Q8_0)
    SWAMP_GEMM_CASE(SWAMP_Q4_K)
#undef SWAMP_GEMM_CASE
  default:
    return SWAMP_EDTYPE;
  }
  return hipGetLastError() == hipSuccess ? SWAMP_OK : SWAMP_ELAUNCH;
}

int swamp_launch_quantize_q8_0(const void *d_x, uint32_t x_type, void *d_q, size_t n,
                               hipStream_t s) {
  const size_t nb = n / 32;
  if (nb == 0) return SWAMP_OK;
  const unsigned grid = unsigned((nb * 32 + 255) / 256);
  if (x_type == SWAMP_BF16)
    quantize_q8_0_kernel<true><<<grid, 256, 0, s>>>(d_x, static_cast<uint8_t *>(d_q), nb);
  else if (x_type == SWAMP_F32)
    quantize_q8_0_kernel<false><<<grid, 256, 0, s>>>(d_x, static_cast<uint8_t *>(d_q), nb);
  else
    return SWAMP_EDTYPE;
  return hipGetLastError() == hipSuccess ? SWAMP_OK : SWAMP_ELAUNCH;
}
