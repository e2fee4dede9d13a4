// gemv.hip -- decode GEMV (one token) for Q4_0 / Q8_0 / Q4_K / Q6_K rows.
//
// Replaces forward_linear (swamp-engine/src/linear.rs:14-90) and the
// kernels it reaches, fused_gemv_q4k (swamp-kernels/src/fused_gemv_q4k.rs:
// 59-82, scalar body :466-508) and fused_gemv_q6k (fused_gemv_q6k.rs:22-41,
// scalar body :248-291), on the device.
//
// Design (HBM-bound; 0.5625 B/weight for Q4_0/Q4_K, 0.8203 for Q6_K, 1.0625
// for Q8_0):
//  * A row is cut into 64-weight "items" (two Q4_0 blocks = 36 B, two Q8_0
//    blocks = 68 B, a quarter Q4_K super-block = 32 B of nibbles + the 16 B
//    header).  Lane j of a workgroup always owns item j (+ T, + 2T, ...) of
//    every row, so its x values are loaded ONCE into registers and reused
//    for every row the workgroup visits (workgroups are persistent over
//    tiles of kRows rows).
//  * Tiles are double-buffered in registers: the loads of the next tile are
//    issued (unconditionally, so the wait counts stay exact) before the
//    current tile is reduced, so a wave never waits on HBM latency between
//    tiles.
//  * Weights become fp16 pairs with one and-or each: a low nibble q under
//    the magic 0x6400 is 1024 + q, a high nibble left in place is
//    1024 + 16 q (its x is pre-divided by 16), an int8 byte flipped to
//    q + 128 is 1024 + q + 128, a 6-bit Q6_K code gets its two qh bits
//    or-ed in above its nibble (1024 + q, or 1024 + 16 q for high
//    nibbles).  V_DOT2_F32_F16 multiplies a pair by two fp16 x values
//    exactly and accumulates in fp32; the constant offset is removed per
//    block with the matching weighted sum of the same fp16 x values.  Per
//    8 nibbles: 1 shift + 4 and-or + 4 dot2 (Q6_K: about twice that).
//  * x is converted to fp16 per item after scaling by a power of two that
//    puts the item's largest |x| in [2^14, 2^15) (exact; fp16 range safe);
//    the item's result is scaled back.
//  * The kRows partial sums of a lane are reduced over the wavefront with a
//    transposed butterfly (cross-half exchanges first, each halving the
//    number of live values, then DPP adds), then over the waves of the
//    workgroup through LDS.
#include "gemv_core.hpp"

namespace {

using swamp::Raw;

// Generic path for shapes the item kernel does not take (n_cols % 64 != 0
// for Q4_0/Q8_0, or rows of more than 65536 weights): one wavefront per row, one 32-weight block per lane step,
// byte loads.  Correct for any n_cols % 32 == 0.
template <int DT>
__global__ void __launch_bounds__(256) gemv_generic_kernel(const uint8_t *__restrict__ w,
                                                           const float *__restrict__ x,
                                                           float *__restrict__ y, int n_rows,
                                                           int n_cols) {
  const int wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  const int nwaves = (gridDim.x * blockDim.x) >> 6;
  const int nb = n_cols / 32;
  const int bbytes = DT == SWAMP_Q4_0 ? 18 : 34;
  for (int row = wave; row < n_rows; row += nwaves) {
    const uint8_t *rp = w + size_t(row) * nb * bbytes;
    float acc = 0.f;
    for (int b = lane; b < nb; b += 64) {
      const uint8_t *blk = rp + size_t(b) * bbytes;
      const float d = swamp::f16_bits_to_f32(uint32_t(blk[0]) | (uint32_t(blk[1]) << 8));
      const float *xb = x + size_t(b) * 32;
      float s = 0.f;
      if (DT == SWAMP_Q4_0) {
        for (int i = 0; i < 32; i++) {
          const uint32_t byte = blk[2 + i / 2];
          const int q = int((i & 1) ? (byte >> 4) : (byte & 0xFu)) - 8;
          s += float(q) * xb[i];
        }
      } else {
        for (int i = 0; i < 32; i++) s += float(int8_t(blk[2 + i])) * xb[i];
      }
      acc += d * s;
    }
    acc = swamp::wave_sum(acc);
    if (lane == 0) y[row] = acc;
  }
}

// Generic Q6_K path for rows of an odd number of blocks (n_cols % 512 ==
// 256), whose blocks start at any even byte offset: one wavefront per row,
// one 16-weight sub-block (one int8 scale) per lane step, byte loads.
__global__ void __launch_bounds__(256) gemv_generic_q6k_kernel(const uint8_t *__restrict__ w,
                                                               const float *__restrict__ x,
                                                               float *__restrict__ y, int n_rows,
                                                               int n_cols) {
  const int wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  const int nwaves = (gridDim.x * blockDim.x) >> 6;
  const int nb = n_cols / 256;
  for (int row = wave; row < n_rows; row += nwaves) {
    const uint8_t *rp = w + size_t(row) * nb * 210;
    float acc = 0.f;
    for (int u = lane; u < nb * 16; u += 64) {
      const int b = u >> 4, g = u & 15;  // sub-block g: elements 16g .. 16g+15
      const uint8_t *blk = rp + size_t(b) * 210;
      const float d = swamp::f16_bits_to_f32(uint32_t(blk[208]) | (uint32_t(blk[209]) << 8));
      const float sc = float(int8_t(blk[192 + g]));
      const int h = g >> 3, j = (g >> 1) & 3, l0 = (g & 1) * 16;
      const float *xg = x + size_t(b) * 256 + 16 * g;
      float s = 0.f;
      for (int c = 0; c < 16; c++) {
        const int l = l0 + c;
        const uint32_t lb = blk[64 * h + 32 * (j & 1) + l];
        const uint32_t hb = blk[128 + 32 * h + l];
        const int q = int(((j >= 2 ? lb >> 4 : lb) & 0xFu) | (((hb >> (2 * j)) & 3u) << 4)) - 32;
        s += float(q) * xg[c];
      }
      acc += d * sc * s;
    }
    acc = swamp::wave_sum(acc);
    if (lane == 0) y[row] = acc;
  }
}

// Generic Q4_K path for rows longer than the item kernel takes (more than
// 65536 weights): one wavefront per row, one 32-weight sub-block per lane
// step, byte loads.  Sub-block j of a super-block uses qs[32 (j/2) ..],
// low nibbles for even j, high for odd (layout A, q4_k.rs:290-319); its
// 6-bit scale and min come unpacked as in q4_k.rs:37-53, and
// sum((d sc) q - dmin m) x is taken as (d sc) sum(q x) - (dmin m) sum(x).
__global__ void __launch_bounds__(256) gemv_generic_q4k_kernel(const uint8_t *__restrict__ w,
                                                               const float *__restrict__ x,
                                                               float *__restrict__ y, int n_rows,
                                                               int n_cols) {
  const int wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  const int nwaves = (gridDim.x * blockDim.x) >> 6;
  const int nb = n_cols / 256;
  for (int row = wave; row < n_rows; row += nwaves) {
    const uint8_t *rp = w + size_t(row) * nb * 144;
    float acc = 0.f;
    for (int u = lane; u < nb * 8; u += 64) {
      const int b = u >> 3, j = u & 7;
      const uint8_t *blk = rp + size_t(b) * 144;
      const float d = swamp::f16_bits_to_f32(uint32_t(blk[0]) | (uint32_t(blk[1]) << 8));
      const float dmin = swamp::f16_bits_to_f32(uint32_t(blk[2]) | (uint32_t(blk[3]) << 8));
      const uint8_t *sc = blk + 4;
      uint32_t scale, mn;
      if (j < 4) {
        scale = sc[j] & 63u;
        mn = sc[j + 4] & 63u;
      } else {
        scale = (sc[j + 4] & 0xFu) | ((uint32_t(sc[j - 4]) >> 6) << 4);
        mn = (uint32_t(sc[j + 4]) >> 4) | ((uint32_t(sc[j]) >> 6) << 4);
      }
      const uint8_t *qs = blk + 16 + 32 * (j >> 1);
      const int sh = 4 * (j & 1);
      const float *xs = x + size_t(b) * 256 + 32 * j;
      float sq = 0.f, sx = 0.f;
      for (int i = 0; i < 32; i++) {
        sq += float((uint32_t(qs[i]) >> sh) & 0xFu) * xs[i];
        sx += xs[i];
      }
      acc += (d * float(scale)) * sq - (dmin * float(mn)) * sx;
    }
    acc = swamp::wave_sum(acc);
    if (lane == 0) y[row] = acc;
  }
}

}  // namespace

namespace {

// Shapes the item kernel does not take: one wavefront per row (fp32 x).
int launch_generic(uint32_t dtype, const void *d_w, const float *d_x, float *d_y, int n_rows,
                   int n_cols, hipStream_t s) {
  const int cus = swamp::device_info().num_cus;
  const int blocks = std::min((n_rows + 3) / 4, cus * 8);
  if (dtype == SWAMP_Q4_K)
    gemv_generic_q4k_kernel<<<blocks, 256, 0, s>>>(static_cast<const uint8_t *>(d_w), d_x, d_y,
                                                   n_rows, n_cols);
  else if (dtype == SWAMP_Q6_K)
    gemv_generic_q6k_kernel<<<blocks, 256, 0, s>>>(static_cast<const uint8_t *>(d_w), d_x, d_y,
                                                   n_rows, n_cols);
  else if (dtype == SWAMP_Q4_0)
    gemv_generic_kernel<SWAMP_Q4_0><<<blocks, 256, 0, s>>>(static_cast<const uint8_t *>(d_w), d_x,
                                                           d_y, n_rows, n_cols);
  else
    gemv_generic_kernel<SWAMP_Q8_0><<<blocks, 256, 0, s>>>(static_cast<const uint8_t *>(d_w), d_x,
                                                           d_y, n_rows, n_cols);
  return hipGetLastError() == hipSuccess ? SWAMP_OK : SWAMP_ELAUNCH;
}

template <bool kX32>
int launch_one(uint32_t dtype, const void *d_w, const float *d_x, float *d_y, int n_rows,
               int n_cols, hipStream_t s) {
  if (n_rows == 0) return SWAMP_OK;
  if (!item_path_ok(dtype, n_cols)) return launch_generic(dtype, d_w, d_x, d_y, n_rows, n_cols, s);
  MatSet ms;
  const void *ws[1] = {d_w};
  float *ys[1] = {d_y};
  const int tr = tile_rows_for(dtype, n_cols, n_rows, kX32);
  build_matset(ms, 1, ws, ys, &n_rows, tr);
  ms.wpc = waves_per_cu_for(dtype, n_cols, n_rows, kX32);
  return dispatch<kProNone, kX32>(dtype, ms, d_x, Pro{}, n_cols, tr, s);
}

}  // namespace

int swamp_launch_gemv(uint32_t dtype, const void *d_w, const float *d_x, float *d_y,
                      int n_rows, int n_cols, hipStream_t s) {
  return launch_one<true>(dtype, d_w, d_x, d_y, n_rows, n_cols, s);
}

int swamp_launch_gemv_f16x(uint32_t dtype, const void *d_w, const float *d_x, float *d_y,
                           int n_rows, int n_cols, hipStream_t s) {
  return launch_one<false>(dtype, d_w, d_x, d_y, n_rows, n_cols, s);
}

int swamp_launch_gemv_multi(int n_mats, const uint32_t *dtypes, const void *const *d_ws,
                            const int *row_counts, const float *d_x, float *const *d_ys,
                            int n_cols, hipStream_t s) {
  return launch_multi<kProNone, true>(n_mats, dtypes, d_ws, row_counts, d_x, Pro{}, d_ys, n_cols,
                                      s);
}

#ifdef SWAMP_STAGE_STAMPS
// Measurement build only: copy the first n stamp slots (8 per wave, five
// used) to host memory, then clear them when reset is set.  0 on success.
extern "C" __attribute__((visibility("default"))) int swamp_gemv_stage_stamps(uint64_t *host,
                                                                               int n, int reset) {
  if (n < 0 || n > kStampWaves * 8) return SWAMP_EINVAL;
  if (n && hipMemcpyFromSymbol(host, HIP_SYMBOL(g_gemv_stamps), size_t(n) * 8, 0,
                               hipMemcpyDeviceToHost) != hipSuccess)
    return SWAMP_ELAUNCH;
  if (reset) {
    static uint64_t zeros[kStampWaves * 8];
    if (hipMemcpyToSymbol(HIP_SYMBOL(g_gemv_stamps), zeros, sizeof(zeros), 0,
                          hipMemcpyHostToDevice) != hipSuccess)
      return SWAMP_ELAUNCH;
  }
  return SWAMP_OK;
}
#endif
