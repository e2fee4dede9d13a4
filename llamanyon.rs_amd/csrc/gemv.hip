// gemv.hip -- decode GEMV (one token) for Q4_0 / Q8_0 / Q4_K rows.
//
// Replaces forward_linear (swamp-engine/src/linear.rs:14-90) and
// fused_gemv_q4k (swamp-kernels/src/fused_gemv_q4k.rs:59-82, scalar body
// :466-508) on the device.
//
// Design (HBM-bound; 0.5625 B/weight for Q4_0/Q4_K, 1.0625 for Q8_0):
//  * A row is cut into 64-weight "items" (two Q4_0 blocks = 36 B, two Q8_0
//    blocks = 68 B, a quarter Q4_K super-block = 32 B of nibbles + the 16 B
//    header).  Lane j of a workgroup always owns item j of every row, so its
//    64 x values are loaded ONCE into registers and reused for every row the
//    workgroup visits (workgroups are persistent over row tiles).
//  * Q4_0/Q4_K: x is held as bf16 pairs; nibbles become bf16 (128 + q) with
//    one and-or per pair and are multiplied by V_DOT2_F32_BF16 (two MACs
//    per instruction, fp32 accumulate).  The 128 (+8 for Q4_0) offset is
//    removed per block with the block sum of the same bf16 x values.
//  * Q8_0: fp32 x, int8 -> fp32 converts (byte-select converts), fp32 FMA.
//  * Each lane's partials are summed over the wavefront, then over the
//    waves of the workgroup through LDS, once per tile of kRows rows.
#include "swamp_common.hpp"
#include "swamp_items.hpp"

#include <cstdlib>

namespace {

using swamp::Raw;
using swamp::load_raw;
using swamp::q4k_scales;
using swamp::shr16;

typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;

constexpr uint32_t kBf16Magic = 0x43004300u;  // bf16 pair (128, 128)

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c,
                                         false);
}

// f32 -> bf16 bits, round to nearest even (x is finite activations).
__device__ __forceinline__ uint32_t bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7F800000u) == 0x7F800000u) return (u >> 16) | ((u & 0xFFFFu) ? 0x40u : 0u);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return u >> 16;
}
__device__ __forceinline__ float bf16_val(uint32_t b) { return __uint_as_float(b << 16); }

// Four bf16 pairs of one nibble dword w: pairs of (byte0, byte2) and
// (byte1, byte3) low nibbles, then the same for the high nibbles.
//   P0 = nib(w, 0), nib(w, 16)     P1 = nib(w, 8),  nib(w, 24)
//   P2 = nib(w, 4), nib(w, 20)     P3 = nib(w, 12), nib(w, 28)
__device__ __forceinline__ float dot_nib_dword(uint32_t w, const uint32_t *xp, float acc) {
  acc = dot2((w & 0x000F000Fu) | kBf16Magic, xp[0], acc);
  acc = dot2(((w >> 8) & 0x000F000Fu) | kBf16Magic, xp[1], acc);
  acc = dot2(((w >> 4) & 0x000F000Fu) | kBf16Magic, xp[2], acc);
  acc = dot2(((w >> 12) & 0x000F000Fu) | kBf16Magic, xp[3], acc);
  return acc;
}

// Element (0..63 within the item) that half h of pair p of nibble dword t
// multiplies.  Nibble n of dword t (n = 0..7, bit offset 4n) is:
//   Q4_0: byte n/2 of the dword, element 8t' + 2(n/2) + (n%2) of block t/4
//         (interleaved layout, q4_0.rs:30-35), t' = t%4;
//   Q4_K: low nibble of byte b -> sub-block A element 4t+b,
//         high nibble -> sub-block B (item elements 32..63) element 4t+b.
template <int DT>
__host__ __device__ constexpr int nib_elem(int t, int p, int h) {
  // bit offset of the nibble for (p, h)
  // p0: 0,16  p1: 8,24  p2: 4,20  p3: 12,28
  const int bit = (p == 0 ? 0 : p == 1 ? 8 : p == 2 ? 4 : 12) + 16 * h;
  const int byte = bit / 8, high = (bit % 8) != 0;
  if (DT == SWAMP_Q4_0) return 32 * (t / 4) + 8 * (t % 4) + 2 * byte + high;
  return 32 * high + 4 * t + byte;  // Q4_K
}

// Per-lane x fragment for one item.
template <int DT>
struct XFrag;

template <>
struct XFrag<SWAMP_Q4_0> {
  uint32_t p[32];  // 8 nibble dwords x 4 bf16 pairs
  float c[2];      // 136 * sum of the block's bf16 x (removes the +128 and -8)
};
template <>
struct XFrag<SWAMP_Q4_K> {
  uint32_t p[32];
  float sa, sb;  // sum of bf16 x over sub-block A and B
};
template <>
struct XFrag<SWAMP_Q8_0> {
  float v[64];
};

template <int DT>
__device__ __forceinline__ void load_xfrag(XFrag<DT> &xf, const float *__restrict__ x, int item) {
  const float4 *xp = reinterpret_cast<const float4 *>(x + size_t(item) * 64);
  float xv[64];
#pragma unroll
  for (int i = 0; i < 16; i++) {
    float4 f = xp[i];
    xv[4 * i] = f.x; xv[4 * i + 1] = f.y; xv[4 * i + 2] = f.z; xv[4 * i + 3] = f.w;
  }
  if constexpr (DT == SWAMP_Q8_0) {
#pragma unroll
    for (int i = 0; i < 64; i++) xf.v[i] = xv[i];
  } else {
    uint32_t xb[64];
#pragma unroll
    for (int i = 0; i < 64; i++) xb[i] = bf16_rne(xv[i]);
#pragma unroll
    for (int t = 0; t < 8; t++)
#pragma unroll
      for (int p = 0; p < 4; p++)
        xf.p[4 * t + p] = xb[nib_elem<DT>(t, p, 0)] | (xb[nib_elem<DT>(t, p, 1)] << 16);
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i++) {
      s0 += bf16_val(xb[i]);
      s1 += bf16_val(xb[32 + i]);
    }
    if constexpr (DT == SWAMP_Q4_0) {
      xf.c[0] = 136.0f * s0;
      xf.c[1] = 136.0f * s1;
    } else {
      xf.sa = s0;
      xf.sb = s1;
    }
  }
}

template <int DT>
__device__ __forceinline__ float item_dot(const Raw<DT> &r, const XFrag<DT> &xf, int item) {
  if constexpr (DT == SWAMP_Q4_0) {
    const float d0 = swamp::f16_bits_to_f32(r.d[0] & 0xFFFFu);
    const float d1 = swamp::f16_bits_to_f32(r.d[4] >> 16);
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int t = 0; t < 4; t++) s0 = dot_nib_dword(shr16(r.d[t + 1], r.d[t]), &xf.p[4 * t], s0);
#pragma unroll
    for (int t = 0; t < 4; t++) s1 = dot_nib_dword(r.d[5 + t], &xf.p[16 + 4 * t], s1);
    return d0 * (s0 - xf.c[0]) + d1 * (s1 - xf.c[1]);
  } else if constexpr (DT == SWAMP_Q8_0) {
    const float d0 = swamp::f16_bits_to_f32(r.d[0] & 0xFFFFu);
    const float d1 = swamp::f16_bits_to_f32(r.d[8] >> 16);
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int t = 0; t < 8; t++) {
      const uint32_t w = shr16(r.d[t + 1], r.d[t]);
#pragma unroll
      for (int b = 0; b < 4; b++) s0 += float(int8_t(uint8_t(w >> (8 * b)))) * xf.v[4 * t + b];
    }
#pragma unroll
    for (int t = 0; t < 8; t++) {
      const uint32_t w = r.d[9 + t];
#pragma unroll
      for (int b = 0; b < 4; b++) s1 += float(int8_t(uint8_t(w >> (8 * b)))) * xf.v[32 + 4 * t + b];
    }
    return d0 * s0 + d1 * s1;
  } else {
    const float d = swamp::f16_bits_to_f32(r.h[0] & 0xFFFFu);
    const float dmin = swamp::f16_bits_to_f32(r.h[0] >> 16);
    uint32_t sc0, m0, sc1, m1;
    q4k_scales(r.h, 2 * (item & 3), sc0, m0, sc1, m1);
    // low nibbles -> sub-block A, high -> B; pairs P0,P1 are low, P2,P3 high
    float sa = 0.f, sb = 0.f;
#pragma unroll
    for (int t = 0; t < 8; t++) {
      const uint32_t w = r.q[t];
      sa = dot2((w & 0x000F000Fu) | kBf16Magic, xf.p[4 * t + 0], sa);
      sa = dot2(((w >> 8) & 0x000F000Fu) | kBf16Magic, xf.p[4 * t + 1], sa);
      sb = dot2(((w >> 4) & 0x000F000Fu) | kBf16Magic, xf.p[4 * t + 2], sb);
      sb = dot2(((w >> 12) & 0x000F000Fu) | kBf16Magic, xf.p[4 * t + 3], sb);
    }
    // sum (d*sc*q - dmin*m) x = d*sc*(S - 128 Sx) - dmin*m*Sx
    const float qa = sa - 128.0f * xf.sa, qb = sb - 128.0f * xf.sb;
    return d * (float(sc0) * qa + float(sc1) * qb) - dmin * (float(m0) * xf.sa + float(m1) * xf.sb);
  }
}

constexpr int kMaxMats = SWAMP_MULTI_MAX;

struct MatSet {
  const uint8_t *w[kMaxMats];
  float *y[kMaxMats];
  int rows[kMaxMats];
  int tile_end[kMaxMats];  // cumulative tile counts
  int n;
};

// One workgroup = 64 * nwaves lanes; lane j owns items j, j + T, ...
// (kPPT items per lane), covering one row of ipr items.  The workgroup
// loops over row tiles of kRows rows.
template <int DT, int kPPT, int kRows>
__global__ void __launch_bounds__(512) gemv_kernel(MatSet ms, const float *__restrict__ x,
                                                   int ipr, size_t row_bytes, int n_tiles) {
  __shared__ float red[2][8][kRows];
  const int tid = threadIdx.x;
  const int T = blockDim.x;
  const int nw = T >> 6, wave = tid >> 6, lane = tid & 63;

  XFrag<DT> xf[kPPT];
  bool valid[kPPT];
#pragma unroll
  for (int j = 0; j < kPPT; j++) {
    const int item = tid + j * T;
    valid[j] = item < ipr;
    if (valid[j]) load_xfrag<DT>(xf[j], x, item);
  }

  int par = 0;
  for (int tile = blockIdx.x; tile < n_tiles; tile += gridDim.x, par ^= 1) {
    int m = 0;
    while (m + 1 < ms.n && tile >= ms.tile_end[m]) m++;
    const int first = m ? ms.tile_end[m - 1] : 0;
    const int row0 = (tile - first) * kRows;
    const int nrows = ms.rows[m];
    const uint8_t *wbase = ms.w[m];

    float acc[kRows];
    Raw<DT> raw[kRows][kPPT];
#pragma unroll
    for (int r = 0; r < kRows; r++) {
      acc[r] = 0.f;
      const int row = row0 + r < nrows ? row0 + r : nrows - 1;  // clamp: stays in bounds
#pragma unroll
      for (int j = 0; j < kPPT; j++)
        if (valid[j]) load_raw<DT>(raw[r][j], wbase + size_t(row) * row_bytes, tid + j * T);
    }
#pragma unroll
    for (int r = 0; r < kRows; r++)
#pragma unroll
      for (int j = 0; j < kPPT; j++)
        if (valid[j]) acc[r] += item_dot<DT>(raw[r][j], xf[j], tid + j * T);

#pragma unroll
    for (int r = 0; r < kRows; r++) acc[r] = swamp::wave_sum(acc[r]);

    float *y = ms.y[m];
    if (nw == 1) {
      if (lane < kRows && row0 + lane < nrows) {
        float v = acc[0];
#pragma unroll
        for (int r = 1; r < kRows; r++) v = lane == r ? acc[r] : v;
        y[row0 + lane] = v;
      }
    } else {
      if (lane == 0) {
#pragma unroll
        for (int r = 0; r < kRows; r++) red[par][wave][r] = acc[r];
      }
      __syncthreads();
      if (tid < kRows && row0 + tid < nrows) {
        float v = 0.f;
        for (int w = 0; w < nw; w++) v += red[par][w][tid];
        y[row0 + tid] = v;
      }
    }
  }
}

// Generic path for shapes the item kernel does not take (n_cols % 64 != 0
// for Q4_0/Q8_0): one wavefront per row, one 32-weight block per lane step,
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

struct Tuning {
  int waves_per_cu = 16;
  Tuning() {
    if (const char *s = std::getenv("SWAMP_GEMV_WAVES_PER_CU")) {
      int v = std::atoi(s);
      if (v >= 1 && v <= 64) waves_per_cu = v;
    }
  }
};
const Tuning &tuning() {
  static Tuning t;
  return t;
}

template <int DT, int kPPT, int kRows>
int launch_items(const MatSet &ms, const float *x, int n_cols, hipStream_t s) {
  const int ipr = n_cols / 64;
  int T = ((ipr + kPPT - 1) / kPPT + 63) / 64 * 64;
  if (T > 512) return SWAMP_ESHAPE;
  const int nw = T / 64;
  const int n_tiles = ms.tile_end[ms.n - 1];
  const int cus = swamp::device_info().num_cus;
  int grid = cus * std::max(1, tuning().waves_per_cu / nw);
  if (grid > n_tiles) grid = n_tiles;
  if (grid < 1) return SWAMP_OK;
  gemv_kernel<DT, kPPT, kRows><<<grid, T, 0, s>>>(ms, x, ipr, swamp::row_bytes(DT, n_cols), n_tiles);
  return hipGetLastError() == hipSuccess ? SWAMP_OK : SWAMP_ELAUNCH;
}

template <int DT>
int launch_dt(const MatSet &ms, const float *x, int n_cols, hipStream_t s) {
  const int ipr = n_cols / 64;
  if (ipr <= 512) return launch_items<DT, 1, 4>(ms, x, n_cols, s);
  if (ipr <= 1024) return launch_items<DT, 2, 4>(ms, x, n_cols, s);
  if (ipr <= 2048) return launch_items<DT, 4, 2>(ms, x, n_cols, s);
  return SWAMP_ESHAPE;
}

int build_matset(MatSet &ms, int n, const void *const *ws, float *const *ys, const int *rows,
                 int tile_rows) {
  ms.n = n;
  int acc = 0;
  for (int i = 0; i < n; i++) {
    ms.w[i] = static_cast<const uint8_t *>(ws[i]);
    ms.y[i] = ys[i];
    ms.rows[i] = rows[i];
    acc += (rows[i] + tile_rows - 1) / tile_rows;
    ms.tile_end[i] = acc;
  }
  return acc;
}

int dispatch(uint32_t dt, const MatSet &ms, const float *x, int n_cols, hipStream_t s) {
  switch (dt) {
  case SWAMP_Q4_0: return launch_dt<SWAMP_Q4_0>(ms, x, n_cols, s);
  case SWAMP_Q8_0: return launch_dt<SWAMP_Q8_0>(ms, x, n_cols, s);
  case SWAMP_Q4_K: return launch_dt<SWAMP_Q4_K>(ms, x, n_cols, s);
  default: return SWAMP_EDTYPE;
  }
}

int tile_rows_for(int n_cols) { return n_cols / 64 <= 1024 ? 4 : 2; }

}  // namespace

int swamp_launch_gemv(uint32_t dtype, const void *d_w, const float *d_x, float *d_y,
                      int n_rows, int n_cols, hipStream_t s) {
  if (n_rows == 0) return SWAMP_OK;
  const bool item_ok = dtype == SWAMP_Q4_K || n_cols % 64 == 0;
  if (!item_ok || n_cols / 64 > 2048) {
    if (dtype == SWAMP_Q4_K) return SWAMP_ESHAPE;
    const int cus = swamp::device_info().num_cus;
    const int blocks = std::min((n_rows + 3) / 4, cus * 8);
    if (dtype == SWAMP_Q4_0)
      gemv_generic_kernel<SWAMP_Q4_0><<<blocks, 256, 0, s>>>(
          static_cast<const uint8_t *>(d_w), d_x, d_y, n_rows, n_cols);
    else
      gemv_generic_kernel<SWAMP_Q8_0><<<blocks, 256, 0, s>>>(
          static_cast<const uint8_t *>(d_w), d_x, d_y, n_rows, n_cols);
    return hipGetLastError() == hipSuccess ? SWAMP_OK : SWAMP_ELAUNCH;
  }
  MatSet ms;
  const void *ws[1] = {d_w};
  float *ys[1] = {d_y};
  build_matset(ms, 1, ws, ys, &n_rows, tile_rows_for(n_cols));
  return dispatch(dtype, ms, d_x, n_cols, s);
}

int swamp_launch_gemv_multi(int n_mats, const uint32_t *dtypes, const void *const *d_ws,
                            const int *row_counts, const float *d_x, float *const *d_ys,
                            int n_cols, hipStream_t s) {
  // Matrices of one dtype share a launch (and the x prologue); a different
  // dtype starts another launch on the same stream.
  bool done[kMaxMats] = {};
  for (int i = 0; i < n_mats; i++) {
    if (done[i]) continue;
    const uint32_t dt = dtypes[i];
    const bool item_ok = dt == SWAMP_Q4_K || (n_cols % 64 == 0 && n_cols / 64 <= 2048);
    if (!item_ok) {
      for (int j = i; j < n_mats; j++)
        if (!done[j] && dtypes[j] == dt) {
          int rc = swamp_launch_gemv(dt, d_ws[j], d_x, d_ys[j], row_counts[j], n_cols, s);
          if (rc) return rc;
          done[j] = true;
        }
      continue;
    }
    const void *ws[kMaxMats];
    float *ys[kMaxMats];
    int rows[kMaxMats];
    int n = 0;
    for (int j = i; j < n_mats; j++)
      if (!done[j] && dtypes[j] == dt && row_counts[j] > 0) {
        ws[n] = d_ws[j];
        ys[n] = d_ys[j];
        rows[n] = row_counts[j];
        n++;
        done[j] = true;
      } else if (dtypes[j] == dt) {
        done[j] = true;
      }
    if (n == 0) continue;
    MatSet ms;
    build_matset(ms, n, ws, ys, rows, tile_rows_for(n_cols));
    int rc = dispatch(dt, ms, d_x, n_cols, s);
    if (rc) return rc;
  }
  return SWAMP_OK;
}
