// gemv_batched.hip -- small-batch (2..16 tokens per pass) quantized GEMV on
// the matrix cores, for speculative verify and continuous batching.
//
// Replaces forward_linear_batch (swamp-engine/src/linear.rs:176-239) and
// fused_gemv_q4k_batched (swamp-kernels/src/fused_gemv_q4k.rs:527-554,
// scalar body :650-698).
//
// Still HBM-bound (at 16 tokens a Q4 weight byte feeds ~57 FLOP, the chip's
// balance is ~300), so the weights must stream exactly once per pass of 16
// tokens.  Layout of the work:
//  * V_MFMA_F32_16X16X32_F16 with A = activations (16 tokens x 32 k) and
//    B = weights (32 k x 16 rows); C = 16 tokens x 16 rows.
//  * A wave owns a 512-wide K slice.  Lane (r = l%16, g = l/16) owns items
//    2g and 2g+1 (64 weights each) of that slice for row r of the current
//    16-row tile, so a wave reads 16 rows x 288-576 contiguous bytes.
//  * The k order inside each MFMA is permuted so that a lane's 8 operand
//    values come from ONE nibble dword (Q4) or two int8 dwords (Q8_0); the
//    activation fragments, held in registers for the whole kernel, use the
//    same permutation, so the dot products are unchanged.
//  * Weights are dequantized to fp16 in registers: nibble -> fp16 (1024+q)
//    with one and-or per pair, then packed fp16 add/mul(-fma) apply the
//    offset and the block scale.  Activations are rounded to fp16.
//  * The 8 waves of a workgroup cover 4096 k; their 16x16 partial tiles are
//    summed through LDS once per row tile.  Longer rows use several K groups
//    (grid.y) that add into y atomically (y is zeroed first unless the call
//    accumulates).
#include "swamp_common.hpp"
#include "swamp_items.hpp"

namespace {

using swamp::Raw;
using swamp::load_raw;
using swamp::q4k_scales;
using swamp::shr16;

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));

constexpr int kWaves = 8;       // waves per workgroup
constexpr int kSlice = 512;     // k per wave
constexpr int kTok = 16;        // tokens per pass
constexpr int kRowsTile = 16;   // rows per tile
constexpr uint32_t kF16Magic = 0x64006400u;  // fp16 pair (1024, 1024)

__device__ __forceinline__ half2_t as_h2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }
__device__ __forceinline__ uint32_t as_u(half2_t h) { return __builtin_bit_cast(uint32_t, h); }

__device__ __forceinline__ uint32_t f16_rne_bits(float f) {
  return __builtin_bit_cast(uint16_t, _Float16(f));  // v_cvt_f16_f32, RNE
}

// Element (0..63 of the item) that operand slot i (0..7) of MFMA step st
// (0..7) multiplies.  Slot i = pair i/2, half i%2; pair p of a nibble dword
// holds the nibbles at bit offsets 4p and 4p+16 (P0..P3 = w>>0,4,8,12).
template <int DT>
__host__ __device__ constexpr int slot_elem(int st, int i) {
  const int p = i / 2, h = i % 2;
  if (DT == SWAMP_Q8_0) {
    // two int8 dwords per step; pair 0/1 of dword 0 -> bytes (0,2), (1,3)
    const int dw = p / 2, pb = p % 2;
    const int byte = pb + 2 * h;
    return 32 * (st / 4) + 8 * (st % 4) + 4 * dw + byte;
  }
  const int n = p + 4 * h;  // nibble index in the dword (bit 4n)
  if (DT == SWAMP_Q4_0) return 32 * (st / 4) + 8 * (st % 4) + n;  // interleaved: nibble n = element n
  // Q4_K quarter: dword st = bytes 4st..4st+3; low nibble -> sub-block A
  // element 4st + byte, high nibble -> sub-block B (item elements 32..63)
  return 32 * (n % 2) + 4 * st + n / 2;
}

// 8 fp16 weights (4 packed dwords) of MFMA step st from one item.
template <int DT>
__device__ __forceinline__ half8_t weights_step(const Raw<DT> &r, int st, int item) {
  uint32_t o[4];
  if constexpr (DT == SWAMP_Q4_0) {
    const int blk = st / 4, t = st % 4;
    const uint32_t w = blk == 0 ? shr16(r.d[t + 1], r.d[t]) : r.d[5 + t];
    const uint32_t dbits = blk == 0 ? (r.d[0] & 0xFFFFu) : (r.d[4] >> 16);
    const half2_t d2 = as_h2(dbits | (dbits << 16));
    const half2_t off = {_Float16(-1032.0f), _Float16(-1032.0f)};
#pragma unroll
    for (int p = 0; p < 4; p++) {
      const uint32_t P = ((w >> (4 * p)) & 0x000F000Fu) | kF16Magic;
      o[p] = as_u((as_h2(P) + off) * d2);  // (q - 8) exact, then one rounding
    }
  } else if constexpr (DT == SWAMP_Q8_0) {
    const int blk = st / 4, t = st % 4;
    uint32_t w0, w1, dbits;
    if (blk == 0) {
      w0 = shr16(r.d[2 * t + 1], r.d[2 * t]);
      w1 = shr16(r.d[2 * t + 2], r.d[2 * t + 1]);
      dbits = r.d[0] & 0xFFFFu;
    } else {
      w0 = r.d[9 + 2 * t];
      w1 = r.d[10 + 2 * t];
      dbits = r.d[8] >> 16;
    }
    const half2_t d2 = as_h2(dbits | (dbits << 16));
    const half2_t off = {_Float16(-1152.0f), _Float16(-1152.0f)};
    const uint32_t u0 = w0 ^ 0x80808080u, u1 = w1 ^ 0x80808080u;  // q + 128
    o[0] = as_u((as_h2((u0 & 0x00FF00FFu) | kF16Magic) + off) * d2);
    o[1] = as_u((as_h2(((u0 >> 8) & 0x00FF00FFu) | kF16Magic) + off) * d2);
    o[2] = as_u((as_h2((u1 & 0x00FF00FFu) | kF16Magic) + off) * d2);
    o[3] = as_u((as_h2(((u1 >> 8) & 0x00FF00FFu) | kF16Magic) + off) * d2);
  } else {
    const float d = swamp::f16_bits_to_f32(r.h[0] & 0xFFFFu);
    const float dmin = swamp::f16_bits_to_f32(r.h[0] >> 16);
    uint32_t sc0, m0, sc1, m1;
    q4k_scales(r.h, 2 * (item & 3), sc0, m0, sc1, m1);
    const _Float16 sa = _Float16(d * float(sc0)), ma = _Float16(-(dmin * float(m0)));
    const _Float16 sb = _Float16(d * float(sc1)), mb = _Float16(-(dmin * float(m1)));
    const half2_t off = {_Float16(-1024.0f), _Float16(-1024.0f)};
    const uint32_t w = r.q[st];
#pragma unroll
    for (int p = 0; p < 4; p++) {
      // pair p: nibbles at bits 4p and 4p+16; p even -> low nibbles (A)
      const uint32_t P = ((w >> (4 * p)) & 0x000F000Fu) | kF16Magic;
      const half2_t q = as_h2(P) + off;
      const bool a = (p % 2) == 0;
      const half2_t s2 = {a ? sa : sb, a ? sa : sb};
      const half2_t m2 = {a ? ma : mb, a ? ma : mb};
      o[p] = as_u(q * s2 + m2);
    }
  }
  half8_t v;
#pragma unroll
  for (int p = 0; p < 4; p++) {
    half2_t h = as_h2(o[p]);
    v[2 * p] = h[0];
    v[2 * p + 1] = h[1];
  }
  return v;
}

// y[t][row] for t < n_tok, rows [row0, row0+16).  mode: 0 = store,
// 1 = add (accumulate, single K group), 2 = atomic add (several K groups).
template <int DT>
__global__ void __launch_bounds__(512) gemv_batched_kernel(const uint8_t *__restrict__ w,
                                                           const float *__restrict__ x,
                                                           float *__restrict__ y, int n_tok,
                                                           int n_rows, int n_cols,
                                                           size_t row_bytes, int mode) {
  __shared__ float red[2][kWaves][kTok * kRowsTile];
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int r16 = lane & 15, g = lane >> 4;
  const int ipr = n_cols / 64;
  const int slice = blockIdx.y * kWaves + wave;  // K slice of this wave
  int item[2];
  bool valid[2];
#pragma unroll
  for (int j = 0; j < 2; j++) {
    item[j] = slice * (kSlice / 64) + 2 * g + j;
    valid[j] = item[j] < ipr;
  }

  // Activation fragments: token r16, items 2g+j, steps st: 8 fp16 each.
  half8_t xa[2][8];
#pragma unroll
  for (int j = 0; j < 2; j++) {
    float xv[64];
    const bool ok = valid[j] && r16 < n_tok;
    const float4 *xp = reinterpret_cast<const float4 *>(x + size_t(r16) * n_cols + size_t(item[j]) * 64);
#pragma unroll
    for (int i = 0; i < 16; i++) {
      float4 f = ok ? xp[i] : make_float4(0.f, 0.f, 0.f, 0.f);
      xv[4 * i] = f.x; xv[4 * i + 1] = f.y; xv[4 * i + 2] = f.z; xv[4 * i + 3] = f.w;
    }
#pragma unroll
    for (int st = 0; st < 8; st++)
#pragma unroll
      for (int i = 0; i < 8; i++) xa[j][st][i] = _Float16(xv[slot_elem<DT>(st, i)]);
  }

  const int n_tiles = (n_rows + kRowsTile - 1) / kRowsTile;
  int par = 0;
  for (int tile = blockIdx.x; tile < n_tiles; tile += gridDim.x, par ^= 1) {
    const int row = min(tile * kRowsTile + r16, n_rows - 1);  // clamped: in bounds
    const uint8_t *rp = w + size_t(row) * row_bytes;
    // Lanes past the end of the row keep all-zero bytes: scale 0 makes
    // their weights exactly 0, so every lane can join every MFMA (the
    // matrix instructions must run with the whole wave active).
    Raw<DT> raw[2] = {};
#pragma unroll
    for (int j = 0; j < 2; j++)
      if (valid[j]) load_raw<DT>(raw[j], rp, item[j]);
    float4_t c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 2; j++) {
#pragma unroll
      for (int st = 0; st < 8; st++) {
        const half8_t b = weights_step<DT>(raw[j], st, item[j]);
        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[j][st], b, c, 0, 0, 0);
      }
    }
    // C layout: lane holds tokens 4g..4g+3 of row r16.
#pragma unroll
    for (int i = 0; i < 4; i++) red[par][wave][(4 * g + i) * kRowsTile + r16] = c[i];
    __syncthreads();
    if (tid < kTok * kRowsTile) {
      const int t = tid / kRowsTile, rr = tid % kRowsTile;
      const int orow = tile * kRowsTile + rr;
      if (t < n_tok && orow < n_rows) {
        float v = 0.f;
#pragma unroll
        for (int wv = 0; wv < kWaves; wv++) v += red[par][wv][tid];
        float *dst = y + size_t(t) * n_rows + orow;
        if (mode == 0) *dst = v;
        else if (mode == 1) *dst += v;
        else atomicAdd(dst, v);
      }
    }
  }
}

__global__ void zero_kernel(float *__restrict__ p, size_t n) {
  const size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.f;
}

template <int DT>
int launch_pass(const uint8_t *w, const float *x, float *y, int n_tok, int n_rows, int n_cols,
                int accumulate, hipStream_t s) {
  const int ipr = n_cols / 64;
  const int slices = (ipr + kSlice / 64 - 1) / (kSlice / 64);
  const int groups = (slices + kWaves - 1) / kWaves;
  if (groups > 1 && !accumulate) {
    const size_t n = size_t(n_tok) * n_rows;
    zero_kernel<<<unsigned((n + 255) / 256), 256, 0, s>>>(y, n);
  }
  const int mode = groups > 1 ? 2 : (accumulate ? 1 : 0);
  const int n_tiles = (n_rows + kRowsTile - 1) / kRowsTile;
  const int cus = swamp::device_info().num_cus;
  int gx = std::max(1, cus * 2 / groups);
  if (gx > n_tiles) gx = n_tiles;
  gemv_batched_kernel<DT><<<dim3(gx, groups), kWaves * 64, 0, s>>>(
      w, x, y, n_tok, n_rows, n_cols, swamp::row_bytes(DT, n_cols), mode);
  return hipGetLastError() == hipSuccess ? SWAMP_OK : SWAMP_ELAUNCH;
}

}  // namespace

int swamp_launch_gemv_batched(uint32_t dtype, const void *d_w, const float *d_x, float *d_y,
                              int n_tok, int n_rows, int n_cols, int accumulate,
                              hipStream_t s) {
  if (n_rows == 0 || n_tok == 0) return SWAMP_OK;
  const uint8_t *w = static_cast<const uint8_t *>(d_w);
  for (int t0 = 0; t0 < n_tok; t0 += kTok) {
    const int nt = std::min(kTok, n_tok - t0);
    const float *x = d_x + size_t(t0) * n_cols;
    float *y = d_y + size_t(t0) * n_rows;
    int rc;
    switch (dtype) {
    case SWAMP_Q4_0: rc = launch_pass<SWAMP_Q4_0>(w, x, y, nt, n_rows, n_cols, accumulate, s); break;
    case SWAMP_Q8_0: rc = launch_pass<SWAMP_Q8_0>(w, x, y, nt, n_rows, n_cols, accumulate, s); break;
    case SWAMP_Q4_K: rc = launch_pass<SWAMP_Q4_K>(w, x, y, nt, n_rows, n_cols, accumulate, s); break;
    default: return SWAMP_EDTYPE;
    }
    if (rc) return rc;
  }
  return SWAMP_OK;
}
