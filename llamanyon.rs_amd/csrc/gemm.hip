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
//  * Two LDS stages (activations 32 KB + dequantized weights 32 KB each,
//    128 KB of the 160 KB) and two register stages: the global loads of
//    K step t+2 are issued while step t computes, and step t+1's bytes
//    (loaded during step t-1) are dequantized and written into the other
//    LDS stage in slices interleaved with step t's MFMAs, so the vector
//    ALU and LDS work hides under the matrix cores.  One barrier per step.
//  * Fragments of the next 16-wide k slice are read from LDS while the
//    current slice's 16 MFMAs run.
//  * Weight dequantization: lane t owns row t of the tile; one 64-weight
//    item per step becomes 8 chunks of 8 bf16 (byte -> float converts, one
//    fma each, packed RNE convert).
//  * LDS rows are 128 B; 16-byte chunks are XOR-swizzled by row so the
//    32-row fragment reads and the row-wise writes spread over the banks.
//  * Workgroup ids are remapped so each XCD (ids i, i+8, ...) walks a
//    contiguous run of tiles that share weight columns in its L2.
//  * Grids with fewer tiles than CUs split K across workgroups; those add
//    into y (zeroed first) with hardware float atomics.
#include "swamp_common.hpp"
#include "swamp_items.hpp"

#include <algorithm>
#include <mutex>

namespace {

using swamp::Raw;
using swamp::load_raw;
using swamp::q4k_scales;
using swamp::shr16;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4v_t __attribute__((ext_vector_type(4)));

constexpr int kBM = 256, kBN = 256, kBK = 64;
constexpr int kThreads = 256;
constexpr int kStageBytes = (kBM + kBN) * kBK * 2;  // 64 KB
constexpr int kSmemBytes = 2 * kStageBytes;         // 128 KB

#ifndef SWAMP_GEMM_SWZ
#define SWAMP_GEMM_SWZ 1
#endif
__device__ __forceinline__ int swz(int row, int chunk) {
#if SWAMP_GEMM_SWZ == 1
  return row * 128 + ((chunk ^ ((row >> 1) & 7)) << 4);
#else
  return row * 128 + ((chunk ^ (row & 7)) << 4);
#endif
}

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  bf16x2_t v;
  v[0] = (__bf16)a;
  v[1] = (__bf16)b;
  return __builtin_bit_cast(uint32_t, v);
}

// byte j of w as a float (V_CVT_F32_UBYTEj)
__device__ __forceinline__ float ubyte(uint32_t w, int j) { return float((w >> (8 * j)) & 0xFFu); }

// Chunk c (weights 8c .. 8c+7 of the item, natural k order) dequantized to
// 8 bf16.  Every value is q*s - o rounded once in fp32 (the fma is exact
// up to that rounding), then rounded to bf16.
template <int DT>
__device__ __forceinline__ u32x4v_t dequant_chunk(const Raw<DT> &r, int item, int c) {
  float v[8];
  if constexpr (DT == SWAMP_Q4_0) {
    // block c/4; chunk dword t = bytes 4t..4t+3 of the block's nibbles;
    // element 2b = low nibble of byte b, 2b+1 = high nibble (q4_0.rs:30-35)
    const int blk = c >> 2, t = c & 3;
    const uint32_t w = blk == 0 ? shr16(r.d[t + 1], r.d[t]) : r.d[5 + t];
    const float d = swamp::f16_bits_to_f32(blk == 0 ? (r.d[0] & 0xFFFFu) : (r.d[4] >> 16));
    const float o = -8.0f * d;
    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
#pragma unroll
    for (int b = 0; b < 4; b++) {
      v[2 * b] = __builtin_fmaf(ubyte(lo, b), d, o);
      v[2 * b + 1] = __builtin_fmaf(ubyte(hi, b), d, o);
    }
  } else if constexpr (DT == SWAMP_Q8_0) {
    const int blk = c >> 2, t = c & 3;
    uint32_t w0, w1;
    if (blk == 0) {
      w0 = shr16(r.d[2 * t + 1], r.d[2 * t]);
      w1 = shr16(r.d[2 * t + 2], r.d[2 * t + 1]);
    } else {
      w0 = r.d[9 + 2 * t];
      w1 = r.d[10 + 2 * t];
    }
    const float d = swamp::f16_bits_to_f32(blk == 0 ? (r.d[0] & 0xFFFFu) : (r.d[8] >> 16));
    const float o = -128.0f * d;  // bytes carry q + 128
    w0 ^= 0x80808080u;
    w1 ^= 0x80808080u;
#pragma unroll
    for (int b = 0; b < 4; b++) {
      v[b] = __builtin_fmaf(ubyte(w0, b), d, o);
      v[4 + b] = __builtin_fmaf(ubyte(w1, b), d, o);
    }
  } else {
    // chunk c < 4: sub-block A elements 8c.. = low nibbles of bytes 8c..;
    // c >= 4: sub-block B = high nibbles of bytes 8(c-4).. (layout A,
    // q4_k.rs:290-319)
    const float d = swamp::f16_bits_to_f32(r.h[0] & 0xFFFFu);
    const float dmin = swamp::f16_bits_to_f32(r.h[0] >> 16);
    uint32_t sc0, m0, sc1, m1;
    q4k_scales(r.h, 2 * (item & 3), sc0, m0, sc1, m1);
    const bool hi = c >= 4;
    const float s = d * float(hi ? sc1 : sc0), o = -(dmin * float(hi ? m1 : m0));
    const int cc = c & 3;
    const uint32_t w0 = hi ? (r.q[2 * cc] >> 4) : r.q[2 * cc];
    const uint32_t w1 = hi ? (r.q[2 * cc + 1] >> 4) : r.q[2 * cc + 1];
    const uint32_t a0 = w0 & 0x0F0F0F0Fu, a1 = w1 & 0x0F0F0F0Fu;
#pragma unroll
    for (int b = 0; b < 4; b++) {
      v[b] = __builtin_fmaf(ubyte(a0, b), s, o);
      v[4 + b] = __builtin_fmaf(ubyte(a1, b), s, o);
    }
  }
  return u32x4v_t{pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]), pack_bf16(v[4], v[5]),
                  pack_bf16(v[6], v[7])};
}

// Raw bytes of one weight item through a buffer resource: the lane's row in
// the VGPR offset, the item's byte offset within a row in the (uniform) SGPR
// offset.  Reads past the descriptor's range return zeros.
template <int DT>
__device__ __forceinline__ void load_item(Raw<DT> &r, __amdgpu_buffer_rsrc_t rs, uint32_t vrow,
                                          int item) {
  if constexpr (DT == SWAMP_Q4_0) {
    const uint32_t so = uint32_t(item) * 36u;
    const u32x4v_t a = __builtin_amdgcn_raw_buffer_load_b128(rs, vrow, so, 0);
    const u32x4v_t b = __builtin_amdgcn_raw_buffer_load_b128(rs, vrow + 16, so, 0);
#pragma unroll
    for (int i = 0; i < 4; i++) { r.d[i] = a[i]; r.d[4 + i] = b[i]; }
    r.d[8] = __builtin_amdgcn_raw_buffer_load_b32(rs, vrow + 32, so, 0);
  } else if constexpr (DT == SWAMP_Q8_0) {
    const uint32_t so = uint32_t(item) * 68u;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const u32x4v_t a = __builtin_amdgcn_raw_buffer_load_b128(rs, vrow + 16 * j, so, 0);
#pragma unroll
      for (int i = 0; i < 4; i++) r.d[4 * j + i] = a[i];
    }
    r.d[16] = __builtin_amdgcn_raw_buffer_load_b32(rs, vrow + 64, so, 0);
  } else {
    const uint32_t hb = uint32_t(item >> 2) * 144u;
    const uint32_t so = hb + 16u + 32u * uint32_t(item & 3);
    const u32x4v_t h = __builtin_amdgcn_raw_buffer_load_b128(rs, vrow, hb, 0);
    const u32x4v_t a = __builtin_amdgcn_raw_buffer_load_b128(rs, vrow, so, 0);
    const u32x4v_t b = __builtin_amdgcn_raw_buffer_load_b128(rs, vrow + 16, so, 0);
#pragma unroll
    for (int i = 0; i < 4; i++) { r.h[i] = h[i]; r.q[i] = a[i]; r.q[4 + i] = b[i]; }
  }
}

// Per-thread load geometry.  Activation chunk i of a step is row
// m0 + 32 i + tid/8, 16-byte chunk tid%8 of the step's 128 bytes; rows past
// M read zeros (descriptor range).  The weight item is row n0 + tid.
struct Geo {
  __amdgpu_buffer_rsrc_t xr, wr;
  uint32_t xv, wv;  // per-lane VGPR offsets
  uint32_t xs;      // m0 * K * 2 (scalar)
  uint32_t xrow;    // 32 * K * 2: scalar step between chunks i
  int xoff[8];      // LDS byte offsets of the chunks (swizzled)
};

__device__ __forceinline__ void xload(u32x4v_t (&xb)[8], const Geo &g, int kt) {
#pragma unroll
  for (int i = 0; i < 8; i++)
    xb[i] = __builtin_amdgcn_raw_buffer_load_b128(g.xr, g.xv,
                                                 g.xs + uint32_t(i) * g.xrow + uint32_t(kt) * 128u, 0);
}

__device__ __forceinline__ void frags(const uint8_t *stg, int ks, int wm, int wn, int lane,
                                      bf16x8_t (&a)[4], bf16x8_t (&b)[4]) {
  const uint8_t *ws = stg + kBM * kBK * 2;
  const int fr = lane & 31, fc = lane >> 5;
#pragma unroll
  for (int i = 0; i < 4; i++)
    a[i] = *reinterpret_cast<const bf16x8_t *>(stg + swz(wm * 128 + i * 32 + fr, 2 * ks + fc));
#pragma unroll
  for (int j = 0; j < 4; j++)
    b[j] = *reinterpret_cast<const bf16x8_t *>(ws + swz(wn * 128 + j * 32 + fr, 2 * ks + fc));
}

// Register stage of one K step: its 8 activation chunks and weight item.
template <int DT>
struct Stage {
  u32x4v_t x[8];
  Raw<DT> w;
};

template <int DT>
__device__ __forceinline__ void sload(Stage<DT> &st, const Geo &g, int kt) {
  xload(st.x, g, kt);
  load_item<DT>(st.w, g.wr, g.wv, kt);
}

// One K step on LDS stage `cur`: 4 slices of 16 MFMAs.  Meanwhile step
// kt+1 (registers `nx`, loaded during step kt-1) goes to LDS stage `nxt`
// -- its activations at once, its weights dequantized two chunks per
// slice -- and step kt+2's global loads land in `fetch`.  Within a slice the
// scheduler is told to alternate one MFMA with three other VALU
// instructions, so the vector work runs in the MFMAs' shadow (a wave
// issues in order: a run of MFMAs stalls it while the matrix pipe is busy,
// a run of VALU leaves the matrix pipe idle).
template <int DT>
__device__ __forceinline__ void kstep(f32x16_t (&acc)[4][4], const uint8_t *cur, uint8_t *nxt,
                                      const Stage<DT> &nx, Stage<DT> &fetch, const Geo &g,
                                      int kt, int kt1, int tid) {
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave & 1, wn = wave >> 1;
  const int k1 = min(kt + 1, kt1 - 1), k2 = min(kt + 2, kt1 - 1);  // past the end: re-read
  sload<DT>(fetch, g, k2);
  // keep the loads at the top of the step (the scheduler would sink them
  // next to their first use and expose their latency)
  __builtin_amdgcn_sched_barrier(0);
  // step kt+1's activations (loaded a step ago) go to LDS first, freeing
  // their registers for the rest of the step
#pragma unroll
  for (int c = 0; c < 8; c++) *reinterpret_cast<u32x4v_t *>(nxt + g.xoff[c]) = nx.x[c];
  uint8_t *ws = nxt + kBM * kBK * 2;
  bf16x8_t a[2][4], b[2][4];
  frags(cur, 0, wm, wn, lane, a[0], b[0]);
#pragma unroll
  for (int ks = 0; ks < 4; ks++) {
    const int p = ks & 1;
    if (ks < 3) frags(cur, ks + 1, wm, wn, lane, a[p ^ 1], b[p ^ 1]);
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 4; j++)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[p][i], b[p][j], acc[i][j], 0, 0, 0);
#pragma unroll
    for (int q = 0; q < 2; q++) {
      const int c = 2 * ks + q;
      *reinterpret_cast<u32x4v_t *>(ws + swz(tid, c)) = dequant_chunk<DT>(nx.w, k1, c);
    }
#pragma unroll
    for (int m = 0; m < 16; m++) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);  // 5 VALU
      if (m < 8 && ks < 3) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // 1 DS read
      if (m == 9 || m == 13) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // 1 DS write
    }
    // slice boundary: the next slice's fragment reads stay in this slice
    __builtin_amdgcn_sched_barrier(0);
  }
  __syncthreads();
}

template <int DT>
__global__ void __launch_bounds__(kThreads, 1) gemm_bf16_kernel(
    const uint8_t *__restrict__ w, const uint16_t *__restrict__ x, float *__restrict__ y, int M,
    int N, int K, size_t row_bytes, int tiles_m, int tiles_n, int kt_per_split, int atomic) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave & 1, wn = wave >> 1;

  // XCD-aware tile order: hardware ids i, i+8, ... run on one XCD; give
  // each XCD a contiguous slice of the (m-fastest) tile sequence, so the
  // M tiles sharing a weight column share that XCD's L2.
  const int tiles = tiles_m * tiles_n;
  const int total = tiles * int(gridDim.y);
  int L = blockIdx.x + blockIdx.y * gridDim.x;
  if (total % 8 == 0) L = (L % 8) * (total / 8) + L / 8;
  const int split = L / tiles, tile = L % tiles;
  const int mt = tile % tiles_m, nt = tile / tiles_m;
  const int m0 = mt * kBM, n0 = nt * kBN;
  const int KT = K / kBK;
  const int kt0 = split * kt_per_split;
  const int kt1 = min(KT, kt0 + kt_per_split);

  Geo g;
  g.xr = swamp::make_rsrc(x, uint32_t(size_t(M) * K * 2));
  g.xv = uint32_t(((tid >> 3) * K + 8 * (tid & 7)) * 2);
  g.xs = uint32_t(size_t(m0) * K * 2);
  g.xrow = uint32_t(32 * K * 2);
#pragma unroll
  for (int i = 0; i < 8; i++) g.xoff[i] = swz(i * 32 + (tid >> 3), tid & 7);
  const int nrows = min(kBN, N - n0);
  g.wr = swamp::make_rsrc(w + size_t(n0) * row_bytes, uint32_t(size_t(nrows) * row_bytes));
  g.wv = uint32_t(size_t(tid) * row_bytes);

  f32x16_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;

  Stage<DT> s0, s1;
  uint8_t *const st0 = smem, *const st1 = smem + kStageBytes;
  // prologue: step kt0 into LDS stage 0, step kt0+1 in registers
  sload<DT>(s0, g, kt0);
  sload<DT>(s1, g, min(kt0 + 1, kt1 - 1));
  {
    uint8_t *ws = st0 + kBM * kBK * 2;
#pragma unroll
    for (int c = 0; c < 8; c++) {
      *reinterpret_cast<u32x4v_t *>(st0 + g.xoff[c]) = s0.x[c];
      *reinterpret_cast<u32x4v_t *>(ws + swz(tid, c)) = dequant_chunk<DT>(s0.w, kt0, c);
    }
  }
  __syncthreads();

  // Two steps per trip so the register stages keep static roles (a copy
  // between them would wait for the in-flight loads); the odd last step
  // runs after the loop (a break inside the trip made the register
  // allocator spill).
  int kt = kt0;
  for (; kt + 1 < kt1; kt += 2) {
    kstep<DT>(acc, st0, st1, s1, s0, g, kt, kt1, tid);
    kstep<DT>(acc, st1, st0, s0, s1, g, kt + 1, kt1, tid);
  }
  if (kt < kt1) kstep<DT>(acc, st0, st1, s1, s0, g, kt, kt1, tid);

  // C layout of a 32x32 tile: lane holds column (lane & 31), rows
  // 8*(e/4) + 4*(lane/32) + (e%4) for e = 0..15.
  const int fr = lane & 31, fc = lane >> 5;
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int n = n0 + wn * 128 + j * 32 + fr;
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const int m = m0 + wm * 128 + i * 32 + 8 * (e >> 2) + 4 * fc + (e & 3);
        if (m < M && n < N) {
          float *dst = y + size_t(m) * N + n;
          if (atomic) unsafeAtomicAdd(dst, acc[i][j][e]);
          else *dst = acc[i][j][e];
        }
      }
    }
}

__global__ void zero_f32_kernel(float *__restrict__ p, size_t n) {
  const size_t stride = size_t(gridDim.x) * blockDim.x;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = 0.f;
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

template <int DT>
int set_smem_attr() {
  static std::once_flag once;
  static hipError_t err = hipSuccess;
  std::call_once(once, [] {
    err = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemm_bf16_kernel<DT>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, kSmemBytes);
  });
  return err == hipSuccess ? SWAMP_OK : SWAMP_ELAUNCH;
}

}  // namespace

int swamp_launch_gemm(uint32_t dtype, const void *d_w, const void *d_x, uint32_t x_type,
                      float *d_y, int m, int n_rows, int n_cols, hipStream_t s) {
  if (m == 0 || n_rows == 0) return SWAMP_OK;
  if (x_type == SWAMP_Q8_0) return swamp_launch_gemm_i8(dtype, d_w, d_x, d_y, m, n_rows, n_cols, s);
  if (x_type != SWAMP_BF16) return SWAMP_EDTYPE;
  if (n_cols % kBK != 0) return SWAMP_ESHAPE;
  const int tiles_m = (m + kBM - 1) / kBM, tiles_n = (n_rows + kBN - 1) / kBN;
  const int tiles = tiles_m * tiles_n;
  const int KT = n_cols / kBK;
  // Split K when the tiles leave CUs idle: as many splits as fit in one
  // pass over the CUs, each at least 8 K steps long.
  const int cus = swamp::device_info().num_cus;
  int splits = std::max(1, std::min(cus / std::max(1, tiles), KT / 8));
  const int kt_per_split = (KT + splits - 1) / splits;
  splits = (KT + kt_per_split - 1) / kt_per_split;
  const int atomic = splits > 1 ? 1 : 0;
  if (atomic) {
    const size_t n = size_t(m) * n_rows;
    zero_f32_kernel<<<unsigned(std::min<size_t>((n + 255) / 256, size_t(cus) * 16)), 256, 0, s>>>(
        d_y, n);
  }
  const dim3 grid{unsigned(tiles), unsigned(splits), 1u};
  const uint8_t *w = static_cast<const uint8_t *>(d_w);
  const uint16_t *x = static_cast<const uint16_t *>(d_x);
  const size_t rb = swamp::row_bytes(int(dtype), size_t(n_cols));
  switch (dtype) {
#define SWAMP_GEMM_CASE(DT)                                                                    \
  case DT:                                                                                     \
    if (int rc = set_smem_attr<DT>()) return rc;                                               \
    gemm_bf16_kernel<DT><<<grid, kThreads, kSmemBytes, s>>>(w, x, d_y, m, n_rows, n_cols, rb,  \
                                                            tiles_m, tiles_n, kt_per_split,    \
                                                            atomic);                           \
    break;
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
