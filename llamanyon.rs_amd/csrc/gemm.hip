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
//  * LDS: three activation stages and two dequantized-weight stages, 32 KB
//    each (160 KB).  Activations go global -> LDS directly (buffer_load ...
//    lds, no VGPRs, no LDS write instructions), two K steps ahead; weight
//    items go to registers two steps ahead and are dequantized one step
//    ahead into the other weight stage, in slices interleaved with the
//    current step's MFMAs, so the vector ALU and LDS work hides under the
//    matrix cores.  One barrier per step, which waits (in-order memory
//    counter) for the next step's activations only.
//  * Fragments of the next 16-wide k slice are read from LDS while the
//    current slice's 16 MFMAs run.
//  * Weight dequantization: lane t owns row t of the tile; one 64-weight
//    item per step becomes 8 chunks of 8 bf16 (byte -> float converts, one
//    fma each, packed RNE convert).
//  * LDS rows are 128 B; 16-byte chunks are XOR-swizzled by row so the
//    32-row fragment reads and the row-wise writes spread over the banks.
//  * Workgroup ids are remapped so each XCD (ids i, i+8, ...) walks a
//    contiguous run of tiles that share weight columns in its L2.
//  * The tiles of an incomplete last round (all tiles, when there are fewer
//    than CUs) are split along K across workgroups; those add into y
//    (their blocks zeroed first) with hardware float atomics.
#include "swamp_common.hpp"
#include "swamp_items.hpp"

#include <algorithm>
#include <mutex>

namespace {

using swamp::Raw;
using swamp::q4k_scales;
using swamp::shr16;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4v_t __attribute__((ext_vector_type(4)));

constexpr int kBM = 256, kBN = 256, kBK = 64;
constexpr int kThreads = 256;
constexpr int kXStage = kBM * kBK * 2;              // 32 KB activations
constexpr int kWStage = kBN * kBK * 2;              // 32 KB dequantized weights
constexpr int kXOff = 0, kWOff = 3 * kXStage;        // 3 activation + 2 weight stages
constexpr int kSmemBytes = 3 * kXStage + 2 * kWStage; // 160 KB

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

// Per-thread load geometry.  Activations go global -> LDS directly
// (buffer_load ... lds): instruction i of wave w fills LDS bytes
// [1024 (8w + i), +1024) of an activation stage = rows 8(8w+i) .. +7, lane L
// writing row 8(8w+i) + L/8, physical 16-byte chunk L%8; the lane fetches
// the logical chunk that the swizzle puts there.  The weight item is row
// n0 + tid, through registers (it is dequantized).
struct Geo {
  __amdgpu_buffer_rsrc_t xr, wr;
  uint32_t xv[2];   // per-lane VGPR offsets for even / odd instructions
  uint32_t xs;      // m0 * K * 2 (scalar)
  uint32_t xinst;   // 8 * K * 2: scalar step between instructions
  uint32_t wv;      // per-lane weight row offset
  int wave;
};

__device__ __forceinline__ void xdma(uint8_t *xstage, const Geo &g, int kt) {
#pragma unroll
  for (int i = 0; i < 8; i++)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        g.xr, (__attribute__((address_space(3))) void *)(xstage + 1024 * (8 * g.wave + i)), 16,
        g.xv[i & 1], g.xs + uint32_t(i) * g.xinst + uint32_t(kt) * 128u, 0, 0);
}

__device__ __forceinline__ void frags(const uint8_t *stg, const uint8_t *ws, int ks, int wm, int wn,
                                      int lane, bf16x8_t (&a)[4], bf16x8_t (&b)[4]) {
  const int fr = lane & 31, fc = lane >> 5;
#pragma unroll
  for (int i = 0; i < 4; i++)
    a[i] = *reinterpret_cast<const bf16x8_t *>(stg + swz(wm * 128 + i * 32 + fr, 2 * ks + fc));
#pragma unroll
  for (int j = 0; j < 4; j++)
    b[j] = *reinterpret_cast<const bf16x8_t *>(ws + swz(wn * 128 + j * 32 + fr, 2 * ks + fc));
}

template <int DT>
__host__ __device__ constexpr int wloads() {
  return DT == SWAMP_Q8_0 ? 5 : 3;  // buffer loads per weight item
}

// One K step: MFMAs on activation stage xc and weight stage wc.  Meanwhile
// step kt+2's activations stream into stage xf by DMA and its weight item
// into registers `fetch`; step kt+1's weight item (registers `nw`, loaded a
// step ago) is dequantized into weight stage wn.  The closing barrier waits
// (in-order memory counter) for step kt+1's DMA only: the loads issued
// after it -- kt+1's weights, kt+2's DMA and weights -- stay in flight.
template <int DT>
__device__ __forceinline__ void kstep(f32x16_t (&acc)[4][4], const uint8_t *xc, const uint8_t *wc,
                                      uint8_t *xf, uint8_t *wn, const Raw<DT> &nw,
                                      Raw<DT> &fetch, const Geo &g, int kt, int kt1, int tid) {
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave & 1, wn_ = wave >> 1;
  const int k1 = min(kt + 1, kt1 - 1), k2 = min(kt + 2, kt1 - 1);  // past the end: re-read
  xdma(xf, g, k2);
  __builtin_amdgcn_sched_barrier(0);
  load_item<DT>(fetch, g.wr, g.wv, k2);
  __builtin_amdgcn_sched_barrier(0);
  bf16x8_t a[2][4], b[2][4];
  frags(xc, wc, 0, wm, wn_, lane, a[0], b[0]);
#pragma unroll
  for (int ks = 0; ks < 4; ks++) {
    const int p = ks & 1;
    if (ks < 3) frags(xc, wc, ks + 1, wm, wn_, lane, a[p ^ 1], b[p ^ 1]);
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 4; j++)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[p][i], b[p][j], acc[i][j], 0, 0, 0);
#pragma unroll
    for (int q = 0; q < 2; q++) {
      const int c = 2 * ks + q;
      *reinterpret_cast<u32x4v_t *>(wn + swz(tid, c)) = dequant_chunk<DT>(nw, k1, c);
    }
#pragma unroll
    for (int m = 0; m < 16; m++) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);  // 5 VALU
      if (m < 8 && ks < 3) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // 1 DS read
      if (m == 9 || m == 13) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // 1 DS write
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  // wait for step kt+1's DMA (8 + 2 weight loads were issued after it)
  constexpr int kAfter = 8 + 2 * wloads<DT>();
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::"n"(kAfter) : "memory");
}

template <int DT>
__global__ void __launch_bounds__(kThreads, 1) gemm_bf16_kernel(
    const uint8_t *__restrict__ w, const uint16_t *__restrict__ x, float *__restrict__ y, int M,
    int N, int K, size_t row_bytes, int tiles_m, int n_full, int splits, int kt_per_split) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave & 1, wn = wave >> 1;

  // Work items: tiles [0, n_full) with their whole K range, then `splits`
  // K pieces of each remaining tile (added into y atomically; their y
  // blocks are zeroed first).  XCD-aware order: hardware ids i, i+8, ...
  // run on one XCD; each XCD gets a contiguous run of the (m-fastest) full
  // tiles -- M tiles sharing a weight column share that XCD's L2 -- and an
  // equal share of the pieces, which come last on every XCD.
  const int n_work = int(gridDim.x);
  const int n_piece = n_work - n_full;
  int L = blockIdx.x;
  if (n_full % 8 == 0 && n_piece % 8 == 0) {
    const int xcd = L % 8, loc = L / 8, f8 = n_full / 8, p8 = n_piece / 8;
    L = loc < f8 ? xcd * f8 + loc : n_full + xcd * p8 + (loc - f8);
  }
  const int KT = K / kBK;
  int tile, kt0, kt1, atomic;
  if (L < n_full) {
    tile = L;
    kt0 = 0;
    kt1 = KT;
    atomic = 0;
  } else {
    const int q = L - n_full;
    tile = n_full + q / splits;
    kt0 = (q % splits) * kt_per_split;
    kt1 = min(KT, kt0 + kt_per_split);
    atomic = 1;
  }
  const int mt = tile % tiles_m, nt = tile / tiles_m;
  const int m0 = mt * kBM, n0 = nt * kBN;

  Geo g;
  g.wave = __builtin_amdgcn_readfirstlane(wave);
  g.xr = swamp::make_rsrc(x, uint32_t(size_t(M) * K * 2));
  {
    // lane L of instruction i: row 8(8w+i) + L/8, physical chunk L%8,
    // logical chunk (L%8) ^ ((row >> 1) & 7) = (L%8) ^ ((4i + L/16) & 7)
    const int rl = wave * 64 + (lane >> 3);
#pragma unroll
    for (int par = 0; par < 2; par++) {
      const int c = (lane & 7) ^ ((4 * par + (lane >> 4)) & 7);
      g.xv[par] = uint32_t((rl * K + 8 * c) * 2);
    }
  }
  g.xs = uint32_t(size_t(m0) * K * 2);
  g.xinst = uint32_t(8 * K * 2);
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

  uint8_t *const X0 = smem + kXOff, *const W0 = smem + kWOff;
  auto xst = [&](int s) { return X0 + kXStage * s; };
  auto wst = [&](int s) { return W0 + kWStage * s; };
  Raw<DT> r0, r1;
  // prologue: step kt0 -> X0 (DMA) and W0 (dequant); kt0+1 -> X1 (DMA) and r1
  xdma(xst(0), g, kt0);
  __builtin_amdgcn_sched_barrier(0);
  load_item<DT>(r0, g.wr, g.wv, kt0);
  __builtin_amdgcn_sched_barrier(0);
  xdma(xst(1), g, min(kt0 + 1, kt1 - 1));
  __builtin_amdgcn_sched_barrier(0);
  load_item<DT>(r1, g.wr, g.wv, min(kt0 + 1, kt1 - 1));
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int c = 0; c < 8; c++)
    *reinterpret_cast<u32x4v_t *>(wst(0) + swz(tid, c)) = dequant_chunk<DT>(r0, kt0, c);
  {
    // step kt0's DMA done: kt0's weights, kt0+1's DMA and weights follow it
    constexpr int kAfter = 8 + 2 * wloads<DT>();
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::"n"(kAfter) : "memory");
  }

  // Two steps per trip (static register roles); LDS stages rotate with the
  // step: activations kt%3, weights kt%2 (counted from kt0).
  int kt = kt0;
  for (; kt + 1 < kt1; kt += 2) {
    const int j = kt - kt0;
    kstep<DT>(acc, xst(j % 3), wst(0), xst((j + 2) % 3), wst(1), r1, r0, g, kt, kt1, tid);
    kstep<DT>(acc, xst((j + 1) % 3), wst(1), xst((j + 3) % 3), wst(0), r0, r1, g, kt + 1, kt1, tid);
  }
  if (kt < kt1) {
    const int j = kt - kt0;
    kstep<DT>(acc, xst(j % 3), wst(0), xst((j + 2) % 3), wst(1), r1, r0, g, kt, kt1, tid);
  }

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

// Zero the y blocks of tiles [first, first + gridDim.x / 64): block b
// clears 4 rows of tile first + b/64, each thread 4 consecutive floats.
__global__ void zero_tiles_kernel(float *__restrict__ y, int M, int N, int tiles_m, int first) {
  const int tile = first + int(blockIdx.x) / 64;
  const int mt = tile % tiles_m, nt = tile / tiles_m;
  const int m = mt * kBM + 4 * (int(blockIdx.x) % 64) + int(threadIdx.x) / 64;
  const int n = nt * kBN + 4 * (int(threadIdx.x) % 64);
  if (m >= M) return;
  float *row = y + size_t(m) * N;
#pragma unroll
  for (int i = 0; i < 4; i++)
    if (n + i < N) row[n + i] = 0.f;
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
  // Balance the last round over the CUs (one workgroup per CU).  Split
  // pieces of a tile add into y with float atomics, which cost about as
  // much as a quarter of a round when every tile of a full round is split
  // (measured), so: fewer tiles than half the CUs -> every tile splits
  // along K into min(cus / tiles, 4) pieces; a last round at most half
  // full -> its tiles split in 2; otherwise no split.  Pieces are at least
  // 8 K steps long.
  const int cus = swamp::device_info().num_cus;
  const int rem = tiles % cus;
  int n_full = tiles, splits = 1;
  if (tiles * 2 <= cus) {
    splits = std::min({cus / tiles, 4, KT / 8});
    n_full = 0;
  } else if (tiles > cus && rem > 0 && rem * 2 <= cus) {
    splits = std::min(2, KT / 8);
    n_full = tiles - rem;
  }
  splits = std::max(1, splits);
  const int kt_per_split = (KT + splits - 1) / splits;
  splits = (KT + kt_per_split - 1) / kt_per_split;
  if (splits <= 1) n_full = tiles;
  const int n_work = n_full + (tiles - n_full) * splits;
  if (n_full < tiles)
    zero_tiles_kernel<<<unsigned((tiles - n_full) * 64), 256, 0, s>>>(d_y, m, n_rows, tiles_m, n_full);
  const dim3 grid{unsigned(n_work), 1u, 1u};
  const uint8_t *w = static_cast<const uint8_t *>(d_w);
  const uint16_t *x = static_cast<const uint16_t *>(d_x);
  const size_t rb = swamp::row_bytes(int(dtype), size_t(n_cols));
  switch (dtype) {
#define SWAMP_GEMM_CASE(DT)                                                                    \
  case DT:                                                                                     \
    if (int rc = set_smem_attr<DT>()) return rc;                                               \
    gemm_bf16_kernel<DT><<<grid, kThreads, kSmemBytes, s>>>(w, x, d_y, m, n_rows, n_cols, rb,  \
                                                            tiles_m, n_full, splits,           \
                                                            kt_per_split);                     \
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
