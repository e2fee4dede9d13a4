// gemm_i8.hip -- prefill GEMM with int8 matrix cores against Q8_0-quantized
// activations: y[m][r] = sum_b d_w[r,b] d_x[m,b] sum_{i in b} qw[r,i] qx[m,i]
// for Q4_0 (qw = nibble - 8) or Q8_0 (qw = int8) weights.  Q4_K weights
// (W = d sc q - dmin m per 32-weight sub-block, q4_k.rs:278-321) take
// qw = q (0..15), d_w = d sc, and subtract dmin m d_x sum_{i in b} qx[m,i]
// per block: the same dot, regrouped.
//
// Replaces, like gemm.hip, the prefill use of forward_linear_batch
// (swamp-engine/src/executor.rs:106-110 -> linear.rs:176-239), with the
// activations quantized per 32-block to Q8_0 first (swamp_quantize_q8_0).
//
// Shape of the work (one 32-weight block = one V_MFMA_I32_32X32X32_I8):
//  * Workgroup tile 128 tokens x 128 weight rows, K step 128 (four
//    blocks), 4 waves in 2 x 2, each 64 x 64 = 2 x 2 MFMA tiles.
//  * Per K step the raw activation and weight blocks of the tile are
//    loaded into registers (one step ahead), unpacked into an LDS stage as
//    int8 rows (Q4_0 nibbles become q - 8 with one byte-wise add and xor)
//    plus per-block fp32 scales; two LDS stages, one barrier per step.
//  * Each block's int32 32 x 32 result is converted and added into the
//    fp32 accumulators with its scale product d_x d_w: two vector ops per
//    output element per block (convert, FMA).  The products are an outer
//    product of the block's scale vectors, d_x per token and d_w per weight
//    row, and come from one V_MFMA_F32_32X32X1_2B_F32 per pair of tiles, in
//    the int32 result's own layout.  They are exact: each is an fp16 times an
//    fp16 (Q4_K: times d sc, an fp16 times a 6-bit code).  For Q4_K the same
//    instruction adds the minimum term's outer product into the accumulators.
//    With a scale per 32-block on both sides the per-element convert and FMA
//    still bound the kernel: the 32-deep int8 MFMA does 32 MACs per element
//    in the time the vector ALU does about five element ops.
//  * The two MFMA operands are read with the same per-lane byte rule, so
//    the dot over a block does not depend on how the instruction orders k
//    inside the block.
#include "swamp_common.hpp"
#include "swamp_items.hpp"

#include <algorithm>
#include <mutex>
#include <type_traits>

namespace {

using swamp::Raw;
using swamp::shr16;

typedef int32_t i32x4_t __attribute__((ext_vector_type(4)));
typedef int32_t i32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x32_t __attribute__((ext_vector_type(32)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4v_t __attribute__((ext_vector_type(4)));

constexpr int kBM = 128, kBN = 128, kBlk = 4;  // K step = 4 blocks of 32
constexpr int kThreads = 256;
// LDS stage: activation quants [128][128 B], weight quants [128][128 B],
// activation scales [4][128] f32, weight scales [4][128] f32.
constexpr int kQBytes = kBM * kBlk * 32;  // 16 KB
constexpr int kSBytes = kBlk * kBM * 4;   // 2 KB
// Q4_K adds two scale arrays: the weight minimums dmin * m [4][128] and
// the activation block sums d_x * sum(qx) [4][128].
template <int DT>
constexpr int stage_bytes() {
  return 2 * kQBytes + (DT == SWAMP_Q4_K ? 4 : 2) * kSBytes;
}
template <int DT>
constexpr int smem_bytes() {  // 72 KB, Q4_K 80 KB (two workgroups per CU)
  return 2 * stage_bytes<DT>();
}
static_assert(2 * smem_bytes<SWAMP_Q4_K>() <= 160 * 1024, "two Q4_K workgroups per CU");

// 16-byte chunk `chunk` (0..7) of quant row `row`, XOR-swizzled by row
// pairs (the 16-row groups of a fragment read hit 16 distinct bank quads).
__device__ __forceinline__ int qswz(int row, int chunk) {
  return row * 128 + ((chunk ^ ((row >> 1) & 7)) << 4);
}

// Q4_0 nibble dword (bytes b0..b3) -> 8 int8 values q - 8 in element order
// lo(b0), hi(b0), lo(b1), hi(b1) | lo(b2), hi(b2), lo(b3), hi(b3).
__device__ __forceinline__ void nib_to_i8(uint32_t w, uint32_t &o0, uint32_t &o1) {
  const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
  // interleave bytes: o0 = lo0 hi0 lo1 hi1, o1 = lo2 hi2 lo3 hi3
  o0 = __builtin_amdgcn_perm(hi, lo, 0x05010400u);
  o1 = __builtin_amdgcn_perm(hi, lo, 0x07030602u);
  // q - 8 per byte without borrows: (q + 0x78) ^ 0x80, q + 0x78 <= 0x87
  o0 = (o0 + 0x78787878u) ^ 0x80808080u;
  o1 = (o1 + 0x78787878u) ^ 0x80808080u;
}

struct Geo {
  __amdgpu_buffer_rsrc_t xr, wr;
  uint32_t xv, wv;  // per-thread VGPR offsets (row start + half)
  int row, half;    // tile row this thread unpacks, which two blocks
};

// Raw bytes of step kt for this thread: two activation Q8_0 blocks (68 B)
// and two weight blocks (one Q4_0 item of 36 B, two Q8_0 blocks of 68 B,
// or a Q4_K quarter: the super-block's 16-byte header and 32 nibble bytes).
template <int DT>
struct Stage {
  Raw<SWAMP_Q8_0> x;
  Raw<DT> w;
};

__device__ __forceinline__ void load_q8_pair(Raw<SWAMP_Q8_0> &r, __amdgpu_buffer_rsrc_t rs,
                                             uint32_t v, uint32_t s) {
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const u32x4v_t a = __builtin_amdgcn_raw_buffer_load_b128(rs, v + 16 * j, s, 0);
#pragma unroll
    for (int i = 0; i < 4; i++) r.d[4 * j + i] = a[i];
  }
  r.d[16] = __builtin_amdgcn_raw_buffer_load_b32(rs, v + 64, s, 0);
}

template <int DT>
__device__ __forceinline__ void sload(Stage<DT> &st, const Geo &g, int kt) {
  load_q8_pair(st.x, g.xr, g.xv, uint32_t(kt) * 136u);
  if constexpr (DT == SWAMP_Q4_0) {
    const uint32_t s = uint32_t(kt) * 72u;
    const u32x4v_t a = __builtin_amdgcn_raw_buffer_load_b128(g.wr, g.wv, s, 0);
    const u32x4v_t b = __builtin_amdgcn_raw_buffer_load_b128(g.wr, g.wv + 16, s, 0);
#pragma unroll
    for (int i = 0; i < 4; i++) { st.w.d[i] = a[i]; st.w.d[4 + i] = b[i]; }
    st.w.d[8] = __builtin_amdgcn_raw_buffer_load_b32(g.wr, g.wv + 32, s, 0);
  } else if constexpr (DT == SWAMP_Q4_K) {
    // item 2 kt + half = quarter 2 (kt & 1) + half of super-block kt / 2:
    // its 16-byte header and 32 nibble bytes (g.wv = row start + 16 + 32 half)
    const uint32_t sb = uint32_t(kt >> 1) * 144u;
    const u32x4v_t h = __builtin_amdgcn_raw_buffer_load_b128(g.wr, g.wv - 16u - 32u * uint32_t(g.half),
                                                             sb, 0);
    const uint32_t sq = sb + 64u * uint32_t(kt & 1);
    const u32x4v_t a = __builtin_amdgcn_raw_buffer_load_b128(g.wr, g.wv, sq, 0);
    const u32x4v_t b = __builtin_amdgcn_raw_buffer_load_b128(g.wr, g.wv + 16, sq, 0);
#pragma unroll
    for (int i = 0; i < 4; i++) { st.w.h[i] = h[i]; st.w.q[i] = a[i]; st.w.q[4 + i] = b[i]; }
  } else {
    load_q8_pair(st.w, g.wr, g.wv, uint32_t(kt) * 136u);
  }
}

// Two Q8_0 blocks (17 dwords, block 0's quants start at byte 2) -> two
// quant chunks of 32 B each and two scales; with `sums`, also each block's
// d * sum(q) (exact: |sum| <= 4096 times an fp16 fits fp32's 24 bits).
__device__ __forceinline__ void unpack_q8_pair(const Raw<SWAMP_Q8_0> &r, uint8_t *q, float *s,
                                               float *sums, const Geo &g) {
#pragma unroll
  for (int b = 0; b < 2; b++) {
    uint32_t v[8];
#pragma unroll
    for (int t = 0; t < 8; t++) v[t] = b == 0 ? shr16(r.d[t + 1], r.d[t]) : r.d[9 + t];
    const int blk = 2 * g.half + b;
    *reinterpret_cast<u32x4v_t *>(q + qswz(g.row, 2 * blk)) = u32x4v_t{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<u32x4v_t *>(q + qswz(g.row, 2 * blk + 1)) = u32x4v_t{v[4], v[5], v[6], v[7]};
    const float d = swamp::f16_bits_to_f32(b == 0 ? (r.d[0] & 0xFFFFu) : (r.d[8] >> 16));
    s[blk * kBM + g.row] = d;
    if (sums) {
      int sum = 0;
#pragma unroll
      for (int t = 0; t < 8; t++) sum = __builtin_amdgcn_sdot4(int(v[t]), 0x01010101, sum, false);
      sums[blk * kBM + g.row] = d * float(sum);
    }
  }
}

template <int DT>
__device__ __forceinline__ void lstore(uint8_t *stg, const Stage<DT> &st, const Geo &g, int kt) {
  uint8_t *xq = stg, *wq = stg + kQBytes;
  float *xs = reinterpret_cast<float *>(stg + 2 * kQBytes);
  float *wsc = xs + kBlk * kBM;
  float *wmn = wsc + kBlk * kBM, *xsum = wmn + kBlk * kBM;  // Q4_K only
  unpack_q8_pair(st.x, xq, xs, DT == SWAMP_Q4_K ? xsum : nullptr, g);
  if constexpr (DT == SWAMP_Q4_K) {
    // quarter 2 (kt & 1) + half: sub-block 2 quarter (low nibbles, block
    // 2 half of the step) and 2 quarter + 1 (high nibbles, block 2 half + 1)
    const int quarter = 2 * (kt & 1) + g.half;
    uint32_t sc0, m0, sc1, m1;
    swamp::q4k_scales(st.w.h, 2 * quarter, sc0, m0, sc1, m1);
    const float d = swamp::f16_bits_to_f32(st.w.h[0] & 0xFFFFu);
    const float dmin = swamp::f16_bits_to_f32(st.w.h[0] >> 16);
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int t = 0; t < 8; t++) {
      lo[t] = st.w.q[t] & 0x0F0F0F0Fu;
      hi[t] = (st.w.q[t] >> 4) & 0x0F0F0F0Fu;
    }
    const int b0 = 2 * g.half, b1 = b0 + 1;
    *reinterpret_cast<u32x4v_t *>(wq + qswz(g.row, 2 * b0)) = u32x4v_t{lo[0], lo[1], lo[2], lo[3]};
    *reinterpret_cast<u32x4v_t *>(wq + qswz(g.row, 2 * b0 + 1)) = u32x4v_t{lo[4], lo[5], lo[6], lo[7]};
    *reinterpret_cast<u32x4v_t *>(wq + qswz(g.row, 2 * b1)) = u32x4v_t{hi[0], hi[1], hi[2], hi[3]};
    *reinterpret_cast<u32x4v_t *>(wq + qswz(g.row, 2 * b1 + 1)) = u32x4v_t{hi[4], hi[5], hi[6], hi[7]};
    // exact products (an fp16 times a 6-bit code), as the dequantizer forms them
    wsc[b0 * kBM + g.row] = d * float(sc0);
    wsc[b1 * kBM + g.row] = d * float(sc1);
    wmn[b0 * kBM + g.row] = dmin * float(m0);
    wmn[b1 * kBM + g.row] = dmin * float(m1);
  } else if constexpr (DT == SWAMP_Q4_0) {
#pragma unroll
    for (int b = 0; b < 2; b++) {
      uint32_t v[8];
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const uint32_t w = b == 0 ? shr16(st.w.d[t + 1], st.w.d[t]) : st.w.d[5 + t];
        nib_to_i8(w, v[2 * t], v[2 * t + 1]);
      }
      const int blk = 2 * g.half + b;
      *reinterpret_cast<u32x4v_t *>(wq + qswz(g.row, 2 * blk)) = u32x4v_t{v[0], v[1], v[2], v[3]};
      *reinterpret_cast<u32x4v_t *>(wq + qswz(g.row, 2 * blk + 1)) =
          u32x4v_t{v[4], v[5], v[6], v[7]};
      wsc[blk * kBM + g.row] =
          swamp::f16_bits_to_f32(b == 0 ? (st.w.d[0] & 0xFFFFu) : (st.w.d[4] >> 16));
    }
  } else {
    unpack_q8_pair(st.w, wq, wsc, nullptr, g);
  }
}

// One K step (four blocks) on LDS stage `stg`.  acc[j] holds the wave's two
// 32 x 32 tiles of weight tile j: element 16 i + e is tile (i, j)'s element e.
template <int DT>
__device__ __forceinline__ void compute(f32x32_t (&acc)[2], const uint8_t *stg, int wm, int wn,
                                        int lane) {
  const uint8_t *xq = stg, *wq = stg + kQBytes;
  const float *xs = reinterpret_cast<const float *>(stg + 2 * kQBytes);
  const float *wsc = xs + kBlk * kBM;
  const float *wmn = wsc + kBlk * kBM, *xsum = wmn + kBlk * kBM;  // Q4_K only
  const int fr = lane & 31, fc = lane >> 5;
  // one block per trip, not unrolled: the int32 tiles and scale products of
  // four unrolled blocks would all be live at once
#pragma unroll 1
  for (int blk = 0; blk < kBlk; blk++) {
    i32x4_t a[2], b[2];
#pragma unroll
    for (int i = 0; i < 2; i++)
      a[i] = *reinterpret_cast<const i32x4_t *>(xq + qswz(wm * 64 + i * 32 + fr, 2 * blk + fc));
#pragma unroll
    for (int j = 0; j < 2; j++)
      b[j] = *reinterpret_cast<const i32x4_t *>(wq + qswz(wn * 64 + j * 32 + fr, 2 * blk + fc));
    // Operands of the two-block outer products: lane l carries row l & 31
    // of activation tile i = l >> 5 (row wm 64 + l) and column l & 31 of
    // weight tile j (the same column for both blocks).
    const float dxl = xs[blk * kBM + wm * 64 + lane];
    float sxl = 0.f;
    if constexpr (DT == SWAMP_Q4_K) sxl = xsum[blk * kBM + wm * 64 + lane];
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int c = wn * 64 + j * 32 + fr;
      const f32x32_t zero32 = {};
      // d_x d_w for every element of tiles (0, j) and (1, j)
      const f32x32_t sc = __builtin_amdgcn_mfma_f32_32x32x1f32(dxl, wsc[blk * kBM + c], zero32, 0, 0, 0);
      // Q4_K's minimum term -dmin m * d_x sum(qx), accumulated directly
      if constexpr (DT == SWAMP_Q4_K)
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x1f32(sxl, -wmn[blk * kBM + c], acc[j], 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 2; i++) {
        const i32x16_t zero = {};
        const i32x16_t q = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], zero, 0, 0, 0);
#pragma unroll
        for (int e = 0; e < 16; e++)
          acc[j][16 * i + e] = __builtin_fmaf(float(q[e]), sc[16 * i + e], acc[j][16 * i + e]);
      }
    }
  }
}

template <int DT>
__global__ void __launch_bounds__(kThreads, 2) gemm_i8_kernel(
    const uint8_t *__restrict__ w, const uint8_t *__restrict__ xq8, float *__restrict__ y, int M,
    int N, int K, size_t row_bytes, int tiles_m, int tiles_n, int kt_per_split, int atomic,
    float *__restrict__ part) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave & 1, wn = wave >> 1;

  // XCD-aware tile order (as in gemm.hip)
  const int tiles = tiles_m * tiles_n;
  const int total = tiles * int(gridDim.y);
  int L = blockIdx.x + blockIdx.y * gridDim.x;
  if (total % 8 == 0) L = (L % 8) * (total / 8) + L / 8;
  const int split = L / tiles, tile = L % tiles;
  const int mt = tile % tiles_m, nt = tile / tiles_m;
  const int m0 = mt * kBM, n0 = nt * kBN;
  const int KT = K / (32 * kBlk);
  const int kt0 = split * kt_per_split;
  const int kt1 = min(KT, kt0 + kt_per_split);

  const size_t xrow = size_t(K) / 32 * 34;  // bytes of one activation row
  Geo g;
  g.row = tid >> 1;
  g.half = tid & 1;
  const int mrows = min(kBM, M - m0), nrows = min(kBN, N - n0);
  g.xr = swamp::make_rsrc(xq8 + size_t(m0) * xrow, uint32_t(size_t(mrows) * xrow));
  g.xv = uint32_t(size_t(g.row) * xrow + 68u * uint32_t(g.half));
  g.wr = swamp::make_rsrc(w + size_t(n0) * row_bytes, uint32_t(size_t(nrows) * row_bytes));
  g.wv = uint32_t(size_t(g.row) * row_bytes +
                  (DT == SWAMP_Q4_0 ? 36u : DT == SWAMP_Q8_0 ? 68u : 32u) * uint32_t(g.half) +
                  (DT == SWAMP_Q4_K ? 16u : 0u));

  f32x32_t acc[2];
#pragma unroll
  for (int j = 0; j < 2; j++)
#pragma unroll
    for (int e = 0; e < 32; e++) acc[j][e] = 0.f;

  Stage<DT> st;
  sload<DT>(st, g, kt0);
  lstore<DT>(smem, st, g, kt0);
  __syncthreads();
  for (int kt = kt0; kt < kt1; kt++) {
    const int s = (kt - kt0) & 1;
    const uint8_t *cur = smem + s * stage_bytes<DT>();
    uint8_t *nxt = smem + (s ^ 1) * stage_bytes<DT>();
    const bool more = kt + 1 < kt1;
    // unconditional (the last step reloads itself): after a conditional
    // load the registers would merge old and new values, and the moves that
    // merge them wait on the loads before compute can start
    sload<DT>(st, g, more ? kt + 1 : kt);
    compute<DT>(acc, cur, wm, wn, lane);
    if (more) lstore<DT>(nxt, st, g, kt + 1);
    __syncthreads();
  }

  const int fr = lane & 31, fc = lane >> 5;
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int n = n0 + wn * 64 + j * 32 + fr;
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const int m = m0 + wm * 64 + i * 32 + 8 * (e >> 2) + 4 * fc + (e & 3);
        if (m < M && n < N) {
          float *dst = y + size_t(m) * N + n;
          const float v = acc[j][16 * i + e];
          if (part) part[(size_t(split) * M + m) * N + n] = v;
          else if (atomic) unsafeAtomicAdd(dst, v);
          else *dst = v;
        }
      }
    }
}

__global__ void zero_f32_i8_kernel(float *__restrict__ p, size_t n) {
  const size_t stride = size_t(gridDim.x) * blockDim.x;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = 0.f;
}

template <int DT>
int set_smem_attr_i8() {
  static std::once_flag once;
  static hipError_t err = hipSuccess;
  std::call_once(once, [] {
    err = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemm_i8_kernel<DT>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, smem_bytes<DT>());
  });
  return err == hipSuccess ? SWAMP_OK : SWAMP_ELAUNCH;
}

}  // namespace

namespace {

// K splits of an int8 GEMM call: two workgroups fit per CU (72 KB LDS
// each); when the tiles do not fill them, K is split into up to 8 pieces.
void plan_i8(int m, int n_rows, int n_cols, int &splits, int &kt_per_split) {
  const int tiles = ((m + kBM - 1) / kBM) * ((n_rows + kBN - 1) / kBN);
  const int KT = n_cols / (32 * kBlk);
  const int cus = swamp::device_info().num_cus;
  splits = std::max(1, std::min({2 * cus / std::max(1, tiles), KT / 4, 8}));
  kt_per_split = (KT + splits - 1) / splits;
  splits = (KT + kt_per_split - 1) / kt_per_split;
}

}  // namespace

size_t swamp_gemm_i8_scratch_bytes(uint32_t dtype, int m, int n_rows, int n_cols) {
  if (m <= 0 || n_rows <= 0 || n_cols % (32 * kBlk) != 0) return 0;
  if (dtype != SWAMP_Q4_0 && dtype != SWAMP_Q8_0 && dtype != SWAMP_Q4_K) return 0;
  int splits, kps;
  plan_i8(m, n_rows, n_cols, splits, kps);
  return splits > 1 ? size_t(splits) * size_t(m) * size_t(n_rows) * sizeof(float) : 0;
}

int swamp_launch_gemm_i8(uint32_t dtype, const void *d_w, const void *d_xq8, float *d_y, int m,
                         int n_rows, int n_cols, swamp::Scratch &sc, hipStream_t s) {
  if (m == 0 || n_rows == 0) return SWAMP_OK;
  if (dtype != SWAMP_Q4_0 && dtype != SWAMP_Q8_0 && dtype != SWAMP_Q4_K) return SWAMP_EDTYPE;
  if (n_cols % (32 * kBlk) != 0) return SWAMP_ESHAPE;
  const int tiles_m = (m + kBM - 1) / kBM, tiles_n = (n_rows + kBN - 1) / kBN;
  const int tiles = tiles_m * tiles_n;
  const int cus = swamp::device_info().num_cus;
  int splits, kt_per_split;
  plan_i8(m, n_rows, n_cols, splits, kt_per_split);
  // split pieces go to scratch and are summed in piece order (deterministic);
  // without scratch they add into zeroed y with float atomics
  const size_t n = size_t(m) * n_rows;
  float *part = splits > 1 ? static_cast<float *>(sc.get(size_t(splits) * n * sizeof(float)))
                           : nullptr;
  const int atomic = splits > 1 && !part ? 1 : 0;
  if (atomic)
    zero_f32_i8_kernel<<<unsigned(std::min<size_t>((n + 255) / 256, size_t(cus) * 16)), 256, 0,
                         s>>>(d_y, n);
  const dim3 grid{unsigned(tiles), unsigned(splits), 1u};
  const uint8_t *w = static_cast<const uint8_t *>(d_w);
  const uint8_t *x = static_cast<const uint8_t *>(d_xq8);
  const size_t rb = swamp::row_bytes(int(dtype), size_t(n_cols));
  auto launch = [&](auto dt) -> int {
    constexpr int DT = decltype(dt)::value;
    if (int rc = set_smem_attr_i8<DT>()) return rc;
    gemm_i8_kernel<DT><<<grid, kThreads, smem_bytes<DT>(), s>>>(
        w, x, d_y, m, n_rows, n_cols, rb, tiles_m, tiles_n, kt_per_split, atomic, part);
    return SWAMP_OK;
  };
  int rc = dtype == SWAMP_Q4_0   ? launch(std::integral_constant<int, SWAMP_Q4_0>{})
           : dtype == SWAMP_Q8_0 ? launch(std::integral_constant<int, SWAMP_Q8_0>{})
                                 : launch(std::integral_constant<int, SWAMP_Q4_K>{});
  if (rc) return rc;
  if (hipGetLastError() != hipSuccess) return SWAMP_ELAUNCH;
  if (part) return swamp_launch_split_reduce(part, d_y, splits, n, s);
  return SWAMP_OK;
}
