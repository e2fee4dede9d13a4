// gemm_bb.hip -- plain bf16 x bf16 -> fp32 GEMM on the matrix cores, the
// second half of the prefill GEMM's dequantize-once route (gemm_dq.hip):
// y[m][n] = sum_k W[n][k] x[m][k], with W the weight rows already
// dequantized to bf16 (row-major [n][K]) and x the bf16 activations
// (row-major [m][K]); y row-major with leading dimension ldy.
//
// Design (MFMA-bound; 2*M*N*K flops over 2 B per weight and activation):
//  * Four waves per workgroup, one per SIMD, each owning a WM*32 token x
//    WN*32 row block of the tile (2 x 2 waves): WM x WN
//    V_MFMA_F32_32X32X16_BF16 accumulators (256 fp32 per lane for the full
//    4 x 4 block, held in the accumulator registers).  A wave block of
//    128 x 128 reads 16 KB of fragments per 64 MFMAs from LDS: 64 bytes of
//    LDS per MFMA cycle for the workgroup.
//  * K step 32: a stage holds the tile's activation rows then its weight
//    rows, 64 bytes each, 16-byte chunks XOR-swizzled by (row / 4) % 4 (no
//    bank conflicts for any 16 consecutive lanes of a fragment read).
//    Stages are filled by direct-to-LDS DMA (buffer_load ... lds, 1 KB per
//    wave instruction, no VGPRs), four K steps ahead through five stages.
//  * One barrier per K step, between its two substeps: the wait before it
//    leaves the last three steps' DMAs in flight (the memory counter is in
//    order); after it the step's DMA is issued and the next step's first
//    fragments are read, so no fragment read waits on a barrier.
//  * Tile order: groups of G token tiles, consecutive tiles walking the
//    token tiles of a group first, then the weight columns; workgroup ids
//    are remapped so each XCD (hardware ids i, i + 8, ...) runs a
//    contiguous run of that order, and a round of its CUs shares few
//    weight columns and activation slabs in its L2.
//  * Work decomposition (host): full 256 x 256 tiles in complete rounds, a
//    last round at most half full as 128-token half tiles; fewer tiles than
//    the CUs: narrower weight tiles (192 or 128 rows) when they fill the
//    CUs better, else K split into pieces summed in piece order.
#include "swamp_common.hpp"
#include "swamp_items.hpp"

#include <algorithm>
#include <mutex>
#include <type_traits>

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kBK = 32;          // K per step (64-byte stage rows)

// A workgroup of NWM x NWN waves, each owning WM x WN 32 x 32 blocks
// (tokens x weight rows).
template <int WM, int WN, int NWM, int NWN>
struct Shape {
  static constexpr int NW = NWM * NWN, kThreads = 64 * NW;
  static constexpr int TM = 32 * WM * NWM, TN = 32 * WN * NWN;  // tile (tokens, rows)
  static constexpr int kStage = (TM + TN) * 64;     // bytes of one stage
  static constexpr int kStages = 5;
  static constexpr int kSmem = kStages * kStage;
  static constexpr int kDma = (TM + TN) / (16 * NW);  // 1 KB DMAs per wave and step
  static constexpr int kDma0 = (kDma + 1) / 2;      // of them in a step's first substep
  static_assert(kStages == 5, "the DMA of step kt + 3 fills the stage of step kt - 2");
  static_assert(TM % (16 * NW) == 0 && TN % (16 * NW) == 0, "a DMA fills 16 rows of one operand");
  static_assert(kSmem <= 160 * 1024, "LDS");
};

// One 16-byte-per-lane DMA into LDS (lane L writes lds + 16 L).  Not a
// template: the host pass rejects the LDS address-space cast inside a
// template instantiation.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint8_t *lds, uint32_t voff,
                                      uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds, 16,
                                           voff, soff, 0, 0);
}

struct BbWork {
  int tiles_m, tiles_n;  // tile grid of the launch's shape
  int first;             // first tile of the launch in the grouped order
  int group;             // token tiles per order group
  int parts;             // token parts per tile (2: the launch runs half tiles)
  int splits, kt_per_split;
  int ldy;
  float *part;           // splits > 1: partial sums [piece][M][ldy]
};

// Tile t of the grouped order -> (token tile, weight tile).
__device__ __forceinline__ void bb_tile(int t, int tiles_m, int tiles_n, int g, int &mt,
                                        int &nt) {
  const int grp = t / (g * tiles_n), first = grp * g;
  const int gs = min(tiles_m - first, g), r = t - grp * g * tiles_n;
  mt = first + r % gs;
  nt = r / gs;
}

template <int WM, int WN, int NWM, int NWN>
__global__ void __launch_bounds__(64 * NWM * NWN, 1)
    gemm_bb_kernel(const uint16_t *w, const uint16_t *x, float *y, int M, int N, int K,
                   BbWork wk) {
  // w and x carry no __restrict__: the hand-counted waits assume every load
  // is issued where the code places it.
  using S = Shape<WM, WN, NWM, NWN>;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  // XCD-aware unit order: hardware ids i, i + 8, ... run on XCD i % 8;
  // each XCD takes a contiguous run of units.
  const int n_units = int(gridDim.x), b = int(blockIdx.x);
  const int q = n_units / 8, rem = n_units % 8, xcd = b % 8;
  const int u = xcd * q + min(xcd, rem) + b / 8;
  const int per_tile = wk.parts * wk.splits;
  const int t = wk.first + u / per_tile, part = (u % per_tile) / wk.splits;
  const int piece = u % wk.splits;
  int mt, nt;
  bb_tile(t, wk.tiles_m, wk.tiles_n, wk.group, mt, nt);
  // a half tile is the first or second TM tokens of a 2 TM token tile
  const int m0 = mt * S::TM * wk.parts + part * S::TM, n0 = nt * S::TN;
  if (m0 >= M) return;  // second half of a short last token tile (uniform)
  const int KT = K / kBK;
  const int kt0 = piece * wk.kt_per_split, kt1 = min(KT, kt0 + wk.kt_per_split);

  const uint32_t pitch = uint32_t(K) * 2;
  const __amdgpu_buffer_rsrc_t xr =
      swamp::make_rsrc(x + size_t(m0) * K, uint32_t(min(S::TM, M - m0)) * pitch);
  const __amdgpu_buffer_rsrc_t wr =
      swamp::make_rsrc(w + size_t(n0) * K, uint32_t(min(S::TN, N - n0)) * pitch);
  // DMA instruction i of wave w fills stage rows R = 16 (NW i + w) .. R + 15:
  // lane L writes row R + L/4, physical chunk L%4, which holds logical
  // chunk (L%4) ^ ((R + L/4) / 4 % 4) = (L%4) ^ (L/16 % 4).
  const uint32_t vdma = uint32_t(lane >> 2) * pitch + uint32_t(((lane & 3) ^ ((lane >> 4) & 3)) << 4);

  // DMAs [i0, i1) of one step's stage
  auto dma_part = [&](uint8_t *st, int kt, auto i0c, auto i1c) {
    constexpr int i0 = decltype(i0c)::value, i1 = decltype(i1c)::value;
#pragma unroll
    for (int i = i0; i < i1; i++) {
      const int R = 16 * (S::NW * i + wave);
      if (16 * S::NW * i < S::TM)
        dma16(xr, st + R * 64, vdma, uint32_t(R) * pitch + uint32_t(kt) * 64u);
      else
        dma16(wr, st + R * 64, vdma, uint32_t(R - S::TM) * pitch + uint32_t(kt) * 64u);
    }
  };
  using I0 = std::integral_constant<int, 0>;
  using IH = std::integral_constant<int, S::kDma0>;
  using IE = std::integral_constant<int, S::kDma>;

  // Fragment of substep s (k = 16 s .. 16 s + 15 of the step): lane l reads
  // row l%32 of its 32-row block, logical chunk 2 s + l/32.
  const int wm = wave % NWM, wn = wave / NWM;
  const uint32_t lrow = uint32_t(lane & 31) * 64;
  const uint32_t sw = uint32_t((lane >> 2) & 3);
  const uint32_t loff0 = lrow + (((uint32_t(lane >> 5)) ^ sw) << 4);
  const uint32_t loff1 = lrow + (((2u + uint32_t(lane >> 5)) ^ sw) << 4);
  const uint32_t a_off = uint32_t(wm * WM * 32) * 64, b_off = uint32_t(S::TM + wn * WN * 32) * 64;

  auto read_frags = [&](const uint8_t *st, uint32_t loff, bf16x8_t (&fa)[WM], bf16x8_t (&fb)[WN]) {
#pragma unroll
    for (int i = 0; i < WM; i++)
      fa[i] = *reinterpret_cast<const bf16x8_t *>(st + a_off + 2048 * i + loff);
#pragma unroll
    for (int j = 0; j < WN; j++)
      fb[j] = *reinterpret_cast<const bf16x8_t *>(st + b_off + 2048 * j + loff);
  };

  f32x16_t acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; i++)
#pragma unroll
    for (int j = 0; j < WN; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;

  auto mfmas = [&](const bf16x8_t (&fa)[WM], const bf16x8_t (&fb)[WN]) {
#pragma unroll
    for (int i = 0; i < WM; i++)
#pragma unroll
      for (int j = 0; j < WN; j++)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
  };

  constexpr int NS = S::kStages;
  // Stage p is smem + kStage p; indices, not pointers, so that every access
  // keeps the LDS address space (a selected generic pointer becomes a flat
  // access, which the memory counter also tracks).  Step kt issues the DMA
  // of step kt + 3, half in each substep, into the stage of step kt - 2,
  // which every wave finished reading before the previous barrier.
  // Prologue: steps kt0 .. kt0 + 2 (past the end: the last step again).
#pragma unroll
  for (int p = 0; p < 3; p++) {
    dma_part(smem + S::kStage * p, min(kt0 + p, kt1 - 1), I0{}, IE{});
    __builtin_amdgcn_sched_barrier(0);
  }
  // step kt0 complete (the two steps issued after it stay in flight)
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(2 * S::kDma) : "memory");

  bf16x8_t fa0[WM], fb0[WN], fa1[WM], fb1[WN];
  read_frags(smem, loff0, fa0, fb0);

  // One substep's instruction order: its WM * WN MFMAs, one fragment read
  // after each of the first WM + WN, its DMAs spread over the rest.
  auto order = [&](auto ndc) {
    constexpr int n_dma = decltype(ndc)::value, R = WM * WN - (WM + WN);
#pragma unroll
    for (int m = 0; m < WM * WN; m++) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
      if (m < WM + WN) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // 1 DS read
      } else if (R > 0) {
        const int r = m - (WM + WN), nd = (r + 1) * n_dma / R - r * n_dma / R;
#pragma unroll
        for (int q = 0; q < nd; q++) __builtin_amdgcn_sched_group_barrier(0x010, 1, 0);  // DMA
      }
    }
  };
  using D0 = std::integral_constant<int, S::kDma0>;
  using D1 = std::integral_constant<int, S::kDma - S::kDma0>;

  int cur = 0;  // stage of step kt
  for (int kt = kt0; kt < kt1; kt++) {
    const int nxt = cur + 1 == NS ? 0 : cur + 1;
    const int fill = cur + 3 < NS ? cur + 3 : cur + 3 - NS;  // stage of step kt + 3
    const int ktf = min(kt + 3, kt1 - 1);
    // substep 0: MFMAs on fa0/fb0; substep 1's fragments; half the DMA
    read_frags(smem + S::kStage * cur, loff1, fa1, fb1);
    mfmas(fa0, fb0);
    dma_part(smem + S::kStage * fill, ktf, I0{}, IH{});
    order(D0{});
    __builtin_amdgcn_sched_barrier(0);
    // step kt + 1 complete for every wave: after it, only step kt + 2's DMA
    // and the first half of step kt + 3's stay in flight
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(S::kDma + S::kDma0) : "memory");
    // substep 1: MFMAs on fa1/fb1; the next step's first fragments; the
    // rest of the DMA
    read_frags(smem + S::kStage * nxt, loff0, fa0, fb0);
    mfmas(fa1, fb1);
    dma_part(smem + S::kStage * fill, ktf, IH{}, IE{});
    order(D1{});
    __builtin_amdgcn_sched_barrier(0);
    cur = nxt;
  }

  // C layout of a 32 x 32 block: lane holds column (weight row) lane % 32,
  // rows (tokens) 8 (e / 4) + 4 (lane / 32) + e % 4 for e = 0..15.
  const int fr = lane & 31, fc = lane >> 5;
  float *dst = wk.splits > 1 ? wk.part + size_t(piece) * size_t(M) * size_t(wk.ldy) : y;
#pragma unroll
  for (int j = 0; j < WN; j++) {
    const int n = n0 + wn * WN * 32 + 32 * j + fr;
    if (n >= N) continue;
#pragma unroll
    for (int i = 0; i < WM; i++)
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const int m = m0 + wm * WM * 32 + 32 * i + 8 * (e >> 2) + 4 * fc + (e & 3);
        if (m < M) dst[size_t(m) * size_t(wk.ldy) + n] = acc[i][j][e];
      }
  }
}

// y[m][n] = sum of the pieces' partials [piece][M][N], in piece order
// (deterministic).
__global__ void bb_reduce_kernel(const float *__restrict__ part, float *__restrict__ y, int pieces,
                                 int M, int N, int ldy) {
  const size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const size_t mn = size_t(M) * size_t(N);
  if (i >= mn) return;
  float v[8];
#pragma unroll
  for (int p = 0; p < 8; p++) v[p] = p < pieces ? part[size_t(p) * mn + i] : 0.f;
  float s = v[0];
#pragma unroll
  for (int p = 1; p < 8; p++) s += v[p];  // missing pieces add 0
  y[(i / size_t(N)) * size_t(ldy) + i % size_t(N)] = s;
}

template <int WM, int WN, int NWM, int NWN>
int launch_bb(const uint16_t *w, const uint16_t *x, float *y, int m, int n, int k,
              const BbWork &wk, int units, hipStream_t s) {
  using S = Shape<WM, WN, NWM, NWN>;
  static std::once_flag once;
  static hipError_t err = hipSuccess;
  std::call_once(once, [] {
    err = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemm_bb_kernel<WM, WN, NWM, NWN>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, S::kSmem);
  });
  if (err != hipSuccess) return SWAMP_ELAUNCH;
  if (units <= 0) return SWAMP_OK;
  gemm_bb_kernel<WM, WN, NWM, NWN>
      <<<unsigned(units), S::kThreads, S::kSmem, s>>>(w, x, y, m, n, k, wk);
  return hipGetLastError() == hipSuccess ? SWAMP_OK : SWAMP_ELAUNCH;
}

#ifndef BB_FULL
#define BB_FULL 4, 4, 2, 2
#endif
#ifndef BB_HALF
#define BB_HALF 2, 4, 2, 2
#endif

}  // namespace

// The decomposition of one call (host side; same plan for the scratch size
// and the launches).
struct BbPlan {
  int wn = 4;          // weight tile 64 * wn rows (4, 3 or 2)
  int n_full = 0;      // full tiles (first in the order)
  int n_half = 0;      // tiles run as two 128-token halves (the last round)
  int pieces = 1, kps = 0;
  size_t part_bytes = 0;
};

static BbPlan plan_bb(int m, int n_rows, int n_cols) {
  const int cus = swamp::device_info().num_cus;
  const int KT = n_cols / kBK;
  const int tiles_m = (m + 255) / 256;
  BbPlan p;
  p.kps = KT;
  auto tiles_for = [&](int wn) { return tiles_m * ((n_rows + 64 * wn - 1) / (64 * wn)); };
  const int full = tiles_for(4);
  if (full >= cus) {
    const int r = full % cus;
    p.n_half = r > 0 && 2 * r <= cus ? r : 0;
    p.n_full = full - p.n_half;
    return p;
  }
  // Fewer tiles than CUs: the weight tile width (4, 3 or 2 blocks of 64
  // rows) with the least time in rounds of tiles, each tile's time taken
  // as proportional to its rows (a narrower tile moves more LDS bytes per
  // MFMA: counted as 10% slower per row at 128 rows).
  double best = 0;
  for (int wn = 4; wn >= 2; wn--) {
    const int t = tiles_for(wn);
    const double rounds = double((t + cus - 1) / cus);
    const double cost = rounds * wn * (wn == 2 ? 1.1 : 1.0);
    if (wn == 4 || cost < best) {
      best = cost;
      p.wn = wn;
    }
  }
  const int t = tiles_for(p.wn);
  p.n_full = t;
  // still at most half the CUs: split K into pieces (partial sums in
  // scratch, summed in piece order)
  if (2 * t <= cus) {
    const int pieces = std::max(1, std::min({cus / t, 8, KT / 16}));
    p.kps = (KT + pieces - 1) / pieces;
    p.pieces = (KT + p.kps - 1) / p.kps;
    if (p.pieces > 1) p.part_bytes = size_t(p.pieces) * size_t(m) * size_t(n_rows) * 4;
  }
  return p;
}

size_t swamp_gemm_bb_scratch_bytes(int m, int n_rows, int n_cols) {
  if (m <= 0 || n_rows <= 0 || n_cols <= 0 || n_cols % kBK) return 0;
  return plan_bb(m, n_rows, n_cols).part_bytes;
}

int swamp_launch_gemm_bb(const void *d_w, const void *d_x, float *d_y, int m, int n_rows,
                         int n_cols, int ldy, swamp::Scratch &sc, hipStream_t s) {
  if (m <= 0 || n_rows <= 0) return SWAMP_OK;
  if (n_cols % kBK) return SWAMP_ESHAPE;
  const uint16_t *w = static_cast<const uint16_t *>(d_w);
  const uint16_t *x = static_cast<const uint16_t *>(d_x);
  const BbPlan p = plan_bb(m, n_rows, n_cols);
  float *part = nullptr;
  if (p.part_bytes) {
    part = static_cast<float *>(sc.get(p.part_bytes));
    if (!part) return SWAMP_EWORKSPACE;
  }
  const int tiles_m = (m + 255) / 256;
  const int group = 8;
  if (p.wn != 4 || p.pieces > 1) {
    const int tiles_n = (n_rows + 64 * p.wn - 1) / (64 * p.wn);
    const BbWork wk{tiles_m, tiles_n, 0, group, 1, p.pieces, p.kps, p.pieces > 1 ? n_rows : ldy,
                    part};
    const int units = p.n_full * p.pieces;
    int rc = SWAMP_EINVAL;
    switch (p.wn) {
      case 4: rc = launch_bb<BB_FULL>(w, x, d_y, m, n_rows, n_cols, wk, units, s); break;
      case 3: rc = launch_bb<4, 3, 2, 2>(w, x, d_y, m, n_rows, n_cols, wk, units, s); break;
      case 2: rc = launch_bb<4, 2, 2, 2>(w, x, d_y, m, n_rows, n_cols, wk, units, s); break;
    }
    if (rc || p.pieces == 1) return rc;
    const size_t total = size_t(m) * size_t(n_rows);
    bb_reduce_kernel<<<unsigned((total + 255) / 256), 256, 0, s>>>(part, d_y, p.pieces, m, n_rows,
                                                                   ldy);
    return hipGetLastError() == hipSuccess ? SWAMP_OK : SWAMP_ELAUNCH;
  }
  const int tiles_n = (n_rows + 255) / 256;
  {
    const BbWork wk{tiles_m, tiles_n, 0, group, 1, 1, p.kps, ldy, nullptr};
    if (int rc = launch_bb<BB_FULL>(w, x, d_y, m, n_rows, n_cols, wk, p.n_full, s)) return rc;
  }
  if (p.n_half) {
    const BbWork wk{tiles_m, tiles_n, p.n_full, group, 2, 1, p.kps, ldy, nullptr};
    if (int rc = launch_bb<BB_HALF>(w, x, d_y, m, n_rows, n_cols, wk, 2 * p.n_half, s)) return rc;
  }
  return SWAMP_OK;
}
