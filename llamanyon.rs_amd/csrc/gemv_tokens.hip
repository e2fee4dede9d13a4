// gemv_tokens.hip -- the small batch of 2 tokens as a GEMV: each weight
// item is loaded and turned into fp16 pairs once and multiplied into the x
// of both tokens with V_DOT2_F32_F16.
//
// Replaces, for this token count, forward_linear_batch
// (swamp-engine/src/linear.rs:176-239) and fused_gemv_q4k_batched
// (swamp-kernels/src/fused_gemv_q4k.rs:527-554) written over y.
//
// Why not the matrix cores: at 2 tokens an MFMA tile of 16 tokens is
// mostly empty, and the small-batch kernel pays for its activation staging
// and K-slice sums like a 16-token pass; the decode GEMV's layout streams
// the same bytes faster (one item per lane, whole rows per wave, x staged
// once per workgroup).  Per 8 Q4 weights this costs 1 shift and 4 and-or
// for the weight pairs plus 4 dot2 per token.  (Built for 4 tokens too,
// the 16 dot2 per 8 weights made it slower than the matrix cores on every
// 8B shape; 3 and more tokens stay there.)
//  * x of each token goes through LDS by DMA (one token at a time through
//    one region) into the per-item fragment of the fp16-x GEMV: scaled per
//    64-weight item by a power of two, rounded to fp16 (2^-11 relative),
//    the magic offsets removed with the matching sums of the same x.  The
//    fragments of both tokens stay in registers (2 x 35 VGPRs); the kernel
//    is built for up to 256 VGPRs per wave and launched with one wave per
//    SIMD (two for Q6_K).
//  * Tiles of 1 or 2 rows, one item per lane, 1..8 waves per row (rows of
//    up to 512 items, n_cols <= 32768), row sets sharing x as in the decode
//    GEMV; the next tile's weights are in flight while the current one is
//    multiplied.  Each token's row sums reduce across the wave by DPP and,
//    with several waves per row, through LDS in wave order.
#include "gemv_core.hpp"

namespace {

template <int DT, int NT, int kRows, int kWaves, int kSets>
__global__ void __launch_bounds__(64 * kWaves * kSets, 2)
    gemv_tok_kernel(const uint8_t *__restrict__ w, const float *__restrict__ x,
                    float *__restrict__ y, int n_tok, int n_rows, int ipr, size_t row_bytes,
                    int n_tiles) {
  constexpr int T = 64 * kWaves;
  constexpr int kWgWaves = kWaves * kSets;
  constexpr int kRegion = kWaves * 16384;  // one token's x: up to 64 kWaves items of 256 B
  __shared__ __align__(16) uint8_t xlds[kRegion];
  __shared__ float red[2][kSets][kWaves][NT * kRows];
  const int tid = kSets == 1 ? int(threadIdx.x) : int(threadIdx.x) % T;
  const int set = kSets == 1 ? 0 : __builtin_amdgcn_readfirstlane(int(threadIdx.x) / T);
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6)), lane = tid & 63;
  const int n_cols = ipr * 64;

  int item[1];
  const bool valid = tid < ipr;
  item[0] = valid ? tid : ipr - 1;  // in-bounds stand-in; its x is zero
  uint32_t off[1];
  off[0] = swamp::item_offset<DT>(item[0]);

  // set s of workgroup b takes tiles kSets b + s, + kSets gridDim.x, ...;
  // a set past the last tile takes part in the staging, then leaves
  const int stride = int(gridDim.x) * kSets;
  int tile = int(blockIdx.x) * kSets + set;
  const bool idle = tile >= n_tiles;
  if (idle) tile = n_tiles - 1;
  const uint32_t m = f16_magic();
  auto ref = [&](int tl) { return TileRef{w, nullptr, tl * kRows, n_rows}; };

  // Token 0's x by DMA, then the first tile's weights, then the fragments;
  // the memory counter is in order, so waiting until only the tile's loads
  // are outstanding means this wave's DMA pieces have landed.
  static_assert(NT == 2, "more tokens run on the matrix cores");
  Raw<DT> ra[kRows][1], rb[kRows][1];
  stage_vec<DT, kWgWaves>(xlds, x, ipr, wave, lane);
  TileRef ta = ref(tile);
  issue_tile<DT, 1, kRows>(ra, ta, row_bytes, item, off);
  __builtin_amdgcn_sched_barrier(0);
  constexpr int kAfter = kRows * loads_per_item(DT);
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(kAfter) : "memory");
  XFrag<DT> xf[NT];
  {
    float4 x4[16];
    read_vec(x4, xlds, item[0]);
    build_xfrag<DT>(xf[0], x4, valid);
  }
#pragma unroll
  for (int t = 1; t < NT; t++) {
    // every wave has read the previous token before the region is reused
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (t < n_tok) stage_vec<DT, kWgWaves>(xlds, x + size_t(t) * n_cols, ipr, wave, lane);
    // (this also waits for the first tile's weights, issued before it)
    asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    float4 x4[16];
    read_vec(x4, xlds, item[0]);
    build_xfrag<DT>(xf[t], x4, valid && t < n_tok);
  }
  if (kWaves == 1 && idle) return;  // one-wave sets meet no barrier below

  // The sums of one tile: per token and row, over the lane's item, then
  // across the wave (and the row's waves); stored by the lane that holds
  // each total.
  auto consume = [&](const Raw<DT> (&raw)[kRows][1], const TileRef &t, float *rd, bool live) {
    float acc[NT][kRows];
#pragma unroll
    for (int r = 0; r < kRows; r++)
#pragma unroll
      for (int k = 0; k < NT; k++) acc[k][r] = item_dot<DT>(raw[r][0], xf[k], item[0], m);
#pragma unroll
    for (int k = 0; k < NT; k++) reduce_rows<kRows>(acc[k], lane);
    constexpr int kGroup = 64 / kRows;  // lanes holding one row's total
    const int rr = lane / kGroup;
    if constexpr (kWaves == 1) {
      if (live && lane % kGroup == 0 && t.row0 + rr < n_rows) {
#pragma unroll
        for (int k = 0; k < NT; k++)
          if (k < n_tok) y[size_t(k) * n_rows + t.row0 + rr] = acc[k][0];
      }
    } else {
      const int wv = tid >> 6;
      if (lane % kGroup == 0) {
#pragma unroll
        for (int k = 0; k < NT; k++) rd[wv * NT * kRows + k * kRows + rr] = acc[k][0];
      }
      __syncthreads();
      if (live && tid < NT * kRows) {
        const int k = tid / kRows, r = tid % kRows;
        if (k < n_tok && t.row0 + r < n_rows) {
          float v = 0.f;
#pragma unroll
          for (int q = 0; q < kWaves; q++) v += rd[q * NT * kRows + k * kRows + r];
          y[size_t(k) * n_rows + t.row0 + r] = v;
        }
      }
    }
  };

  // two tiles per trip (static register names); the next tile's loads are
  // issued unconditionally (past the end they re-read the current tile)
  bool live_a = !idle;
  int base = int(blockIdx.x) * kSets;
  for (;;) {
    const int cur = tile;
    int nb = base + stride;
    const bool live_b = nb + set < n_tiles;
    const TileRef tb = ref(live_b ? nb + set : cur);
    issue_tile<DT, 1, kRows>(rb, tb, row_bytes, item, off);
    __builtin_amdgcn_sched_barrier(0);
    consume(ra, ta, &red[0][set][0][0], live_a);
    if (kWaves > 1 ? nb >= n_tiles : !live_b) break;
    base = __builtin_amdgcn_readfirstlane(nb);
    tile = live_b ? base + set : cur;
    nb = base + stride;
    live_a = nb + set < n_tiles;
    ta = ref(live_a ? nb + set : tile);
    issue_tile<DT, 1, kRows>(ra, ta, row_bytes, item, off);
    __builtin_amdgcn_sched_barrier(0);
    consume(rb, tb, &red[1][set][0][0], live_b);
    if (kWaves > 1 ? nb >= n_tiles : !live_a) break;
    base = __builtin_amdgcn_readfirstlane(nb);
    tile = live_a ? base + set : tile;
  }
}

template <int DT, int NT, int kRows, int kWaves, int kSets>
int launch_tok(const void *d_w, const float *d_x, float *d_y, int n_tok, int n_rows, int n_cols,
               hipStream_t s) {
  const int ipr = n_cols / 64;
  const int n_tiles = (n_rows + kRows - 1) / kRows;
  const int cus = swamp::device_info().num_cus;
  // Waves per CU: 4 (one per SIMD) for Q4_0 / Q4_K / Q8_0: on the 8B shapes
  // at 2 tokens (Q4_K layer, Q8_0 lm_head) 137.2 us against 142.7 with 8
  // per CU (lm_head 93.1 against 97.7, qkv 6.6 against 7.5, o_proj 5.6
  // against 6.7; gate_up alone is slower, 19.1 against 17.7).  8 for Q6_K,
  // whose heavier decode needs a second wave per SIMD (its 8B lm_head:
  // 114 us on 4 waves per CU against 88 on 8).
  constexpr int kWavesPerCu = DT == SWAMP_Q6_K ? 8 : 4;
  int grid = cus * std::max(1, kWavesPerCu / (kWaves * kSets));
  const int need = (n_tiles + kSets - 1) / kSets;
  if (grid > need) grid = need;
  gemv_tok_kernel<DT, NT, kRows, kWaves, kSets><<<grid, 64 * kWaves * kSets, 0, s>>>(
      static_cast<const uint8_t *>(d_w), d_x, d_y, n_tok, n_rows, ipr,
      swamp::row_bytes(DT, n_cols), n_tiles);
  return hipGetLastError() == hipSuccess ? SWAMP_OK : SWAMP_ELAUNCH;
}

// Waves per row and row sets per workgroup by row length (as the decode
// GEMV: 4 one-wave sets up to 64 items, 2 two-wave sets up to 128).
template <int DT, int NT, int kRows>
int launch_tok_rows(const void *d_w, const float *d_x, float *d_y, int n_tok, int n_rows,
                    int n_cols, hipStream_t s) {
  const int ipr = n_cols / 64;
  if (ipr <= 64) return launch_tok<DT, NT, kRows, 1, 4>(d_w, d_x, d_y, n_tok, n_rows, n_cols, s);
  if (ipr <= 128) return launch_tok<DT, NT, kRows, 2, 2>(d_w, d_x, d_y, n_tok, n_rows, n_cols, s);
  if (ipr <= 256) return launch_tok<DT, NT, kRows, 4, 1>(d_w, d_x, d_y, n_tok, n_rows, n_cols, s);
  return launch_tok<DT, NT, kRows, 8, 1>(d_w, d_x, d_y, n_tok, n_rows, n_cols, s);
}

// Rows per tile: 2 when every row set of the grid gets at least two 2-row
// tiles (counted at 8 waves per CU); Q6_K only from 16384 rows, else 1.
template <int DT, int NT>
int launch_tok_dt(const void *d_w, const float *d_x, float *d_y, int n_tok, int n_rows,
                  int n_cols, hipStream_t s) {
  const int cus = swamp::device_info().num_cus;
  const long slots = long(cus) * std::max(1, 8 / waves_for(n_cols / 64));
  // Q6_K from 16384 rows only (8B gate_up and lm_head faster with 2-row
  // tiles, the shorter qkv, o_proj and down slower)
  if (DT != SWAMP_Q6_K || n_rows >= 16384) {
    if (long(n_rows) / 2 >= slots)
      return launch_tok_rows<DT, NT, 2>(d_w, d_x, d_y, n_tok, n_rows, n_cols, s);
  }
  return launch_tok_rows<DT, NT, 1>(d_w, d_x, d_y, n_tok, n_rows, n_cols, s);
}

template <int NT>
int launch_tok_nt(uint32_t dt, const void *d_w, const float *d_x, float *d_y, int n_tok,
                  int n_rows, int n_cols, hipStream_t s) {
  switch (dt) {
  case SWAMP_Q4_0: return launch_tok_dt<SWAMP_Q4_0, NT>(d_w, d_x, d_y, n_tok, n_rows, n_cols, s);
  case SWAMP_Q8_0: return launch_tok_dt<SWAMP_Q8_0, NT>(d_w, d_x, d_y, n_tok, n_rows, n_cols, s);
  case SWAMP_Q4_K: return launch_tok_dt<SWAMP_Q4_K, NT>(d_w, d_x, d_y, n_tok, n_rows, n_cols, s);
  case SWAMP_Q6_K: return launch_tok_dt<SWAMP_Q6_K, NT>(d_w, d_x, d_y, n_tok, n_rows, n_cols, s);
  default: return SWAMP_EDTYPE;
  }
}

}  // namespace

bool swamp_gemv_tokens_ok(uint32_t dtype, int n_tok, int n_cols) {
  return n_tok == 2 && n_cols > 0 && n_cols / 64 <= 512 && item_path_ok(dtype, n_cols);
}

int swamp_launch_gemv_tokens(uint32_t dtype, const void *d_w, const float *d_x, float *d_y,
                             int n_tok, int n_rows, int n_cols, hipStream_t s) {
  if (!swamp_gemv_tokens_ok(dtype, n_tok, n_cols)) return SWAMP_ESHAPE;
  if (n_rows == 0) return SWAMP_OK;
  return launch_tok_nt<2>(dtype, d_w, d_x, d_y, n_tok, n_rows, n_cols, s);
}
