// gemm_dq.hip -- the prefill GEMM's dequantize-once route, for prompts long
// enough to amortise it: the weight rows are dequantized to bf16 in row
// chunks (dequant.hip, each value the reference's exact fp32 weight rounded
// to nearest even -- the same bf16 values the fused kernel of gemm.hip
// feeds its matrix cores), and each chunk is multiplied by the bf16
// activations with the plain bf16 x bf16 -> fp32 GEMM of gemm_bb.hip into
// its column block of y (leading dimension n_rows).
#include <algorithm>
#include <cstdlib>

#include "swamp_common.hpp"

size_t swamp_gemm_bb_scratch_bytes(int m, int n_rows, int n_cols);
int swamp_launch_gemm_bb(const void *d_w, const void *d_x, float *d_y, int m, int n_rows,
                         int n_cols, int ldy, swamp::Scratch &sc, hipStream_t s);

namespace {

// bf16 bytes of weights per chunk (tuning override: SWAMP_DQ_CHUNK_MB, read
// per call)
size_t chunk_target() {
  const char *e = std::getenv("SWAMP_DQ_CHUNK_MB");
  const long v = e ? std::atol(e) : 0;
  return size_t(v >= 16 && v <= 4096 ? v : 512) << 20;
}

// Rows per chunk: at most about chunk_target() bytes of bf16, in whole
// rounds of 256 x 256 tiles (256 rows times the CUs a 256-token tile row
// leaves per weight column) where the matrix has that many, else whole
// 256-row tiles.  The 8B matrices fit one chunk; the 70B gate+up (940 MB
// of bf16) takes two.
int chunk_rows(int m, int n_rows, int n_cols) {
  const size_t total = size_t(n_rows) * size_t(n_cols) * 2;
  const size_t target = chunk_target();
  if (total <= target) return n_rows;
  const int chunks = int((total + target - 1) / target);
  const int tiles_m = (m + 255) / 256, cus = swamp::device_info().num_cus;
  const int round = 256 * std::max(1, cus / tiles_m);
  int r = (n_rows + chunks - 1) / chunks;
  const int unit = round < n_rows ? round : 256;
  r = (r + unit - 1) / unit * unit;
  return std::min(r, n_rows);
}

int route_forced() {  // tuning override, read per call: SWAMP_GEMM_ROUTE=fused|dq
  const char *e = std::getenv("SWAMP_GEMM_ROUTE");
  if (!e) return 0;
  if (e[0] == 'f') return 1;
  if (e[0] == 'd') return 2;
  return 0;
}

}  // namespace

bool swamp_gemm_dq_route(uint32_t dtype, int m, int n_rows, int n_cols) {
  if (dtype == SWAMP_Q6_K) return true;  // no fused kernel for Q6_K
  if (dtype != SWAMP_Q4_0 && dtype != SWAMP_Q8_0 && dtype != SWAMP_Q4_K) return false;
  if (int f = route_forced()) return f == 2;
  // The fused kernel reads 0.56-1.06 bytes per weight per tile, the plain
  // bf16 GEMM 2 (its loads from L2 bound it, not the dequantization), so the
  // fused kernel is faster wherever its 256 x 256 tiles fill whole rounds of
  // the CUs or split along K.  Between half a round and one round they leave
  // CUs idle, and the plain GEMM's 256-token x 192-row tiles fill them: this
  // route, once every weight meets enough tokens to repay the dequantization.
  // `bench.py --route-crossover` (8B shapes, us, fused / this route, Q4_0):
  // 2048 tokens qkv 113.1 / 109.4, gate_up 514.0 / 599.1, down 253.0 / 324.4,
  // o_proj 76.5 / 84.9; Q8_0 qkv 128.7 / 112.8; Q4_K qkv 116.8 / 111.4.
  if (m < 1024 || n_cols < 1024) return false;
  const int cus = swamp::device_info().num_cus;
  const long tiles = long((m + 255) / 256) * long((n_rows + 255) / 256);
  return 2 * tiles > cus && tiles < cus;
}

size_t swamp_gemm_dq_scratch_bytes(int m, int n_rows, int n_cols) {
  const int cr = chunk_rows(m, n_rows, n_cols);
  const size_t w = (size_t(cr) * size_t(n_cols) * 2 + 255) & ~size_t(255);
  // partial sums of a K split (few tiles), for the larger of the two chunk shapes
  const int last = n_rows - (n_rows - 1) / cr * cr;
  const size_t part = std::max(swamp_gemm_bb_scratch_bytes(m, cr, n_cols),
                               swamp_gemm_bb_scratch_bytes(m, last, n_cols));
  return w + ((part + 255) & ~size_t(255));
}

int swamp_launch_gemm_dq(uint32_t dtype, const void *d_w, const void *d_x, float *d_y, int m,
                         int n_rows, int n_cols, swamp::Scratch &sc, hipStream_t s) {
  const int cr = chunk_rows(m, n_rows, n_cols);
  void *wb = sc.get(size_t(cr) * size_t(n_cols) * 2);
  if (!wb) return kDqUnavailable;
  const size_t rb = swamp::row_bytes(int(dtype), size_t(n_cols));
  for (int r0 = 0; r0 < n_rows; r0 += cr) {
    const int rows = std::min(cr, n_rows - r0);
    const uint8_t *w = static_cast<const uint8_t *>(d_w) + size_t(r0) * rb;
    if (int rc = swamp_launch_dequant_bf16(dtype, w, wb, size_t(rows) * size_t(n_cols), s))
      return rc;
    // the chunk's K-split partial sums (if any) follow the weights; each
    // chunk reuses the same region after the previous chunk's kernels
    swamp::Scratch part = sc;
    if (int rc = swamp_launch_gemm_bb(wb, d_x, d_y + r0, m, rows, n_cols, n_rows, part, s))
      return rc;
  }
  return SWAMP_OK;
}
