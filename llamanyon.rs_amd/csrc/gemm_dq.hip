// gemm_dq.hip -- the prefill GEMM's dequantize-once route, for prompts long
// enough to amortise it: the weight rows are dequantized to bf16 in row
// chunks (dequant.hip, each value the reference's exact fp32 weight rounded
// to nearest even -- the same bf16 values the fused kernel of gemm.hip
// feeds its matrix cores), and each chunk is multiplied by the bf16
// activations with hipBLASLt (a plain bf16 x bf16 -> fp32 GEMM, fp32
// accumulation) into its column block of y.
//
// Layout for the library (column-major): y row-major [m][n_rows] is the
// column-major n_rows x m matrix D with ld n_rows; a chunk of weight rows
// [r0, r1) is the column-major K x (r1 - r0) matrix A with ld K, used
// transposed; x row-major [m][K] is the column-major K x m matrix B with ld
// K.  D[r0:r1, :] = A^T B, written at y + r0 with ld n_rows.
#include <hipblaslt/hipblaslt.h>

#include <algorithm>
#include <cstdlib>
#include <map>
#include <mutex>
#include <tuple>
#include <vector>

#include "swamp_common.hpp"

namespace {

// bf16 bytes of weights per chunk (tuning override: SWAMP_DQ_CHUNK_MB)
size_t chunk_target() {
  static const size_t t = [] {
    const char *e = std::getenv("SWAMP_DQ_CHUNK_MB");
    const long v = e ? std::atol(e) : 0;
    return size_t(v >= 16 && v <= 4096 ? v : 128) << 20;
  }();
  return t;
}
constexpr size_t kLtWorkspace = size_t(32) << 20;   // hipBLASLt workspace offered
constexpr int kLtCandidates = 16;                    // heuristic candidates measured per shape

struct LtAlgo {
  hipblasLtMatmulAlgo_t algo{};
  size_t ws = 0;
};

struct LtPlan {
  hipblasLtMatmulDesc_t op = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, d = nullptr;
  std::vector<LtAlgo> cands;  // the heuristic's candidates, best guess first
  LtAlgo use;                 // the one the launches run
  bool tuned = false;         // `use` was chosen by measurement
  bool ok = false;
};

struct LtState {
  std::mutex mu;
  hipblasLtHandle_t handle = nullptr;
  bool init = false, ok = false;
  std::map<std::tuple<int, int, int, int>, LtPlan> plans;  // (m, rows, K, ld)
};

LtState &lt_state(int dev) {
  static LtState st[64];
  return st[dev & 63];
}

// Rows per chunk: whole 256-row tiles, at most about chunk_target() bytes of
// bf16.  (Chunks dequantized on a second stream beside the previous chunk's
// GEMM measured slower: two smaller GEMMs lose more than the overlap wins.)
int chunk_rows(int n_rows, int n_cols) {
  const size_t total = size_t(n_rows) * size_t(n_cols) * 2;
  const int chunks = int(std::max<size_t>(1, (total + chunk_target() - 1) / chunk_target()));
  int r = (n_rows + chunks - 1) / chunks;
  r = (r + 255) / 256 * 256;
  return std::min(r, n_rows);
}


// The matmul plan for one chunk shape (created once, kept for the process).
LtPlan *lt_plan(int dev, int m, int rows, int k, int ld) {
  LtState &st = lt_state(dev);
  std::lock_guard<std::mutex> lock(st.mu);
  if (!st.init) {
    st.init = true;
    st.ok = hipblasLtCreate(&st.handle) == HIPBLAS_STATUS_SUCCESS;
  }
  if (!st.ok) return nullptr;
  auto key = std::make_tuple(m, rows, k, ld);
  auto it = st.plans.find(key);
  if (it != st.plans.end()) return it->second.ok ? &it->second : nullptr;
  LtPlan &p = st.plans[key];
  bool ok = hipblasLtMatmulDescCreate(&p.op, HIPBLAS_COMPUTE_32F, HIP_R_32F) ==
            HIPBLAS_STATUS_SUCCESS;
  const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
  ok = ok && hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSA, &ta,
                                             sizeof(ta)) == HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSB, &tb,
                                             sizeof(tb)) == HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatrixLayoutCreate(&p.a, HIP_R_16BF, uint64_t(k), uint64_t(rows),
                                         int64_t(k)) == HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatrixLayoutCreate(&p.b, HIP_R_16BF, uint64_t(k), uint64_t(m),
                                         int64_t(k)) == HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatrixLayoutCreate(&p.d, HIP_R_32F, uint64_t(rows), uint64_t(m),
                                         int64_t(ld)) == HIPBLAS_STATUS_SUCCESS;
  if (ok) {
    hipblasLtMatmulPreference_t pref = nullptr;
    ok = hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS;
    const uint64_t cap = kLtWorkspace;
    ok = ok && hipblasLtMatmulPreferenceSetAttribute(
                   pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &cap, sizeof(cap)) ==
                   HIPBLAS_STATUS_SUCCESS;
    hipblasLtMatmulHeuristicResult_t res[kLtCandidates];
    int n = 0;
    ok = ok && hipblasLtMatmulAlgoGetHeuristic(st.handle, p.op, p.a, p.b, p.d, p.d, pref,
                                               kLtCandidates, res, &n) == HIPBLAS_STATUS_SUCCESS;
    for (int i = 0; ok && i < n; i++)
      if (res[i].state == HIPBLAS_STATUS_SUCCESS && res[i].workspaceSize <= cap)
        p.cands.push_back({res[i].algo, res[i].workspaceSize});
    ok = ok && !p.cands.empty();
    if (ok) p.use = p.cands[0];
    if (pref) hipblasLtMatmulPreferenceDestroy(pref);
  }
  p.ok = ok;
  return ok ? &p : nullptr;
}

// The heuristic's first candidate is not always the fastest: for 2048 x
// 4096 x 14336 (the 8B down projection) it measured 256 us against 183 us
// for the second.  So the first launch of a shape on a device times each
// candidate on the caller's stream (one warm-up and three timed launches
// each, with the call's own buffers; this blocks the host once) and keeps
// the fastest; a candidate within 3% of the heuristic's earlier choice
// does not displace it, so the choice is stable from run to run.  Not
// under graph capture (the plan then keeps the heuristic's first candidate
// and is measured at the next eager call), and not with
// SWAMP_GEMM_TUNE=0.
bool tune_enabled() {
  static const bool v = [] {
    const char *e = std::getenv("SWAMP_GEMM_TUNE");
    return !(e && e[0] == '0');
  }();
  return v;
}

void lt_tune(int dev, LtPlan &p, const void *wb, const void *x, float *y, void *ws,
             hipStream_t s) {
  if (p.tuned || !tune_enabled()) return;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return;
  p.tuned = true;
  if (p.cands.size() < 2) return;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) {
    if (e0) (void)hipEventDestroy(e0);
    return;
  }
  const float alpha = 1.0f, beta = 0.0f;
  hipblasLtHandle_t h = lt_state(dev).handle;
  float best = 0.f;
  size_t best_i = 0;
  for (size_t i = 0; i < p.cands.size(); i++) {
    const LtAlgo &c = p.cands[i];
    bool ok = true;
    for (int r = 0; r < 4 && ok; r++) {
      if (r == 1) ok = hipEventRecord(e0, s) == hipSuccess;
      ok = ok && hipblasLtMatmul(h, p.op, &alpha, wb, p.a, x, p.b, &beta, y, p.d, y, p.d,
                                 &c.algo, ws, c.ws, s) == HIPBLAS_STATUS_SUCCESS;
    }
    float ms = 0.f;
    ok = ok && hipEventRecord(e1, s) == hipSuccess && hipEventSynchronize(e1) == hipSuccess &&
         hipEventElapsedTime(&ms, e0, e1) == hipSuccess;
    if (!ok) {
      (void)hipGetLastError();
      (void)hipStreamSynchronize(s);
      continue;
    }
    if (best == 0.f || ms < 0.97f * best) {
      best = ms;
      best_i = i;
    }
  }
  if (best > 0.f) p.use = p.cands[best_i];
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
}

int route_forced() {  // tuning override: SWAMP_GEMM_ROUTE=fused|dq
  static const int v = [] {
    const char *e = std::getenv("SWAMP_GEMM_ROUTE");
    if (!e) return 0;
    if (e[0] == 'f') return 1;
    if (e[0] == 'd') return 2;
    return 0;
  }();
  return v;
}

}  // namespace

bool swamp_gemm_dq_route(uint32_t dtype, int m, int n_rows, int n_cols) {
  if (dtype == SWAMP_Q6_K) return true;  // no fused kernel for Q6_K
  if (dtype != SWAMP_Q4_0 && dtype != SWAMP_Q8_0 && dtype != SWAMP_Q4_K) return false;
  if (route_forced()) return route_forced() == 2;
  // The dequant pass costs about 2.6 bytes of HBM traffic per weight (read
  // the blocks, write bf16): it pays once every weight meets enough tokens.
  // `bench.py --route-crossover` (8B Q4_0 shapes, us, fused / this route):
  // 512 tokens gate_up 141.6 / 178.8, down 91.2 / 112.0, qkv 55.9 / 50.8,
  // o_proj 39.3 / 40.6; 1024 tokens gate_up 281.3 / 259.1, down 156.3 /
  // 152.9, qkv 70.3 / 66.5, o_proj 57.1 / 51.8; 2048 tokens gate_up 501.2 /
  // 454.0, down 282.7 / 234.2.
  return m >= 1024 && n_rows >= 1024 && n_cols >= 1024;
}

size_t swamp_gemm_dq_scratch_bytes(int n_rows, int n_cols) {
  const size_t w = size_t(chunk_rows(n_rows, n_cols)) * size_t(n_cols) * 2;
  return ((w + 255) & ~size_t(255)) + kLtWorkspace;
}

int swamp_launch_gemm_dq(uint32_t dtype, const void *d_w, const void *d_x, float *d_y, int m,
                         int n_rows, int n_cols, swamp::Scratch &sc, hipStream_t s) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return SWAMP_ENODEVICE;
  const int cr = chunk_rows(n_rows, n_cols);
  // every chunk's plan (at most two shapes) before anything is launched: a
  // shape the library has no algorithm for leaves the call to the fused
  // kernel
  const int last = n_rows - (n_rows - 1) / cr * cr;
  LtPlan *p_full = lt_plan(dev, m, cr, n_cols, n_rows);
  LtPlan *p_last = last == cr ? p_full : lt_plan(dev, m, last, n_cols, n_rows);
  if (!p_full || !p_last) return kDqUnavailable;
  void *wb = sc.get(size_t(cr) * size_t(n_cols) * 2);
  void *ws = sc.get(kLtWorkspace);
  if (!wb || !ws) return kDqUnavailable;

  const size_t rb = swamp::row_bytes(int(dtype), size_t(n_cols));
  const float alpha = 1.0f, beta = 0.0f;
  for (int r0 = 0; r0 < n_rows; r0 += cr) {
    const int rows = std::min(cr, n_rows - r0);
    LtPlan *p = rows == cr ? p_full : p_last;
    const uint8_t *w = static_cast<const uint8_t *>(d_w) + size_t(r0) * rb;
    if (int rc = swamp_launch_dequant_bf16(dtype, w, wb, size_t(rows) * size_t(n_cols), s))
      return rc;
    float *y = d_y + r0;
    LtAlgo use;
    {
      // first launch of the shape: measure the candidates on this chunk's
      // weights (its part of y is written over by the launch below)
      std::lock_guard<std::mutex> lock(lt_state(dev).mu);
      lt_tune(dev, *p, wb, d_x, y, ws, s);
      use = p->use;
    }
    if (hipblasLtMatmul(lt_state(dev).handle, p->op, &alpha, wb, p->a, d_x, p->b, &beta, y, p->d,
                        y, p->d, &use.algo, ws, use.ws, s) != HIPBLAS_STATUS_SUCCESS)
      return SWAMP_ELAUNCH;
  }
  return SWAMP_OK;
}
