// gemv_fused.hip -- decode GEMV with the engine's adjacent f32 step fused
// into the x prologue of the item kernel (gemv_core.hpp):
//
//  * RMSNorm -> GEMV: rmsnorm(x_norm, x, w_norm, eps) followed by
//    forward_linear_multi / forward_linear on x_norm (swamp-engine/src/
//    executor.rs:433-445 for QKV, :488-499 for gate+up, :530-533 for the
//    logits).  Every workgroup loads all of x anyway, so it computes the sum
//    of squares itself (a 16 KB re-read from L2 per workgroup) and never
//    writes x_norm.
//  * SiLU * up -> down GEMV: silu(gate); mul_in_place(gate, up);
//    forward_linear(down, gate) and, when accumulate is set, the residual
//    add_in_place(x, ffn_down) (executor.rs:501-506): y += W h.
//
// Both keep one 64-weight item per lane (n_cols <= 32768), which covers the
// hidden and intermediate sizes of the Llama family.
#include "gemv_core.hpp"

int swamp_launch_gemv_rmsnorm(int n_mats, const uint32_t *dtypes, const void *const *d_ws,
                              const int *row_counts, const float *d_x, const float *d_norm_w,
                              float eps, float *const *d_ys, int n_cols, hipStream_t s) {
  Pro pro;
  pro.x2 = d_norm_w;
  pro.eps = eps;
  return launch_multi<kProRmsNorm, true>(n_mats, dtypes, d_ws, row_counts, d_x, pro, d_ys, n_cols, s);
}

int swamp_launch_gemv_swiglu(uint32_t dtype, const void *d_w, const float *d_gate,
                             const float *d_up, float *d_y, int n_rows, int n_cols,
                             int accumulate, hipStream_t s) {
  if (n_rows == 0) return SWAMP_OK;
  if (!item_path_ok(dtype, n_cols) || n_cols / 64 > 512) return SWAMP_ESHAPE;
  MatSet ms;
  const void *ws[1] = {d_w};
  float *ys[1] = {d_y};
  const int tr = tile_rows_for(dtype, n_cols, n_rows, true);
  build_matset(ms, 1, ws, ys, &n_rows, tr);
  ms.wpc = waves_per_cu_for(dtype, n_cols, n_rows, true);
  Pro pro;
  pro.x2 = d_up;
  if (accumulate) return dispatch<kProSwiGLUAcc, true>(dtype, ms, d_gate, pro, n_cols, tr, s);
  return dispatch<kProSwiGLU, true>(dtype, ms, d_gate, pro, n_cols, tr, s);
}
