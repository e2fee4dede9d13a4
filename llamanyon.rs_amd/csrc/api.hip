// api.hip -- the C ABI of libswamp_gpu.so (declared in include/swamp_qmm.h).
//
// Validation and dispatch only; kernels live in dequant.hip, gemv.hip,
// gemv_fused.hip, gemv_batched.hip, gemm.hip and gemm_i8.hip.  The error behaviour mirrors the
// reference: shape asserts of fused_gemv_q4k (fused_gemv_q4k.rs:66-70) and
// the bail! of forward_linear (linear.rs:23-25) become negative return
// codes, checked before anything is launched; the two legacy host-pointer
// exports keep their silent-return behaviour.
#include <algorithm>
#include <mutex>
#include <thread>
#include <vector>

#include "swamp_common.hpp"
#include "swamp_gguf.h"

namespace swamp {

// Scratch of swamp_qgemv_batched_noalloc: a fixed array in device memory,
// one copy per device the library runs on (held until the process ends),
// shared by every call of that entry point on that device.  Host code uses
// it only through the address hipGetSymbolAddress returns for the device
// (g_scratch), never through its name.
constexpr size_t kNoAllocScratchBytes = size_t(32) << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
DeviceInfo g_info[kMaxDevices];
std::once_flag g_once[kMaxDevices];
void *g_scratch[kMaxDevices];  // device address of `scratch` per device (nullptr: lookup failed)

size_t block_size(uint32_t dt) {
  switch (dt) {
  case SWAMP_F32: case SWAMP_F16: case SWAMP_BF16: return 1;
  case SWAMP_Q4_0: case SWAMP_Q8_0: return 32;
  case SWAMP_Q4_K: case SWAMP_Q6_K: return 256;
  default: break;
  }
  // rest of the GgmlDType table (swamp-gguf/src/dtype.rs:79-89)
  switch (dt) {
  case 24: case 25: case 26: case 27: case 28: return 1;
  case 3: case 6: case 7: case 9: case 20: case 23: return 32;
  case 10: case 11: case 13: case 14: case 15: case 16: case 17: case 18:
  case 19: case 21: case 22: case 29: return 256;
  default: return 0;
  }
}

size_t type_size(uint32_t dt) {
  switch (dt) {  // swamp-gguf/src/dtype.rs:92-132
  case 0: return 4;   case 1: return 2;   case 30: return 2;  case 28: return 8;
  case 24: return 1;  case 25: return 2;  case 26: return 4;  case 27: return 8;
  case 2: return 18;  case 3: return 20;  case 6: return 22;  case 7: return 24;
  case 8: return 34;  case 9: return 40;  case 10: return 84; case 11: return 110;
  case 12: return 144; case 13: return 176; case 14: return 210; case 15: return 292;
  case 16: return 66; case 17: return 74; case 22: return 82; case 18: return 98;
  case 21: return 110; case 20: return 18; case 23: return 136; case 19: return 50;
  case 29: return 56;
  default: return 0;
  }
}

bool is_weight_dtype(uint32_t dt) {
  return dt == SWAMP_Q4_0 || dt == SWAMP_Q8_0 || dt == SWAMP_Q4_K || dt == SWAMP_Q6_K;
}

bool aligned(const void *p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

// Required base alignment of a weight buffer (dword vector loads; Q4_K
// also loads its 16-byte headers as one vector).
uintptr_t weight_align(uint32_t dt) { return dt == SWAMP_Q4_K ? 16 : 4; }

int ensure_device(int *dev_out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return SWAMP_ENODEVICE;
  if (dev < 0 || dev >= kMaxDevices) return SWAMP_ENODEVICE;
  std::call_once(g_once[dev], [dev] {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
        cus > 0)
      g_info[dev].num_cus = cus;
    g_info[dev].device = dev;
    // this device's copy of the no-alloc scratch array (dev is current)
    void *p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) == hipSuccess) {
      g_scratch[dev] = p;
    } else {
      (void)hipGetLastError();
      g_scratch[dev] = nullptr;
    }
  });
  if (dev_out) *dev_out = dev;
  return SWAMP_OK;
}

int check_gemv_args(uint32_t dtype, const void *d_w, size_t w_len, int n_rows, int n_cols) {
  if (!is_weight_dtype(dtype)) return SWAMP_EDTYPE;
  if (!d_w || n_rows < 0 || n_cols < 0) return SWAMP_EINVAL;
  if (n_cols % int(block_size(dtype)) != 0) return SWAMP_ESHAPE;
  if (!aligned(d_w, weight_align(dtype))) return SWAMP_EINVAL;
  const size_t need = size_t(n_rows) * (size_t(n_cols) / block_size(dtype)) * type_size(dtype);
  if (w_len < need) return SWAMP_ESHAPE;
  return SWAMP_OK;
}

// Rows the fused-prologue GEMVs take: the item kernel with one item per
// lane (whole 64-weight items, Q6_K rows of an even number of blocks,
// n_cols <= 32768).
bool fused_cols_ok(uint32_t dt, int n_cols) {
  if (n_cols <= 0 || n_cols > 32768) return false;
  return n_cols % (dt == SWAMP_Q6_K ? 512 : dt == SWAMP_Q4_K ? 256 : 64) == 0;
}

}  // namespace

const DeviceInfo &device_info() {
  int dev = 0;
  ensure_device(&dev);
  return g_info[dev];
}

void *stream_workspace(hipStream_t s, size_t bytes) {
  struct Entry {
    int dev;
    hipStream_t s;
    std::thread::id tid;  // for hipStreamPerThread, one stream per host thread
    void *p;
    size_t bytes;
    bool captured;  // handed out while s was being captured: a graph may hold it
  };
  static std::mutex mu;
  static std::vector<Entry> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  const std::thread::id tid =
      s == hipStreamPerThread ? std::this_thread::get_id() : std::thread::id();
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &st) != hipSuccess) return nullptr;
  const bool capturing = st != hipStreamCaptureStatusNone;
  std::lock_guard<std::mutex> lock(mu);
  Entry *e = nullptr;
  for (Entry &c : cache)
    if (c.dev == dev && c.s == s && c.tid == tid) e = &c;
  if (e && e->bytes >= bytes) {
    e->captured = e->captured || capturing;
    return e->p;
  }
  // a (larger) buffer is needed: never while the stream is being captured
  if (capturing) return nullptr;
  void *p = nullptr;
  if (hipMallocAsync(&p, bytes, s) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  if (e) {
    // A buffer a captured call used is never released: the graph's replays
    // write it until the process ends.  Any other is released after the
    // work already queued on s.
    if (!e->captured) (void)hipFreeAsync(e->p, s);
    e->p = p;
    e->bytes = bytes;
    e->captured = false;
  } else {
    cache.push_back(Entry{dev, s, tid, p, bytes, false});
  }
  return p;
}

}  // namespace swamp

using namespace swamp;

namespace {

__global__ void i8dot_kernel(const int8_t *__restrict__ w, const int8_t *__restrict__ a, int k,
                             int *__restrict__ out) {
  // one workgroup of 256 lanes; exact int32 dot (the reference's scalar
  // arm, swamp-kernels/src/lib.rs:477-481)
  __shared__ int part[4];
  int s = 0;
  for (int i = threadIdx.x; i < k; i += blockDim.x) s += int(w[i]) * int(a[i]);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off, 64);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) *out = part[0] + part[1] + part[2] + part[3];
}

}  // namespace

// y[0..n) = 0 for a sum over no columns (n_cols == 0), with a kernel so the
// call stays capturable in a graph.
static __global__ void fill_zero_kernel(float *__restrict__ y, size_t n) {
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += size_t(gridDim.x) * blockDim.x)
    y[i] = 0.0f;
}

static int fill_zero(float *d_y, size_t n, hipStream_t s) {
  if (n == 0) return SWAMP_OK;
  const size_t blocks = std::min<size_t>((n + 255) / 256, 4096);
  fill_zero_kernel<<<unsigned(blocks), 256, 0, s>>>(d_y, n);
  return hipGetLastError() == hipSuccess ? SWAMP_OK : SWAMP_ELAUNCH;
}

int swamp_launch_i8dot(const int8_t *d_w, const int8_t *d_a, int k, int *d_out, hipStream_t s) {
  i8dot_kernel<<<1, 256, 0, s>>>(d_w, d_a, k, d_out);
  return hipGetLastError() == hipSuccess ? SWAMP_OK : SWAMP_ELAUNCH;
}

extern "C" {

int swamp_gpu_init(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return SWAMP_ENODEVICE;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return SWAMP_ENODEVICE;
  if (hipSetDevice(dev) != hipSuccess) return SWAMP_ENODEVICE;
  if (hipFree(nullptr) != hipSuccess) return SWAMP_ENODEVICE;  // create the context
  return ensure_device(nullptr);
}

const char *swamp_strerror(int code) {
  switch (code) {
  case SWAMP_OK: return "ok";
  case SWAMP_EINVAL: return "invalid argument (null, negative size or misaligned pointer)";
  case SWAMP_EDTYPE: return "dtype not supported by this entry point";
  case SWAMP_ESHAPE: return "shape mismatch (n_cols not a multiple of the block, or buffer too small)";
  case SWAMP_ELAUNCH: return "HIP launch or copy failed";
  case SWAMP_ENODEVICE: return "no HIP device";
  case SWAMP_EWORKSPACE: return "workspace missing or too small";
  case SWAMP_EIO: return "GGUF file could not be opened, mapped or fully read";
  case SWAMP_EMAGIC: return "not a GGUF file (bad magic)";
  case SWAMP_EVERSION: return "unsupported GGUF version";
  case SWAMP_ENOTFOUND: return "tensor or metadata key not found";
  case SWAMP_ETENSOR: return "tensor bytes lie outside the file";
  default: return "unknown error";
  }
}

size_t swamp_block_size(uint32_t dtype) { return block_size(dtype); }
size_t swamp_type_size(uint32_t dtype) { return type_size(dtype); }
size_t swamp_nbytes_for(uint32_t dtype, size_t n) {
  const size_t bs = block_size(dtype);
  return bs ? (n + bs - 1) / bs * type_size(dtype) : 0;
}

int swamp_qdequant(uint32_t dtype, const void *d_raw, size_t raw_len, float *d_dst, size_t n,
                   void *stream) {
  const bool ok_dt = is_weight_dtype(dtype) || dtype == SWAMP_F32 || dtype == SWAMP_F16 ||
                     dtype == SWAMP_BF16;
  if (!ok_dt) return SWAMP_EDTYPE;
  if (n == 0) return SWAMP_OK;
  if (!d_raw || !d_dst) return SWAMP_EINVAL;
  if (raw_len < swamp_nbytes_for(dtype, n)) return SWAMP_ESHAPE;
  const uintptr_t al = dtype == SWAMP_Q4_K ? 16 : dtype == SWAMP_F32 ? 4 : 2;
  if (!aligned(d_raw, al) || !aligned(d_dst, 4)) return SWAMP_EINVAL;
  if (int rc = ensure_device(nullptr)) return rc;
  return swamp_launch_dequant(dtype, d_raw, d_dst, n, static_cast<hipStream_t>(stream));
}

int swamp_qdequant_bf16(uint32_t dtype, const void *d_raw, size_t raw_len, void *d_dst, size_t n,
                        void *stream) {
  if (!is_weight_dtype(dtype)) return SWAMP_EDTYPE;
  if (n == 0) return SWAMP_OK;
  if (!d_raw || !d_dst) return SWAMP_EINVAL;
  if (n % swamp_block_size(dtype) != 0) return SWAMP_ESHAPE;
  if (raw_len < swamp_nbytes_for(dtype, n)) return SWAMP_ESHAPE;
  const uintptr_t al = dtype == SWAMP_Q6_K ? 2 : weight_align(dtype);
  if (!aligned(d_raw, al) || !aligned(d_dst, 16)) return SWAMP_EINVAL;
  if (int rc = ensure_device(nullptr)) return rc;
  return swamp_launch_dequant_bf16(dtype, d_raw, d_dst, n, static_cast<hipStream_t>(stream));
}

int swamp_qgemv(uint32_t dtype, const void *d_w, size_t w_len, const float *d_x, float *d_y,
                int n_rows, int n_cols, void *stream) {
  if (int rc = check_gemv_args(dtype, d_w, w_len, n_rows, n_cols)) return rc;
  if (!d_x || !d_y) return SWAMP_EINVAL;
  if (!aligned(d_x, 16) || !aligned(d_y, 4)) return SWAMP_EINVAL;
  if (n_rows == 0) return SWAMP_OK;
  if (int rc = ensure_device(nullptr)) return rc;
  if (n_cols == 0) return fill_zero(d_y, size_t(n_rows), static_cast<hipStream_t>(stream));
  return swamp_launch_gemv(dtype, d_w, d_x, d_y, n_rows, n_cols, static_cast<hipStream_t>(stream));
}

int swamp_qgemv_f16x(uint32_t dtype, const void *d_w, size_t w_len, const float *d_x, float *d_y,
                     int n_rows, int n_cols, void *stream) {
  if (int rc = check_gemv_args(dtype, d_w, w_len, n_rows, n_cols)) return rc;
  if (!d_x || !d_y) return SWAMP_EINVAL;
  if (!aligned(d_x, 16) || !aligned(d_y, 4)) return SWAMP_EINVAL;
  if (n_rows == 0) return SWAMP_OK;
  if (int rc = ensure_device(nullptr)) return rc;
  if (n_cols == 0) return fill_zero(d_y, size_t(n_rows), static_cast<hipStream_t>(stream));
  return swamp_launch_gemv_f16x(dtype, d_w, d_x, d_y, n_rows, n_cols,
                                static_cast<hipStream_t>(stream));
}

int swamp_qgemv_multi(int n_mats, const uint32_t *dtypes, const void *const *d_ws,
                      const size_t *w_lens, const int *row_counts, const float *d_x,
                      float *const *d_ys, int n_cols, void *stream) {
  if (n_mats < 0 || n_mats > SWAMP_MULTI_MAX) return SWAMP_EINVAL;
  if (n_mats == 0) return SWAMP_OK;
  if (!dtypes || !d_ws || !w_lens || !row_counts || !d_ys || !d_x) return SWAMP_EINVAL;
  if (!aligned(d_x, 16)) return SWAMP_EINVAL;
  for (int i = 0; i < n_mats; i++) {
    if (int rc = check_gemv_args(dtypes[i], d_ws[i], w_lens[i], row_counts[i], n_cols)) return rc;
    if (!d_ys[i] || !aligned(d_ys[i], 4)) return SWAMP_EINVAL;
  }
  if (int rc = ensure_device(nullptr)) return rc;
  if (n_cols == 0) {
    for (int i = 0; i < n_mats; i++)
      if (int rc = fill_zero(d_ys[i], size_t(row_counts[i]), static_cast<hipStream_t>(stream)))
        return rc;
    return SWAMP_OK;
  }
  return swamp_launch_gemv_multi(n_mats, dtypes, d_ws, row_counts, d_x, d_ys, n_cols,
                                 static_cast<hipStream_t>(stream));
}

int swamp_qgemv_many(int n, const uint32_t *dtypes, const void *const *d_ws,
                     const size_t *w_lens, const int *n_rows, const int *n_cols,
                     const float *const *d_xs, float *const *d_ys, void *stream) {
  if (n < 0) return SWAMP_EINVAL;
  if (n == 0) return SWAMP_OK;
  if (!dtypes || !d_ws || !w_lens || !n_rows || !n_cols || !d_xs || !d_ys) return SWAMP_EINVAL;
  for (int i = 0; i < n; i++) {  // every GEMV is checked before any is launched
    if (int rc = check_gemv_args(dtypes[i], d_ws[i], w_lens[i], n_rows[i], n_cols[i])) return rc;
    if (!d_xs[i] || !d_ys[i] || !aligned(d_xs[i], 16) || !aligned(d_ys[i], 4)) return SWAMP_EINVAL;
  }
  if (int rc = ensure_device(nullptr)) return rc;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  for (int i = 0; i < n; i++) {
    if (n_rows[i] == 0) continue;
    const int rc = n_cols[i] == 0
                       ? fill_zero(d_ys[i], size_t(n_rows[i]), s)
                       : swamp_launch_gemv(dtypes[i], d_ws[i], d_xs[i], d_ys[i], n_rows[i],
                                           n_cols[i], s);
    if (rc) return rc;
  }
  return SWAMP_OK;
}

int swamp_qgemv_rmsnorm(int n_mats, const uint32_t *dtypes, const void *const *d_ws,
                        const size_t *w_lens, const int *row_counts, const float *d_x,
                        const float *d_norm_w, float eps, float *const *d_ys, int n_cols,
                        void *stream) {
  if (n_mats < 0 || n_mats > SWAMP_MULTI_MAX) return SWAMP_EINVAL;
  if (n_mats == 0) return SWAMP_OK;
  if (!dtypes || !d_ws || !w_lens || !row_counts || !d_ys || !d_x || !d_norm_w)
    return SWAMP_EINVAL;
  if (!aligned(d_x, 16) || !aligned(d_norm_w, 16)) return SWAMP_EINVAL;
  for (int i = 0; i < n_mats; i++) {
    if (int rc = check_gemv_args(dtypes[i], d_ws[i], w_lens[i], row_counts[i], n_cols)) return rc;
    if (!fused_cols_ok(dtypes[i], n_cols)) return SWAMP_ESHAPE;
    if (!d_ys[i] || !aligned(d_ys[i], 4)) return SWAMP_EINVAL;
  }
  if (int rc = ensure_device(nullptr)) return rc;
  return swamp_launch_gemv_rmsnorm(n_mats, dtypes, d_ws, row_counts, d_x, d_norm_w, eps, d_ys,
                                   n_cols, static_cast<hipStream_t>(stream));
}

int swamp_qgemv_swiglu(uint32_t dtype, const void *d_w, size_t w_len, const float *d_gate,
                       const float *d_up, float *d_y, int n_rows, int n_cols, int accumulate,
                       void *stream) {
  if (int rc = check_gemv_args(dtype, d_w, w_len, n_rows, n_cols)) return rc;
  if (!fused_cols_ok(dtype, n_cols)) return SWAMP_ESHAPE;
  if (!d_gate || !d_up || !d_y) return SWAMP_EINVAL;
  if (!aligned(d_gate, 16) || !aligned(d_up, 16) || !aligned(d_y, 4)) return SWAMP_EINVAL;
  if (n_rows == 0) return SWAMP_OK;
  if (int rc = ensure_device(nullptr)) return rc;
  return swamp_launch_gemv_swiglu(dtype, d_w, d_gate, d_up, d_y, n_rows, n_cols,
                                  accumulate ? 1 : 0, static_cast<hipStream_t>(stream));
}

int swamp_qgemv_batched(uint32_t dtype, const void *d_w, size_t w_len, const float *d_x,
                        float *d_y, int n_tok, int n_rows, int n_cols, int accumulate,
                        void *stream) {
  if (int rc = check_gemv_args(dtype, d_w, w_len, n_rows, n_cols)) return rc;
  if (n_tok < 0) return SWAMP_EINVAL;
  if (dtype == SWAMP_Q6_K && accumulate) return SWAMP_EDTYPE;  // no Q6_K batched kernel contract
  if (n_tok == 0 || n_rows == 0) return SWAMP_OK;  // linear.rs:184
  if (!d_x || !d_y || !aligned(d_x, 16) || !aligned(d_y, 4)) return SWAMP_EINVAL;
  if (dtype != SWAMP_Q4_K && n_cols % 64 != 0) return SWAMP_ESHAPE;
  if (int rc = ensure_device(nullptr)) return rc;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (n_cols == 0)
    return accumulate ? SWAMP_OK : fill_zero(d_y, size_t(n_tok) * size_t(n_rows), s);
  const int acc = accumulate ? 1 : 0;
  Scratch sc = stream_scratch(s, swamp_batched_scratch_bytes(dtype, n_tok, n_rows, n_cols, acc));
  return swamp_launch_gemv_batched(dtype, d_w, d_x, d_y, n_tok, n_rows, n_cols, acc, sc, s);
}

int swamp_qgemm(uint32_t dtype, const void *d_w, size_t w_len, const void *d_x, uint32_t x_type,
                float *d_y, int m, int n_rows, int n_cols, void *stream) {
  if (int rc = check_gemv_args(dtype, d_w, w_len, n_rows, n_cols)) return rc;
  if (m < 0) return SWAMP_EINVAL;
  if (x_type != SWAMP_BF16 && x_type != SWAMP_Q8_0) return SWAMP_EDTYPE;
  if (x_type == SWAMP_Q8_0 && dtype == SWAMP_Q6_K) return SWAMP_EDTYPE;
  if (m == 0 || n_rows == 0) return SWAMP_OK;
  if (!d_x || !d_y || !aligned(d_x, 16) || !aligned(d_y, 4)) return SWAMP_EINVAL;
  if (n_cols % (x_type == SWAMP_Q8_0 ? 128 : 64) != 0) return SWAMP_ESHAPE;
  if (int rc = ensure_device(nullptr)) return rc;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (n_cols == 0) return fill_zero(d_y, size_t(m) * size_t(n_rows), s);
  Scratch sc = stream_scratch(s, swamp_gemm_scratch_bytes(dtype, x_type, m, n_rows, n_cols));
  return swamp_launch_gemm(dtype, d_w, d_x, x_type, d_y, m, n_rows, n_cols, sc, s);
}

int swamp_qgemv_batched_noalloc(uint32_t dtype, const void *d_w, size_t w_len, const float *d_x,
                                float *d_y, int n_tok, int n_rows, int n_cols, int accumulate,
                                void *stream) {
  if (int rc = check_gemv_args(dtype, d_w, w_len, n_rows, n_cols)) return rc;
  if (n_tok < 0) return SWAMP_EINVAL;
  if (dtype == SWAMP_Q6_K && accumulate) return SWAMP_EDTYPE;
  if (n_tok == 0 || n_rows == 0) return SWAMP_OK;
  if (!d_x || !d_y || !aligned(d_x, 16) || !aligned(d_y, 4)) return SWAMP_EINVAL;
  if (dtype != SWAMP_Q4_K && n_cols % 64 != 0) return SWAMP_ESHAPE;
  int dev = 0;
  if (int rc = ensure_device(&dev)) return rc;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (n_cols == 0)
    return accumulate ? SWAMP_OK : fill_zero(d_y, size_t(n_tok) * size_t(n_rows), s);
  const int acc = accumulate ? 1 : 0;
  const size_t need =
      swamp_batched_scratch_bytes(dtype, n_tok, n_rows, n_cols, acc, kNoAllocScratchBytes);
  if (need > kNoAllocScratchBytes) return SWAMP_EWORKSPACE;
  Scratch sc;
  if (need) {
    if (!g_scratch[dev]) return SWAMP_EWORKSPACE;
    sc.base = static_cast<uint8_t *>(g_scratch[dev]);
    sc.cap = kNoAllocScratchBytes;
  }
  return swamp_launch_gemv_batched(dtype, d_w, d_x, d_y, n_tok, n_rows, n_cols, acc, sc, s);
}

size_t swamp_qgemv_batched_workspace(uint32_t dtype, int n_tok, int n_rows, int n_cols,
                                     int accumulate) {
  if (ensure_device(nullptr) != SWAMP_OK) return 0;
  return swamp_batched_scratch_bytes(dtype, n_tok, n_rows, n_cols, accumulate ? 1 : 0);
}

size_t swamp_qgemm_workspace(uint32_t dtype, uint32_t x_type, int m, int n_rows, int n_cols) {
  if (ensure_device(nullptr) != SWAMP_OK) return 0;
  return swamp_gemm_scratch_bytes(dtype, x_type, m, n_rows, n_cols);
}

int swamp_workspace_reserve(void *stream, size_t bytes) {
  if (int rc = ensure_device(nullptr)) return rc;
  if (bytes == 0) return SWAMP_OK;
  return stream_workspace(static_cast<hipStream_t>(stream), bytes) ? SWAMP_OK : SWAMP_EWORKSPACE;
}

int swamp_rmsnorm_rows(const float *d_x, const float *d_norm_w, float eps, void *d_out,
                       uint32_t out_type, int n_tok, int n_cols, void *stream) {
  if (out_type != SWAMP_F32 && out_type != SWAMP_BF16) return SWAMP_EDTYPE;
  if (n_tok < 0 || n_cols < 0) return SWAMP_EINVAL;
  if (n_cols % 4 != 0) return SWAMP_ESHAPE;
  if (n_tok == 0 || n_cols == 0) return SWAMP_OK;
  if (!d_x || !d_norm_w || !d_out || !aligned(d_x, 16) || !aligned(d_norm_w, 16) ||
      !aligned(d_out, out_type == SWAMP_BF16 ? 8 : 16))
    return SWAMP_EINVAL;
  if (int rc = ensure_device(nullptr)) return rc;
  return swamp_launch_rmsnorm_rows(d_x, d_norm_w, eps, d_out, out_type, n_tok, n_cols,
                                   static_cast<hipStream_t>(stream));
}

int swamp_swiglu(const float *d_gate, const float *d_up, void *d_out, uint32_t out_type, size_t n,
                 void *stream) {
  if (out_type != SWAMP_F32 && out_type != SWAMP_BF16) return SWAMP_EDTYPE;
  if (n % 4 != 0) return SWAMP_ESHAPE;
  if (n == 0) return SWAMP_OK;
  if (!d_gate || !d_up || !d_out || !aligned(d_gate, 16) || !aligned(d_up, 16) ||
      !aligned(d_out, out_type == SWAMP_BF16 ? 8 : 16))
    return SWAMP_EINVAL;
  if (int rc = ensure_device(nullptr)) return rc;
  return swamp_launch_swiglu(d_gate, d_up, d_out, out_type, n, static_cast<hipStream_t>(stream));
}

int swamp_quantize_q8_0(const void *d_x, uint32_t x_type, void *d_q, size_t n, void *stream) {
  if (x_type != SWAMP_F32 && x_type != SWAMP_BF16) return SWAMP_EDTYPE;
  if (n % 32 != 0) return SWAMP_ESHAPE;
  if (n == 0) return SWAMP_OK;
  if (!d_x || !d_q || !aligned(d_x, 4)) return SWAMP_EINVAL;
  if (int rc = ensure_device(nullptr)) return rc;
  return swamp_launch_quantize_q8_0(d_x, x_type, d_q, n, static_cast<hipStream_t>(stream));
}

void swamp_fused_gemv_q4k(const uint8_t *w_raw, const float *x, float *out, int n_rows,
                          int n_cols) {
  // fused_gemv_q4k.rs:799-823: null -> return; n_cols % 256 -> return; out
  // zeroed then written.
  if (!w_raw || !x || !out) return;
  if (n_cols % 256 != 0 || n_rows < 0 || n_cols < 0) return;
  if (ensure_device(nullptr) != SWAMP_OK) return;
  const size_t wb = size_t(n_rows) * (size_t(n_cols) / 256) * 144;
  void *dw = nullptr;
  float *dx = nullptr, *dy = nullptr;
  bool ok = hipMalloc(&dw, wb ? wb : 16) == hipSuccess &&
            hipMalloc(reinterpret_cast<void **>(&dx), size_t(n_cols ? n_cols : 4) * 4) == hipSuccess &&
            hipMalloc(reinterpret_cast<void **>(&dy), size_t(n_rows ? n_rows : 1) * 4) == hipSuccess;
  if (ok) ok = hipMemcpy(dw, w_raw, wb, hipMemcpyHostToDevice) == hipSuccess &&
               hipMemcpy(dx, x, size_t(n_cols) * 4, hipMemcpyHostToDevice) == hipSuccess;
  for (int i = 0; i < n_rows; i++) out[i] = 0.0f;
  if (ok && n_rows > 0 && n_cols > 0)
    ok = swamp_launch_gemv(SWAMP_Q4_K, dw, dx, dy, n_rows, n_cols, nullptr) == SWAMP_OK &&
         hipMemcpy(out, dy, size_t(n_rows) * 4, hipMemcpyDeviceToHost) == hipSuccess;
  (void)hipFree(dw);
  (void)hipFree(dx);
  (void)hipFree(dy);
}

float swamp_gemv_q8_vnni(const int8_t *weights, const int8_t *activations, int k, float scale) {
  if (!weights || !activations || k <= 0) return 0.0f;  // lib.rs:458
  if (ensure_device(nullptr) != SWAMP_OK) return __builtin_nanf("");
  int8_t *dw = nullptr, *da = nullptr;
  int *dout = nullptr;
  int dot = 0;
  bool ok = hipMalloc(reinterpret_cast<void **>(&dw), size_t(k)) == hipSuccess &&
            hipMalloc(reinterpret_cast<void **>(&da), size_t(k)) == hipSuccess &&
            hipMalloc(reinterpret_cast<void **>(&dout), sizeof(int)) == hipSuccess;
  if (ok) ok = hipMemcpy(dw, weights, size_t(k), hipMemcpyHostToDevice) == hipSuccess &&
               hipMemcpy(da, activations, size_t(k), hipMemcpyHostToDevice) == hipSuccess &&
               swamp_launch_i8dot(dw, da, k, dout, nullptr) == SWAMP_OK &&
               hipMemcpy(&dot, dout, sizeof(int), hipMemcpyDeviceToHost) == hipSuccess;
  (void)hipFree(dw);
  (void)hipFree(da);
  (void)hipFree(dout);
  if (!ok) return __builtin_nanf("");
  return float(dot) * scale;
}

}  // extern "C"
