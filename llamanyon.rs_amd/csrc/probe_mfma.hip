// probe_mfma.hip -- microbenchmark of the matrix-core issue rules the GEMM
// kernels are designed around (libswamp_probe.so, driven by
// `bench.py --mfma-probe`; not part of libswamp_gpu.so).
//
// Every configuration runs one workgroup per CU; each MFMA wave issues
// back-to-back V_MFMA_F32_32X32X16_BF16 on 8 independent accumulators, with
// V vector-ALU fmas per MFMA beside them, and optionally re-reads its A
// fragment from LDS after each MFMA (one 16-byte read per MFMA, as the
// prefill GEMMs do) and takes random instead of constant bf16 operands (the
// card lowers its clock under random data).  Waves per SIMD:
//   kind 0: one wave per SIMD, MFMAs and VALU in that wave;
//   kind 1: two waves per SIMD, both issuing MFMAs and VALU;
//   kind 2: two waves per SIMD, one issuing only MFMAs, the other only the
//           VALU work.
// The result is the wall time of the launch; TFLOP/s follow from the MFMA
// count.
#include <hip/hip_runtime.h>
#include <stdint.h>

#define SWAMP_PROBE_API extern "C" __attribute__((visibility("default")))

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kLds = 65536;

template <int KIND, int V, bool RND, bool LDS>
__global__ void __launch_bounds__(KIND == 0 ? 256 : 512, 1)
    probe_kernel(float *__restrict__ out, int iters) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[kLds];
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  for (int i = t; i < kLds / 4; i += blockDim.x) {
    uint32_t h = uint32_t(i) * 2654435761u;
    h ^= h >> 13;
    h *= 0x5bd1e995u;
    h ^= h >> 15;
    // two bf16 values in [-1, 1) (random) or 1.0 (constant)
    const uint32_t lo = 0x3f00u | (h & 0x7fu) | ((h >> 7 & 1u) << 15);
    const uint32_t hi = 0x3f00u | (h >> 8 & 0x7fu) | ((h >> 15 & 1u) << 15);
    reinterpret_cast<uint32_t *>(lds)[i] = RND ? (lo | hi << 16) : 0x3f803f80u;
  }
  __syncthreads();
  const bool mfma_wave = KIND != 2 || w < 4, valu_wave = KIND != 2 || w >= 4;
  f32x16_t acc[8];
  for (int j = 0; j < 8; j++)
    for (int e = 0; e < 16; e++) acc[j][e] = 0.f;
  bf16x8_t a[8];
  for (int j = 0; j < 8; j++)
    a[j] = *reinterpret_cast<const bf16x8_t *>(lds + ((t * 16 + j * 1024) & (kLds - 1)));
  const bf16x8_t b = *reinterpret_cast<const bf16x8_t *>(lds + ((t * 16 + 4096) & (kLds - 1)));
  float f[8];
  for (int i = 0; i < 8; i++) f[i] = float(lane + i) * 0.37f;
  const uint32_t off = uint32_t(t * 16) & (kLds - 1);
  for (int it = 0; it < iters; it++) {
    if (mfma_wave) {
#pragma unroll
      for (int j = 0; j < 8; j++) {
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[j], b, acc[j], 0, 0, 0);
        if (LDS)
          a[j] = *reinterpret_cast<const bf16x8_t *>(
              lds + ((off + uint32_t(j) * 2048u + uint32_t(it) * 16u) & (kLds - 1)));
      }
    }
    if (valu_wave) {
#pragma unroll
      for (int v = 0; v < 8 * V; v++) f[v % 8] = __builtin_fmaf(f[v % 8], 0.999f, 0.001f * v);
    }
    if (KIND != 2) {
#pragma unroll
      for (int j = 0; j < 8; j++) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (LDS) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        if (V > 0) __builtin_amdgcn_sched_group_barrier(0x002, V, 0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  float s = 0.f;
  for (int j = 0; j < 8; j++)
    for (int e = 0; e < 16; e++) s += acc[j][e];
  for (int i = 0; i < 8; i++) s += f[i];
  out[size_t(blockIdx.x) * blockDim.x + t] = s;
}

struct Config {
  void (*fn)(float *, int);
  int kind, valu, rnd, lds;
};

#define PROBE(K, V, R, L) {probe_kernel<K, V, R, L>, K, V, R, L}
const Config kConfigs[] = {
    PROBE(0, 0, false, false), PROBE(0, 2, false, false), PROBE(0, 4, false, false),
    PROBE(1, 0, false, false), PROBE(1, 2, false, false), PROBE(1, 4, false, false),
    PROBE(2, 2, false, false), PROBE(2, 4, false, false),
    PROBE(1, 0, true, false),  PROBE(1, 0, true, true),   PROBE(1, 3, true, true),
    PROBE(0, 3, true, true),
};
#undef PROBE

}  // namespace

// Number of configurations, and configuration i's kind, VALU per MFMA,
// random operands and LDS re-reads (any pointer may be null).
SWAMP_PROBE_API int swamp_probe_mfma_configs(int i, int *kind, int *valu, int *rnd, int *lds) {
  const int n = int(sizeof(kConfigs) / sizeof(kConfigs[0]));
  if (i < 0 || i >= n) return n;
  if (kind) *kind = kConfigs[i].kind;
  if (valu) *valu = kConfigs[i].valu;
  if (rnd) *rnd = kConfigs[i].rnd;
  if (lds) *lds = kConfigs[i].lds;
  return n;
}

// Runs configuration i once untimed and `reps` times timed, one workgroup per
// CU, `iters` trips of 8 MFMAs per MFMA wave; *ms = mean time per launch and
// *mfmas = MFMA instructions per launch.  0 on success, -1 on a bad index or
// a HIP error.
SWAMP_PROBE_API int swamp_probe_mfma_run(int i, int iters, int reps, float *ms, double *mfmas) {
  const int n = int(sizeof(kConfigs) / sizeof(kConfigs[0]));
  if (i < 0 || i >= n || iters <= 0 || reps <= 0 || !ms || !mfmas) return -1;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return -1;
  const Config &c = kConfigs[i];
  const int threads = c.kind == 0 ? 256 : 512;
  float *out = nullptr;
  if (hipMalloc(&out, size_t(cus) * threads * sizeof(float)) != hipSuccess) return -1;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  int rc = -1;
  if (hipEventCreate(&e0) == hipSuccess && hipEventCreate(&e1) == hipSuccess) {
    hipLaunchKernelGGL(c.fn, dim3(cus), dim3(threads), 0, nullptr, out, iters);
    bool ok = hipEventRecord(e0, nullptr) == hipSuccess;
    for (int r = 0; ok && r < reps; r++)
      hipLaunchKernelGGL(c.fn, dim3(cus), dim3(threads), 0, nullptr, out, iters);
    float t = 0.f;
    ok = ok && hipGetLastError() == hipSuccess && hipEventRecord(e1, nullptr) == hipSuccess &&
         hipEventSynchronize(e1) == hipSuccess && hipEventElapsedTime(&t, e0, e1) == hipSuccess;
    if (ok) {
      *ms = t / float(reps);
      // MFMA waves per CU: 4 (kinds 0 and 2) or 8 (kind 1), 8 MFMAs per trip
      *mfmas = double(cus) * (c.kind == 1 ? 8 : 4) * 8.0 * double(iters);
      rc = 0;
    }
  }
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  (void)hipFree(out);
  return rc;
}
