// device.hip -- device management for callers of libswamp_gpu.so
// (include/swamp_gpu.h): buffers, copies, streams and events, under the
// names the reference's Rust bridge resolves in the library it loads
// (swamp-gpu/src/lib.rs:62-71, :110-142, :239-347, :599-665).  Return
// conventions follow swamp-gpu/kernels/fused_attention.cu:133-189,
// :411-455, :816-858: 0 / -1 for status, NULL for a failed handle,
// -1.0f for a failed elapsed time, one stderr line per failure.
#include <cstdio>

#include "swamp_common.hpp"
#include "swamp_gpu.h"

namespace {

int fail(const char *what, hipError_t e) {
  std::fprintf(stderr, "%s failed: %s\n", what, hipGetErrorString(e));
  return -1;
}

}  // namespace

extern "C" {

int gpu_init(void) {
  // the reference binds device 0 (fused_attention.cu:134)
  hipError_t e = hipSetDevice(0);
  if (e != hipSuccess) return fail("gpu_init: hipSetDevice", e);
  e = hipFree(nullptr);  // create the context now rather than on first use
  if (e != hipSuccess) return fail("gpu_init: context", e);
  return swamp_gpu_init() == SWAMP_OK ? 0 : -1;
}

void *gpu_alloc(size_t bytes) {
  void *p = nullptr;
  const hipError_t e = hipMalloc(&p, bytes);
  if (e != hipSuccess) {
    std::fprintf(stderr, "gpu_alloc(%zu) failed: %s\n", bytes, hipGetErrorString(e));
    return nullptr;
  }
  return p;
}

void gpu_free(void *ptr) {
  if (ptr) (void)hipFree(ptr);
}

int gpu_copy_to_device(void *dst, const void *src, size_t bytes) {
  const hipError_t e = hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice);
  return e == hipSuccess ? 0 : fail("gpu_copy_to_device", e);
}

int gpu_copy_to_host(void *dst, const void *src, size_t bytes) {
  const hipError_t e = hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost);
  return e == hipSuccess ? 0 : fail("gpu_copy_to_host", e);
}

int gpu_sync(void) {
  const hipError_t e = hipDeviceSynchronize();
  return e == hipSuccess ? 0 : fail("gpu_sync", e);
}

void *gpu_stream_create(void) {
  hipStream_t s = nullptr;
  const hipError_t e = hipStreamCreate(&s);  // default priority
  if (e != hipSuccess) {
    fail("gpu_stream_create", e);
    return nullptr;
  }
  return s;
}

void gpu_stream_destroy(void *stream) {
  if (stream) (void)hipStreamDestroy(static_cast<hipStream_t>(stream));
}

int gpu_stream_synchronize(void *stream) {
  const hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
  return e == hipSuccess ? 0 : fail("gpu_stream_synchronize", e);
}

int gpu_copy_to_device_async(void *dst, const void *src, size_t bytes, void *stream) {
  const hipError_t e =
      hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? 0 : fail("gpu_copy_to_device_async", e);
}

int gpu_copy_to_host_async(void *dst, const void *src, size_t bytes, void *stream) {
  const hipError_t e =
      hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? 0 : fail("gpu_copy_to_host_async", e);
}

void *gpu_event_create(void) {
  hipEvent_t ev = nullptr;
  const hipError_t e = hipEventCreate(&ev);
  if (e != hipSuccess) {
    fail("gpu_event_create", e);
    return nullptr;
  }
  return ev;
}

int gpu_event_record(void *event, void *stream) {
  const hipError_t e =
      hipEventRecord(static_cast<hipEvent_t>(event), static_cast<hipStream_t>(stream));
  return e == hipSuccess ? 0 : fail("gpu_event_record", e);
}

int gpu_event_synchronize(void *event) {
  const hipError_t e = hipEventSynchronize(static_cast<hipEvent_t>(event));
  return e == hipSuccess ? 0 : fail("gpu_event_synchronize", e);
}

float gpu_event_elapsed_ms(void *start, void *end) {
  float ms = 0.0f;
  const hipError_t e =
      hipEventElapsedTime(&ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(end));
  if (e != hipSuccess) {
    fail("gpu_event_elapsed_ms", e);
    return -1.0f;
  }
  return ms;
}

void gpu_event_destroy(void *event) {
  if (event) (void)hipEventDestroy(static_cast<hipEvent_t>(event));
}

}  // extern "C"
