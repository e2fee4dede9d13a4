/*
 * swamp_gpu.h -- device-management C API of libswamp_gpu.so.
 *
 * The reference's GPU bridge (swamp-gpu/src/lib.rs) dlopens one library
 * named libswamp_gpu.so (lib.rs:30-54) and looks every symbol up in it by
 * name on each call.  Its device buffers come from gpu_alloc / gpu_free
 * (lib.rs:110-142), its streams from gpu_stream_create (lib.rs:275-347) and
 * its timing events from gpu_event_* (lib.rs:599-665).  This library takes
 * that file name, so it exports the same functions with the same names,
 * signatures and return conventions as the reference's CUDA implementation
 * (swamp-gpu/kernels/fused_attention.cu:133-189, :411-455, :816-858),
 * here on HIP.  Failures print one line to stderr and return -1 / NULL /
 * -1.0f, as there.
 *
 * Handles: a stream is a hipStream_t and an event a hipEvent_t, both passed
 * as void* (the reference's cudaStream_t / cudaEvent_t are opaque pointers
 * too); NULL is the default stream.  Every stream is created at the default
 * priority.
 *
 * The attention entry points of the reference's library (gpu_attention_*,
 * gpu_alloc_kv_buffer*, gpu_copy_kv_*, gpu_graph_*) are not part of the
 * quantized-matmul path and are not exported: their lookup fails with
 * GpuError::Symbol and the engine keeps attention on the CPU
 * (swamp-engine/src/executor.rs:331-349).
 */
#ifndef SWAMP_GPU_H
#define SWAMP_GPU_H

#include <stddef.h>

#ifndef SWAMP_API
#define SWAMP_API __attribute__((visibility("default")))
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* gpu_init (fused_attention.cu:133-143): selects device 0, creates its
 * context.  0 on success, -1 on failure. */
SWAMP_API int gpu_init(void);

/* gpu_alloc / gpu_free (fused_attention.cu:146-159): device memory.
 * gpu_alloc returns NULL on failure; gpu_free(NULL) does nothing. */
SWAMP_API void *gpu_alloc(size_t bytes);
SWAMP_API void gpu_free(void *ptr);

/* Synchronous copies and device-wide synchronisation
 * (fused_attention.cu:162-189).  0 / -1. */
SWAMP_API int gpu_copy_to_device(void *dst, const void *src, size_t bytes);
SWAMP_API int gpu_copy_to_host(void *dst, const void *src, size_t bytes);
SWAMP_API int gpu_sync(void);

/* Streams (fused_attention.cu:411-432).  gpu_stream_create returns NULL on
 * failure; gpu_stream_destroy(NULL) does nothing. */
SWAMP_API void *gpu_stream_create(void);
SWAMP_API void gpu_stream_destroy(void *stream);
SWAMP_API int gpu_stream_synchronize(void *stream);

/* Copies queued on a stream (fused_attention.cu:436-454); the host side
 * must be pinned memory for the copy to overlap.  0 / -1. */
SWAMP_API int gpu_copy_to_device_async(void *dst, const void *src, size_t bytes, void *stream);
SWAMP_API int gpu_copy_to_host_async(void *dst, const void *src, size_t bytes, void *stream);

/* Events (fused_attention.cu:816-856).  gpu_event_create returns NULL on
 * failure; gpu_event_elapsed_ms returns -1.0f on failure. */
SWAMP_API void *gpu_event_create(void);
SWAMP_API int gpu_event_record(void *event, void *stream);
SWAMP_API int gpu_event_synchronize(void *event);
SWAMP_API float gpu_event_elapsed_ms(void *start, void *end);
SWAMP_API void gpu_event_destroy(void *event);

#ifdef __cplusplus
}
#endif
#endif
