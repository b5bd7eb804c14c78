/* Device runtime of the boundary: C-ABI of
 * minitorch_amd/cuda_kernels/cuda_runtime.so. Device 0 (the current HIP
 * device), the calling thread's default stream (the libraries are built with
 * per-thread default streams; one host thread sees the reference's legacy
 * null-stream ordering). Status convention as in mt_paged.h.
 */
#ifndef MT_RUNTIME_H
#define MT_RUNTIME_H
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Replaces reference mt_malloc / mt_free (src/cuda_runtime.cu:8-9). */
int mt_malloc(void** p, size_t bytes);
int mt_free(void* p);
/* kind: 0 host->host, 1 host->device, 2 device->host, 3 device->device,
 * 4 inferred. Replaces reference mt_copy (src/cuda_runtime.cu:10-12). */
int mt_copy(void* dst, const void* src, size_t bytes, int kind);
/* Asynchronous copy on the default stream. No reference counterpart. */
int mt_copy_async(void* dst, const void* src, size_t bytes, int kind);
/* Replaces reference mt_sync (src/cuda_runtime.cu:13). */
int mt_sync(void);
/* Replaces reference mt_error (src/cuda_runtime.cu:14). */
const char* mt_error(int code);
/* Events on the default stream; elapsed waits for the second event.
 * Replace reference mt_event_* (src/cuda_runtime.cu:15-21). */
int mt_event_create(void** e);
int mt_event_record(void* e);
int mt_event_elapsed(float* ms, void* a, void* b);
int mt_event_destroy(void* e);
/* Wait for an event. No reference counterpart. */
int mt_event_synchronize(void* e);
/* 0 when the work before the event's record has completed, 600
 * (hipErrorNotReady) while it is pending. No reference counterpart (the
 * sync-free decode loop polls token readbacks with it). */
int mt_event_query(void* e);
/* Number of visible devices. No reference counterpart. */
int mt_device_count(int* n);
/* Compute units of the current device (256 on MI355X); sizes the row
 * visiting order of the decode. No reference counterpart. */
int mt_compute_units(int* n);
/* BENCH-ONLY measuring kernel, not part of the runtime the reference binds
 * (its CudaRuntime table, minitorch/cuda_storage.py:29-45, never names it) and
 * not called by any product path: reads `count` chunks of chunk_bytes (multiple of 1 KiB,
 * addresses listed in the device array `chunks`, 16-byte aligned) with
 * `blocks` workgroups of 4 waves, each wave taking every (waves)-th chunk.
 * Used by bench.py --ceiling to time a decode step's exact K/V access pattern
 * without the decode's work. No reference counterpart. */
int mt_chunk_read(const unsigned long long* chunks, int count, int chunk_bytes, int blocks,
                  unsigned* sink);
/* Graph capture of the calling thread's default stream (where every entry of
 * these libraries launches): mt_graph_begin starts a thread-local capture;
 * mt_graph_end ends it and instantiates the graph (*exec; null and the
 * capture discarded on failure); mt_graph_launch replays it on the same
 * stream; mt_graph_destroy releases it. Used to replay a decode step whose
 * shapes are fixed. No reference counterpart. */
int mt_graph_begin(void);
int mt_graph_end(void** exec);
int mt_graph_launch(void* exec);
int mt_graph_destroy(void* exec);
/* Pinned host memory (hipHostMalloc) for asynchronous uploads.
 * No reference counterpart. */
int mt_host_alloc(void** p, size_t bytes);
int mt_host_free(void* p);
/* p[0:n] = v (fp32). Replaces reference mt_fill (src/cuda_runtime.cu:54-57). */
int mt_fill(float* p, int n, float v);
/* p[0:n] uniform in [0, 1), a deterministic function of (seed, index): the
 * SplitMix64 output function of seed * 0x9E3779B97F4A7C15 + index, top 24
 * bits. Same range and contract as the reference, not cuRAND's Philox stream.
 * Replaces reference mt_random (src/cuda_runtime.cu:37-44,58-61). */
int mt_random(float* p, int n, unsigned long long seed);
/* out[i] = 1 if i % classes == (int)ids[i / classes] else 0, i < size (the
 * id truncated toward zero; NaN reads as 0, out-of-range ids saturate).
 * Replaces reference mt_one_hot (src/cuda_runtime.cu:45-48,62-65). */
int mt_one_hot(float* out, const float* ids, int size, int classes);
/* width == 0: out[i] = i; else out[i] = -3.402823466e38 if
 * i % width > i / width, else 0 (causal mask rows).
 * Replaces reference mt_sequence (src/cuda_runtime.cu:49-52,66-69). */
int mt_sequence(float* out, int size, int width);
/* hipBLASLt handle and row-major fp32 GEMM out[m,n] = a[m,k] @ b[k,n],
 * forwarded to model_kernels.so (include/mt_model.h) found next to this
 * library, so one handle serves both; hipErrorSharedObjectInitFailed (303)
 * when that library is missing.
 * Replace reference mt_blas_create / mt_blas_destroy / mt_gemm
 * (src/cuda_runtime.cu:22-30). */
int mt_blas_create(void** handle);
int mt_blas_destroy(void* handle);
int mt_gemm(void* handle, float* out, const float* a, const float* b, int m, int n, int k);
/* Fill `words` 32-bit words with `value` by a kernel (graph-capturable,
 * unlike a memset node). No reference counterpart. */
int mt_fill_words(void* p, size_t words, unsigned int value);
/* n elements of dtype set to a deterministic hash of (seed, index), uniform
 * in [-2, 2): synthetic data for large pools. No reference counterpart
 * (stands in for reference mt_random, src/cuda_runtime.cu:37-44,58-61). */
int mt_fill_random(void* p, long long n, unsigned long long seed, int dtype);

#ifdef __cplusplus
}
#endif
#endif /* MT_RUNTIME_H */
