/* Device runtime of the boundary: C-ABI of
 * minitorch_amd/cuda_kernels/cuda_runtime.so. Device 0 (the current HIP
 * device), null stream. Status convention as in mt_paged.h.
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
/* Asynchronous copy on the null stream. No reference counterpart. */
int mt_copy_async(void* dst, const void* src, size_t bytes, int kind);
/* Replaces reference mt_sync (src/cuda_runtime.cu:13). */
int mt_sync(void);
/* Replaces reference mt_error (src/cuda_runtime.cu:14). */
const char* mt_error(int code);
/* Events on the null stream; elapsed waits for the second event.
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
/* Measuring kernel: reads `count` chunks of chunk_bytes (multiple of 1 KiB,
 * addresses listed in the device array `chunks`, 16-byte aligned) with
 * `blocks` workgroups of 4 waves, each wave taking every (waves)-th chunk.
 * Used by bench.py --ceiling to time a decode step's exact K/V access pattern
 * without the decode's work. No reference counterpart. */
int mt_chunk_read(const unsigned long long* chunks, int count, int chunk_bytes, int blocks,
                  unsigned* sink);
/* Pinned host memory (hipHostMalloc) for asynchronous uploads.
 * No reference counterpart. */
int mt_host_alloc(void** p, size_t bytes);
int mt_host_free(void* p);
/* p[0:n] = v (fp32). Replaces reference mt_fill (src/cuda_runtime.cu:54-57). */
int mt_fill(float* p, int n, float v);
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
