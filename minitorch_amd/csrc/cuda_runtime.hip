// Device runtime of the boundary: allocation, copies, synchronization, error
// strings and events on the calling thread's default stream of device 0 (the
// libraries are built with per-thread default streams, so that a decode step
// can be captured into a graph; with one host thread this orders work exactly
// as the reference's legacy null stream does), with the reference's symbol
// names and status convention (src/cuda_runtime.cu:7-21; status 0 = success,
// otherwise the hipError_t value, whose numbering matches the CUDA codes the
// reference's Python checks: 1 = invalid value, 2 = out of memory).
#include <hip/hip_runtime.h>
#include <dlfcn.h>
#include <climits>
#include <cstdint>
#include <mutex>
#include <string>

namespace {

__global__ __launch_bounds__(256) void fill_kernel(float* out, int64_t size, float value) {
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < size;
       i += int64_t(gridDim.x) * blockDim.x)
    out[i] = value;
}

__global__ __launch_bounds__(256) void fill_bytes_kernel(uint32_t* out, int64_t words, uint32_t value) {
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < words;
       i += int64_t(gridDim.x) * blockDim.x)
    out[i] = value;
}

// Counter-based hash (SplitMix64 finalizer) of (seed, i) mapped to [-2, 2).
__device__ __forceinline__ float hash_uniform(unsigned long long seed, unsigned long long i) {
  unsigned long long z = seed * 0x9E3779B97F4A7C15ull + i + 0x632BE59BD9B4E019ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  z ^= z >> 31;
  return float(z >> 40) * (4.0f / 16777216.0f) - 2.0f;
}

__global__ __launch_bounds__(256) void fill_random_kernel(void* out, int64_t n, unsigned long long seed, int dtype) {
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x) {
    const float v = hash_uniform(seed, (unsigned long long)i);
    if (dtype == 0) {
      static_cast<float*>(out)[i] = v;
    } else if (dtype == 1) {
      static_cast<_Float16*>(out)[i] = static_cast<_Float16>(v);
    } else {
      const unsigned u = __float_as_uint(v);
      static_cast<unsigned short*>(out)[i] = static_cast<unsigned short>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
    }
  }
}

// Uniform float in [0, 1) from (seed, index): the SplitMix64 output function
// (Steele, Lea and Flood, "Fast splittable pseudorandom number generators",
// OOPSLA 2014) applied to seed * golden-ratio increment + index, top 24 bits.
// This is this library's own stream; it is not cuRAND's Philox sequence.
__device__ __forceinline__ float unit_uniform(unsigned long long seed, unsigned long long i) {
  unsigned long long z = seed * 0x9E3779B97F4A7C15ull + i;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  z ^= z >> 31;
  return float(z >> 40) * (1.0f / 16777216.0f);
}

__global__ __launch_bounds__(256) void random_kernel(float* out, int64_t n, unsigned long long seed) {
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x)
    out[i] = unit_uniform(seed, (unsigned long long)i);
}

// float -> int as a truncating hardware conversion does it: NaN gives 0,
// values beyond the int range saturate.
__device__ __forceinline__ int to_int_saturating(float f) {
  if (isnan(f)) return 0;
  if (f >= 2147483648.0f) return INT_MAX;
  if (f <= -2147483648.0f) return INT_MIN;
  return int(f);
}

__global__ __launch_bounds__(256) void one_hot_kernel(float* out, const float* ids, int64_t size, int classes) {
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < size; i += int64_t(gridDim.x) * blockDim.x) {
    const int64_t row = i / classes;
    out[i] = int64_t(to_int_saturating(ids[row])) == i - row * classes ? 1.f : 0.f;
  }
}

__global__ __launch_bounds__(256) void sequence_kernel(float* out, int64_t size, int width) {
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < size; i += int64_t(gridDim.x) * blockDim.x) {
    if (width) out[i] = (i % width > i / width) ? -3.402823466e38f : 0.f;
    else out[i] = float(i);
  }
}

int blocks_for(int64_t n) {
  const int64_t b = (n + 255) / 256;
  return int(b < (1 << 20) ? b : (1 << 20));
}

// The hipBLASLt handle and GEMM live in model_kernels.so (built next to this
// library); the runtime's BLAS symbols forward to it, so a handle created
// through either library is valid for both.
void* blas_symbol(const char* name) {
  static std::once_flag once;
  static void* lib = nullptr;
  std::call_once(once, [] {
    Dl_info info{};
    if (!dladdr(reinterpret_cast<void*>(&blas_symbol), &info) || !info.dli_fname) return;
    std::string path(info.dli_fname);
    const size_t slash = path.rfind('/');
    path = (slash == std::string::npos ? std::string(".") : path.substr(0, slash)) + "/model_kernels.so";
    lib = dlopen(path.c_str(), RTLD_NOW | RTLD_LOCAL);
  });
  return lib ? dlsym(lib, name) : nullptr;
}

}  // namespace

extern "C" {

int mt_malloc(void** p, size_t bytes) { return hipMalloc(p, bytes); }
int mt_free(void* p) { return hipFree(p); }
// kind: 0 host->host, 1 host->device, 2 device->host, 3 device->device, 4 default.
int mt_copy(void* dst, const void* src, size_t bytes, int kind) {
  if (kind < 0 || kind > 4) return hipErrorInvalidValue;
  return hipMemcpy(dst, src, bytes, static_cast<hipMemcpyKind>(kind));
}
int mt_copy_async(void* dst, const void* src, size_t bytes, int kind) {
  if (kind < 0 || kind > 4) return hipErrorInvalidValue;
  return hipMemcpyAsync(dst, src, bytes, static_cast<hipMemcpyKind>(kind), nullptr);
}
int mt_sync() { return hipStreamSynchronize(nullptr); }
const char* mt_error(int code) { return hipGetErrorString(static_cast<hipError_t>(code)); }
int mt_event_create(hipEvent_t* e) { return hipEventCreate(e); }
int mt_event_record(hipEvent_t e) { return hipEventRecord(e, nullptr); }
int mt_event_elapsed(float* ms, hipEvent_t a, hipEvent_t b) {
  hipError_t e = hipEventSynchronize(b);
  return e == hipSuccess ? hipEventElapsedTime(ms, a, b) : e;
}
int mt_event_destroy(hipEvent_t e) { return hipEventDestroy(e); }
int mt_event_synchronize(hipEvent_t e) { return hipEventSynchronize(e); }
int mt_event_query(hipEvent_t e) { return hipEventQuery(e); }
int mt_device_count(int* n) { return hipGetDeviceCount(n); }
// Compute units of the current device.
int mt_compute_units(int* n) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  return hipDeviceGetAttribute(n, hipDeviceAttributeMultiprocessorCount, dev);
}
// Graph capture of the calling thread's default stream, where the libraries
// of this build launch everything (they are built with per-thread default
// streams; the legacy null stream cannot be captured). Thread-local mode:
// an allocation or synchronization issued by this thread inside the capture
// fails instead of being recorded.
int mt_graph_begin() { return hipStreamBeginCapture(hipStreamPerThread, hipStreamCaptureModeThreadLocal); }

// Ends the capture begun by mt_graph_begin and instantiates it; on any
// failure the capture is still ended (and discarded) and *exec is null.
int mt_graph_end(void** exec) {
  if (!exec) return hipErrorInvalidValue;
  *exec = nullptr;
  hipGraph_t graph = nullptr;
  hipError_t e = hipStreamEndCapture(hipStreamPerThread, &graph);
  if (e != hipSuccess) {
    if (graph) hipGraphDestroy(graph);
    return e;
  }
  hipGraphExec_t x = nullptr;
  e = hipGraphInstantiate(&x, graph, nullptr, nullptr, 0);
  hipGraphDestroy(graph);
  if (e != hipSuccess) return e;
  *exec = x;
  return hipSuccess;
}

int mt_graph_launch(void* exec) {
  if (!exec) return hipErrorInvalidValue;
  return hipGraphLaunch(static_cast<hipGraphExec_t>(exec), hipStreamPerThread);
}

int mt_graph_destroy(void* exec) {
  if (!exec) return hipErrorInvalidValue;
  return hipGraphExecDestroy(static_cast<hipGraphExec_t>(exec));
}

// Pinned host memory for asynchronous uploads (allocated, never registered).
int mt_host_alloc(void** p, size_t bytes) { return hipHostMalloc(p, bytes, hipHostMallocDefault); }
int mt_host_free(void* p) { return hipHostFree(p); }

// out[0:n] = value (reference mt_fill, src/cuda_runtime.cu:33-35,54-57).
int mt_fill(float* p, int n, float v) {
  if (n < 0) return hipErrorInvalidValue;
  if (n) fill_kernel<<<blocks_for(n), 256>>>(p, n, v);
  return hipGetLastError();
}

// out[0:n] uniform in [0, 1) from `seed` (reference mt_random,
// src/cuda_runtime.cu:37-44,58-61). Deterministic per (seed, index); the
// stream is this library's own, not cuRAND's.
int mt_random(float* p, int n, unsigned long long seed) {
  if (n < 0 || (!p && n)) return hipErrorInvalidValue;
  if (n) random_kernel<<<blocks_for(n), 256>>>(p, n, seed);
  return hipGetLastError();
}

// out[i] = 1 where i % classes == int(ids[i / classes]), else 0, for `size`
// outputs (reference mt_one_hot, src/cuda_runtime.cu:45-48,62-65).
int mt_one_hot(float* out, const float* ids, int size, int classes) {
  if (size < 0 || (size && (!out || !ids || classes < 1))) return hipErrorInvalidValue;
  if (size) one_hot_kernel<<<blocks_for(size), 256>>>(out, ids, size, classes);
  return hipGetLastError();
}

// width == 0: out[i] = i; else the causal mask of rows of `width`:
// -3.402823466e38 where i % width > i / width, else 0 (reference
// mt_sequence, src/cuda_runtime.cu:49-52,66-69).
int mt_sequence(float* out, int size, int width) {
  if (size < 0 || width < 0 || (!out && size)) return hipErrorInvalidValue;
  if (size) sequence_kernel<<<blocks_for(size), 256>>>(out, size, width);
  return hipGetLastError();
}

// Replace reference mt_blas_create / mt_blas_destroy / mt_gemm
// (src/cuda_runtime.cu:22-30): forwarded to model_kernels.so's hipBLASLt
// implementation. hipErrorSharedObjectInitFailed if that library is absent.
int mt_blas_create(void** handle) {
  auto f = reinterpret_cast<int (*)(void**)>(blas_symbol("mt_blas_create"));
  return f ? f(handle) : hipErrorSharedObjectInitFailed;
}

int mt_blas_destroy(void* handle) {
  auto f = reinterpret_cast<int (*)(void*)>(blas_symbol("mt_blas_destroy"));
  return f ? f(handle) : hipErrorSharedObjectInitFailed;
}

int mt_gemm(void* handle, float* out, const float* a, const float* b, int m, int n, int k) {
  auto f = reinterpret_cast<int (*)(void*, float*, const float*, const float*, int, int, int)>(
      blas_symbol("mt_gemm"));
  return f ? f(handle, out, a, b, m, n, k) : hipErrorSharedObjectInitFailed;
}

// Fill `words` 32-bit words with a bit pattern: a small kernel rather than a
// memset node, so callers may capture it in a graph.
int mt_fill_words(void* p, size_t words, unsigned int value) {
  if (!p && words) return hipErrorInvalidValue;
  if (words) fill_bytes_kernel<<<blocks_for(int64_t(words)), 256>>>(static_cast<uint32_t*>(p), int64_t(words), value);
  return hipGetLastError();
}

// n elements of dtype (0 fp32, 1 fp16, 2 bf16) set to a deterministic
// hash of (seed, index), uniform in [-2, 2): synthetic K/V for large pools.
// Reads `count` chunks of `chunk_bytes` (a multiple of 1 KiB) whose addresses
// are listed in `chunks`, each wave taking chunks wave, wave + waves, ...,
// with non-temporal 16-byte loads (as the decode kernel reads K/V), and XORs
// what it read into sink[0] only if the XOR equals a sentinel (so the loads
// cannot be dropped and nothing is written in practice). A measuring kernel:
// the bandwidth of exactly the K/V access pattern of a decode step, with no
// address arithmetic, math or merging.
__global__ __launch_bounds__(256) void chunk_read_kernel(const unsigned long long* chunks, int count,
                                                          int vec_per_chunk, unsigned* sink) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const int lane = threadIdx.x & 63;
  const int wave = (blockIdx.x * int(blockDim.x) + int(threadIdx.x)) >> 6;
  const int waves = int(gridDim.x * blockDim.x) >> 6;
  unsigned acc = 0;
  for (int c = wave; c < count; c += waves) {
    const auto* p = reinterpret_cast<const __attribute__((address_space(1))) u32x4*>(chunks[c]);
    for (int v = lane; v < vec_per_chunk; v += 64) {
      const u32x4 x = __builtin_nontemporal_load(p + v);  // as the decode kernel loads K/V
      acc ^= x.x ^ x.y ^ x.z ^ x.w;
    }
  }
  if (acc == 0x9e3779b9u) sink[0] = acc;
}

int mt_chunk_read(const unsigned long long* chunks, int count, int chunk_bytes, int blocks,
                  unsigned* sink) {
  if (!chunks || !sink || count < 1 || chunk_bytes < 1024 || chunk_bytes % 1024 || blocks < 1)
    return hipErrorInvalidValue;
  chunk_read_kernel<<<blocks, 256>>>(chunks, count, chunk_bytes / 16, sink);
  return hipGetLastError();
}

int mt_fill_random(void* p, long long n, unsigned long long seed, int dtype) {
  if ((!p && n) || n < 0 || dtype < 0 || dtype > 2) return hipErrorInvalidValue;
  if (n) fill_random_kernel<<<blocks_for(n), 256>>>(p, n, seed, dtype);
  return hipGetLastError();
}

}  // extern "C"
