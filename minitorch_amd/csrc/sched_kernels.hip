// Device-side page allocator and decode-step metadata for gfx950.
//
// The reference keeps the page free list, per-cache page lists, block tables
// and decode offsets on the host and uploads them every step
// (minitorch/paged_kv_cache.py:71-103,171-189; minitorch/paged_decode.py:40-54).
// Here they live in one device "pool state" blob and are updated by small
// single-workgroup kernels on the default stream, so admitting, stepping and
// finishing requests never reads device memory back. Page IDs follow the
// reference's host allocator exactly:
//   * the free list is a LIFO stack; pops take the top;
//   * when a pop of `count` pages finds fewer than `count` free pages, whole
//     new slabs are opened first and their IDs pushed in reverse order on top
//     of the older free pages, then all `count` pages are popped
//     (paged_kv_cache.py:78-89) -- "bulk" pops, used by prepare_append(n);
//   * a decode step acquires one page per row that needs it, row by row, each
//     as its own pop of one page (paged_decode.py:44-46 calling
//     paged_kv_cache.py:171-186) -- "sequential" pops;
//   * releases push pages in the given order (paged_kv_cache.py:96-103).
// The state blob layout is computed by pool_layout() and exported through
// mt_pool_layout() so the host can address the slab table and slot rows.
#include "mt_device.h"
#include <climits>

namespace {

constexpr int kThreads = 1024;
constexpr int kPrepareRows = 2048;  // rows of a decode step whose slot and page count stay in LDS
constexpr int kTableUnroll = 8;     // block-table entries each thread loads before storing
// Block-table entries each thread of decode_prepare_kernel holds in registers
// when the whole table of a step fits (b * columns <= kThreads * kEarlyTable).
constexpr int kEarlyTable = 16;

struct Header {           // must match include/mt_sched.h (mt_pool_header)
  int top;                // free pages on the stack
  int slabs_opened;
  int leased;
  int error;              // nonzero after an invalid release
  long long acquires, releases, reuses;
};

struct Layout {
  size_t header, stack, issued, owner, slab_table, slot_len, slot_npages, slot_pages, total;
};

size_t align256(size_t x) { return (x + 255) / 256 * 256; }

Layout pool_layout(int max_pages, int max_slabs, int max_slots, int max_cols) {
  Layout l{};
  size_t o = 0;
  l.header = o; o = align256(o + sizeof(Header));
  l.stack = o; o = align256(o + size_t(max_pages) * 4);
  l.issued = o; o = align256(o + size_t((max_pages + 31) / 32) * 4);
  l.owner = o; o = align256(o + size_t(max_pages) * 4);
  l.slab_table = o; o = align256(o + size_t(max_slabs) * 8);
  l.slot_len = o; o = align256(o + size_t(max_slots) * 4);
  l.slot_npages = o; o = align256(o + size_t(max_slots) * 4);
  l.slot_pages = o; o = align256(o + size_t(max_slots) * max_cols * 4);
  l.total = o;
  return l;
}

struct Pool {
  Header* h;
  int* stack;
  unsigned* issued;
  int* owner;
  unsigned long long* slab_table;
  int* slot_len;
  int* slot_npages;
  int* slot_pages;
  int max_pages, max_slabs, max_slots, max_cols, pages_per_slab;
  unsigned long long pool_base, slab_bytes;
};

Pool make_pool(void* state, int max_pages, int max_slabs, int max_slots, int max_cols, int pps,
               unsigned long long pool_base, unsigned long long slab_bytes) {
  const Layout l = pool_layout(max_pages, max_slabs, max_slots, max_cols);
  char* s = static_cast<char*>(state);
  Pool p{};
  p.h = reinterpret_cast<Header*>(s + l.header);
  p.stack = reinterpret_cast<int*>(s + l.stack);
  p.issued = reinterpret_cast<unsigned*>(s + l.issued);
  p.owner = reinterpret_cast<int*>(s + l.owner);
  p.slab_table = reinterpret_cast<unsigned long long*>(s + l.slab_table);
  p.slot_len = reinterpret_cast<int*>(s + l.slot_len);
  p.slot_npages = reinterpret_cast<int*>(s + l.slot_npages);
  p.slot_pages = reinterpret_cast<int*>(s + l.slot_pages);
  p.max_pages = max_pages; p.max_slabs = max_slabs; p.max_slots = max_slots;
  p.max_cols = max_cols; p.pages_per_slab = pps; p.pool_base = pool_base; p.slab_bytes = slab_bytes;
  return p;
}

// Record the pop of page `page` for `owner`; returns 1 if it was issued before.
__device__ __forceinline__ int mark_issued(const Pool& p, int page, int owner) {
  p.owner[page] = owner;
  const unsigned bit = 1u << (page & 31);
  return (atomicOr(&p.issued[page >> 5], bit) & bit) ? 1 : 0;
}

__device__ __forceinline__ void open_slabs(const Pool& p, int first, int count) {
  for (int s = threadIdx.x; s < count; s += kThreads)
    p.slab_table[first + s] = p.pool_base + (unsigned long long)(first + s) * p.slab_bytes;
}

// Workgroup-wide exclusive prefix sums of N ints per thread, in thread order
// (workgroups of kThreads threads, all of them calling): DPP wave scans, then
// every thread adds the totals of the waves before its own. sh: N * 16 ints.
template <int N>
__device__ __forceinline__ void block_scan(int (&x)[N], int (&total)[N], int* sh) {
  constexpr int W = kThreads / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int incl[N];
#pragma unroll
  for (int j = 0; j < N; ++j) incl[j] = mt::wave_inclusive_add(x[j]);
  if (lane == 63) {
#pragma unroll
    for (int j = 0; j < N; ++j) sh[j * W + wave] = incl[j];
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < N; ++j) {
    int before = 0, all = 0;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const int v = sh[j * W + w];
      before += w < wave ? v : 0;
      all += v;
    }
    x[j] = before + incl[j] - x[j];
    total[j] = all;
  }
  __syncthreads();
}

__device__ __forceinline__ int block_exclusive_scan(int x, int* total, int* sh) {
  int v[1] = {x}, t[1];
  block_scan<1>(v, t, sh);
  *total = t[0];
  return v[0];
}

// Bulk pop of `count` pages (one reference acquire(count)): opens slabs first
// when the stack is short, then pops. out[r] is the r-th popped page.
__device__ void bulk_pop(const Pool& p, int count, int owner, int* out, int* s_red) {
  const int F = p.h->top, opened = p.h->slabs_opened, pps = p.pages_per_slab;
  const int nslab = count > F ? (count - F + pps - 1) / pps : 0;
  const int T = F + nslab * pps;
  int reused = 0;
  for (int r = threadIdx.x; r < count; r += blockDim.x) {
    const int idx = T - 1 - r;
    int page;
    if (idx >= F) {
      const int j = (idx - F) / pps, i = (idx - F) % pps;
      page = (opened + j) * pps + (pps - 1 - i);
    } else {
      page = p.stack[idx];
    }
    out[r] = page;
    reused += mark_issued(p, page, owner);
  }
  __syncthreads();  // all reads of old stack entries are done
  // Materialize the unpopped entries of the new slabs.
  for (int idx = F + threadIdx.x; idx < T - count; idx += blockDim.x) {
    const int j = (idx - F) / pps, i = (idx - F) % pps;
    p.stack[idx] = (opened + j) * pps + (pps - 1 - i);
  }
  open_slabs(p, opened, nslab);
  atomicAdd(s_red, reused);
  __syncthreads();
  if (threadIdx.x == 0) {
    p.h->top = T - count;
    p.h->slabs_opened = opened + nslab;
    p.h->leased += count;
    p.h->acquires += count;
    p.h->reuses += *s_red;
    *s_red = 0;
  }
  __syncthreads();
}

// Push pages[0..n) (in order) on the free stack.
__device__ void push_pages(const Pool& p, const int* pages, int n, int expect_owner, bool check) {
  const int top = p.h->top;
  int bad = 0;
  for (int r = threadIdx.x; r < n; r += blockDim.x) {
    const int page = pages[r];
    if (check && (page < 0 || page >= p.max_pages || p.owner[page] != expect_owner)) { bad = 1; continue; }
    p.stack[top + r] = page;
    p.owner[page] = -1;
  }
  if (bad) atomicOr(&p.h->error, 1);
  __syncthreads();
  if (threadIdx.x == 0) {
    p.h->top = top + n;
    p.h->leased -= n;
    p.h->releases += n;
  }
  __syncthreads();
}

__global__ __launch_bounds__(kThreads) void init_kernel(Pool p) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    p.h->top = 0; p.h->slabs_opened = 0; p.h->leased = 0; p.h->error = 0;
    p.h->acquires = 0; p.h->releases = 0; p.h->reuses = 0;
  }
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  const int64_t t0 = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  for (int64_t i = t0; i < (p.max_pages + 31) / 32; i += stride) p.issued[i] = 0;
  for (int64_t i = t0; i < p.max_pages; i += stride) p.owner[i] = -1;
  for (int64_t i = t0; i < p.max_slabs; i += stride) p.slab_table[i] = 0;
  for (int64_t i = t0; i < p.max_slots; i += stride) { p.slot_len[i] = 0; p.slot_npages[i] = 0; }
  for (int64_t i = t0; i < int64_t(p.max_slots) * p.max_cols; i += stride) p.slot_pages[i] = -1;
}

// Reference acquire(count, owner) returning the pages (API path).
__global__ __launch_bounds__(kThreads) void pop_kernel(Pool p, int count, int owner, int* out) {
  __shared__ int s_red;
  if (threadIdx.x == 0) s_red = 0;
  __syncthreads();
  bulk_pop(p, count, owner, out, &s_red);
}

// Reference release(pages, owner) (API path); invalid ownership sets error.
__global__ __launch_bounds__(kThreads) void push_kernel(Pool p, const int* pages, int n, int owner) {
  push_pages(p, pages, n, owner, true);
}

// prepare_append(tokens) of a cache whose rows are slots[0..rows): one bulk
// pop of rows * per_row pages, distributed row by row.
__global__ __launch_bounds__(kThreads) void acquire_rows_kernel(Pool p, const int* slots, int rows,
                                                                int per_row, int* scratch) {
  __shared__ int s_red;
  if (threadIdx.x == 0) s_red = 0;
  __syncthreads();
  const int count = rows * per_row;
  // owner of a cache's pages is its first slot
  bulk_pop(p, count, slots[0], scratch, &s_red);
  for (int r = threadIdx.x; r < count; r += blockDim.x) {
    const int row = r / per_row, j = r - row * per_row;
    const int slot = slots[row];
    p.slot_pages[int64_t(slot) * p.max_cols + p.slot_npages[slot] + j] = scratch[r];
  }
  __syncthreads();
  for (int row = threadIdx.x; row < rows; row += blockDim.x) p.slot_npages[slots[row]] += per_row;
}

// prepare_append of n one-row caches in order, as n acquire_rows_kernel
// launches of one row would run: for i = 0..n-1 one bulk pop of counts[i]
// pages (owner slots[i]) appended to slot i's page list.
__global__ __launch_bounds__(kThreads) void acquire_lists_kernel(Pool p, const int* slots, const int* counts, int n,
                                                                 int* scratch) {
  __shared__ int s_red;
  if (threadIdx.x == 0) s_red = 0;
  __syncthreads();
  for (int i = 0; i < n; ++i) {
    const int slot = slots[i], count = counts[i];
    if (count <= 0) continue;
    // The counts come from device memory: an entry that names no slot, would
    // write past its slot's columns or pop beyond the budget is skipped and
    // flagged (every thread reads the same header and page count after the
    // previous entry's barrier, so all skip together).
    if (slot < 0 || slot >= p.max_slots || count > p.max_cols - p.slot_npages[slot] ||
        count > p.max_pages - p.h->leased) {
      if (threadIdx.x == 0) atomicOr(&p.h->error, 2);
      continue;
    }
    bulk_pop(p, count, slot, scratch, &s_red);
    const int have = p.slot_npages[slot];
    for (int r = threadIdx.x; r < count; r += blockDim.x)
      p.slot_pages[int64_t(slot) * p.max_cols + have + r] = scratch[r];
    __syncthreads();  // every thread has read `have` and its scratch entries
    if (threadIdx.x == 0) p.slot_npages[slot] = have + count;
    __syncthreads();
  }
}

// Release the pages [keep:] of each row slots[0..rows), row by row, in page
// order (close: keep = 0; abort of an append: keep = the count before it).
__global__ __launch_bounds__(kThreads) void release_rows_kernel(Pool p, const int* slots, int rows,
                                                                int keep, int reset_length) {
  __shared__ int sh[33];
  int top = p.h->top;
  int released = 0;
  for (int base = 0; base < rows; base += blockDim.x) {
    const int row = base + threadIdx.x;
    const int slot = row < rows ? slots[row] : 0;
    const int n = row < rows ? max(p.slot_npages[slot] - keep, 0) : 0;
    int total;
    const int at = block_exclusive_scan(n, &total, sh);
    for (int j = 0; j < n; ++j) {
      const int page = p.slot_pages[int64_t(slot) * p.max_cols + keep + j];
      p.stack[top + at + j] = page;
      p.owner[page] = -1;
      p.slot_pages[int64_t(slot) * p.max_cols + keep + j] = -1;
    }
    if (row < rows) {
      if (n) p.slot_npages[slot] = keep;
      if (reset_length) p.slot_len[slot] = 0;
    }
    top += total;
    released += total;
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    p.h->top = top;
    p.h->leased -= released;
    p.h->releases += released;
  }
}

// Decode-step metadata for a batch of slots (one token per row):
//   offsets[i] = committed length, positions[i] = float(offsets[i]),
//   cu_seqlens = exclusive prefix sum of offsets[i] + 1,
//   rows whose next token starts a new page pop one page each, row by row
//   (sequential pops, limited to `limit` pops), new_page[i] = popped page or -1,
//   table[i, :columns] = the row's pages, -1 beyond them.
__device__ __forceinline__ void decode_prepare_body(Pool p, const int* slots, int b, int columns,
                                                    int page_size, int limit, int* table, int* offsets,
                                                    float* positions, int* cu_seqlens, int* new_page) {
  constexpr int TOPS = kPrepareRows / kThreads;  // stack-top candidates per thread
  // Every argument is loaded at entry and kept in scalar registers; global
  // memory is reached through global-address-space pointers only.
  const auto h = mt::pin_global(p.h);
  const auto stack = mt::pin_global(p.stack);
  const auto issued = mt::pin_global(p.issued);
  const auto owner = mt::pin_global(p.owner);
  const auto slab_table = mt::pin_global(p.slab_table);
  const auto slot_len = mt::pin_global(p.slot_len);
  const auto slot_npages = mt::pin_global(p.slot_npages);
  const auto slot_pages = mt::pin_global(p.slot_pages);
  const auto g_slots = mt::pin_global(slots);
  const auto g_table = mt::pin_global(table);
  const auto g_offsets = mt::pin_global(offsets);
  const auto g_positions = mt::pin_global(positions);
  const auto g_cu = mt::pin_global(cu_seqlens);
  const auto g_new = mt::pin_global(new_page);
  const int max_pages = mt::pin_arg(p.max_pages), max_cols = mt::pin_arg(p.max_cols);
  const unsigned long long pool_base = mt::pin_arg(p.pool_base), slab_bytes = mt::pin_arg(p.slab_bytes);
  b = mt::pin_arg(b); columns = mt::pin_arg(columns);
  page_size = mt::pin_arg(page_size); limit = mt::pin_arg(limit);
  __shared__ int sh[2 * (kThreads / 64)];
  __shared__ int s_red;
  // Each row's slot, page count before this step and popped page (-1: none),
  // kept for the table (rows past kPrepareRows read them from the pool
  // state); s_top[k]: the k-th page from the top of the free stack, and
  // s_topbit[k] its issued bit (a pop of it is a reuse).
  __shared__ int s_slot[kPrepareRows], s_have[kPrepareRows], s_new[kPrepareRows], s_top[kPrepareRows];
  __shared__ unsigned char s_topbit[kPrepareRows];
  const int tid = threadIdx.x;
  if (tid == 0) s_red = 0;
  const int F = h->top, opened = h->slabs_opened, pps = mt::pin_arg(p.pages_per_slab);
  // limit -1: the pages the budget has left, read from the pool header on
  // the device (so that a captured step needs no host-computed budget).
  if (limit < 0) limit = max_pages - h->leased;
  // Every load is issued from straight-line code at clamped (always valid)
  // addresses, so the compiler counts them exactly and a wait covers only
  // the loads it needs, and every load is consumed before the first global
  // store (gfx9 counts stores and loads together, so a load consumed after
  // stores would wait for their acknowledgements). The chain:
  //   1. the slots of this thread's row and of its table entries;
  //   2. the row's length and page count, every table entry's current
  //      page-list value (when the whole table fits the threads' registers;
  //      this step changes only the entry at each popping row's old page
  //      count) and the top of the free stack;
  //   3. the issued bits of those stack pages (a page from a slab opened now
  //      was never issued), in flight while the ranks are scanned.
  const int64_t entries = int64_t(b) * columns;
  const bool early = entries <= int64_t(kThreads) * kEarlyTable && b <= kPrepareRows;
  const float inv_columns = 1.0f / float(columns);
  auto entry_row = [&](int e) {  // e / columns for e < 2^24 (one correction step)
    int i = int(float(e) * inv_columns);
    i -= i * columns > e;
    i += (i + 1) * columns <= e;
    return i;
  };
  const int last_entry = int(min(entries, int64_t(kThreads) * kEarlyTable)) - 1;
  const int slot0 = g_slots[min(tid, b - 1)];
  int tslot[kEarlyTable], tcol[kEarlyTable], tv[kEarlyTable];
  if (early) {
#pragma unroll
    for (int u = 0; u < kEarlyTable; ++u) {
      const int e = min(tid + u * kThreads, last_entry);
      const int i = entry_row(e);
      tcol[u] = e - i * columns;
      tslot[u] = g_slots[i];
    }
  }
  const int len0 = slot_len[slot0];
  const int have0 = slot_npages[slot0];
  if (early) {
#pragma unroll
    for (int u = 0; u < kEarlyTable; ++u) tv[u] = slot_pages[int64_t(tslot[u]) * max_cols + tcol[u]];
  }
  const int top_n = min(min(b, F), kPrepareRows);
  int sv[TOPS];
#pragma unroll
  for (int j = 0; j < TOPS; ++j) {
    const int k = min(j * kThreads + tid, max(top_n - 1, 0));
    sv[j] = stack[top_n > 0 ? F - 1 - k : 0];
  }
  unsigned bw[TOPS];
#pragma unroll
  for (int j = 0; j < TOPS; ++j) {
    sv[j] = min(max(sv[j], 0), max_pages - 1);  // in the pool whatever the stack holds
    bw[j] = issued[sv[j] >> 5];
    if (j * kThreads + tid < top_n) s_top[j * kThreads + tid] = sv[j];
  }
  __syncthreads();
  int need_base = 0, seq_base = 0, reused = 0;
  int rank0 = 0, seq0 = 0, need0 = 0;
  auto scan_pass = [&](int base, int len, int have, int& rank, int& seq, int& need) {
    const bool in = base + tid < b;
    need = (in && (len + page_size) / page_size > have) ? 1 : 0;
    int x[2] = {need, in ? len + 1 : 0}, tot[2];
    block_scan<2>(x, tot, sh);
    rank = need_base + x[0];
    seq = seq_base + x[1];
    need_base += tot[0];
    seq_base += tot[1];
  };
  // Pops of one pass of kThreads rows (every load already consumed).
  auto pop_pass = [&](int base, int slot, int len, int have, int rank, int seq, int need) {
    const int i = base + tid;
    const bool in = i < b;
    const bool pop = need && rank < limit;
    int page = -1;
    if (pop) {
      if (rank < F) {
        if (rank < top_n) {
          page = s_top[rank];
          reused += s_topbit[rank];
        } else {  // past the candidates kept in LDS (batches above kPrepareRows rows)
          page = stack[F - 1 - rank];
          reused += (issued[page >> 5] >> (page & 31)) & 1;
        }
      } else {
        const int k = rank - F;
        page = (opened + k / pps) * pps + k % pps;
      }
      owner[page] = slot;
      __hip_atomic_fetch_or(&issued[page >> 5], 1u << (page & 31), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      slot_pages[int64_t(slot) * max_cols + have] = page;
      slot_npages[slot] = have + 1;
    }
    if (in) {
      g_offsets[i] = len;
      g_positions[i] = float(len);
      g_cu[i] = seq;
      g_new[i] = page;
      if (i < kPrepareRows) {
        s_slot[i] = slot;
        s_have[i] = have;
        s_new[i] = page;
      }
    }
  };
  scan_pass(0, len0, have0, rank0, seq0, need0);
#pragma unroll
  for (int j = 0; j < TOPS; ++j)
    if (j * kThreads + tid < top_n) s_topbit[j * kThreads + tid] = (bw[j] >> (sv[j] & 31)) & 1;
  __syncthreads();
  pop_pass(0, slot0, len0, have0, rank0, seq0, need0);
  for (int base = kThreads; base < b; base += kThreads) {
    const int slot = g_slots[min(base + tid, b - 1)];
    const int len = slot_len[slot], have = slot_npages[slot];
    int rank, seq, need;
    scan_pass(base, len, have, rank, seq, need);
    pop_pass(base, slot, len, have, rank, seq, need);
  }
  if (tid == 0) g_cu[b] = seq_base;
  const int pops = need_base < limit ? need_base : limit;
  // Leftover pages of the last slab opened by the sequential pops stay on the
  // stack, reversed (its unused IDs with the smallest unused on top).
  int nslab = 0, top = F - pops;
  if (pops > F) {
    const int m = pops - F;
    nslab = (m + pps - 1) / pps;
    const int used_last = m - (nslab - 1) * pps;
    const int last = opened + nslab - 1;
    top = pps - used_last;
    for (int j = tid; j < top; j += kThreads) stack[j] = last * pps + pps - 1 - j;
  }
  for (int s = tid; s < nslab; s += kThreads)
    slab_table[opened + s] = pool_base + (unsigned long long)(opened + s) * slab_bytes;
  atomicAdd(&s_red, reused);
  __syncthreads();
  if (early) {
    // entry (i, c): the old page list below the row's old count, the popped
    // page at it, -1 beyond
#pragma unroll
    for (int u = 0; u < kEarlyTable; ++u) {
      const int e = tid + u * kThreads;
      if (e < entries) {
        const int i = entry_row(e), c = tcol[u];
        const int have = s_have[i];
        g_table[e] = c < have ? tv[u] : (c == have ? s_new[i] : -1);
      }
    }
  } else {
    // Table rows: kTableUnroll entries per thread are loaded before any is
    // stored, so their page-list reads overlap instead of taking one round
    // trip each.
    for (int64_t e0 = tid; e0 < entries; e0 += int64_t(kThreads) * kTableUnroll) {
      int v[kTableUnroll];
#pragma unroll
      for (int u = 0; u < kTableUnroll; ++u) {
        const int64_t e = e0 + int64_t(u) * kThreads;
        v[u] = -1;
        if (e < entries) {
          const int i = int(e / columns), c = int(e - int64_t(i) * columns);
          const int slot = i < kPrepareRows ? s_slot[i] : g_slots[i];
          const int np = i < kPrepareRows ? s_have[i] + (s_new[i] >= 0) : slot_npages[slot];
          if (c < np) v[u] = slot_pages[int64_t(slot) * max_cols + c];
        }
      }
#pragma unroll
      for (int u = 0; u < kTableUnroll; ++u) {
        const int64_t e = e0 + int64_t(u) * kThreads;
        if (e < entries) g_table[e] = v[u];
      }
    }
  }
  if (tid == 0) {
    h->top = top;
    h->slabs_opened = opened + nslab;
    h->leased += pops;
    h->acquires += pops;
    h->reuses += s_red;
  }
}

__global__ __launch_bounds__(kThreads) void decode_prepare_kernel(Pool p, const int* slots, int b,
                                                                  int columns, int page_size,
                                                                  int limit, int* table,
                                                                  int* offsets, float* positions,
                                                                  int* cu_seqlens, int* new_page) {
  decode_prepare_body(p, slots, b, columns, page_size, limit, table, offsets, positions, cu_seqlens,
                      new_page);
}

// The embeddings of a decode step's tokens, x[i, :] = wte[id_i, :] +
// wpe[pos_i, :] (fp32), with id_i the slot's last token and pos_i its
// committed length: the rule of the inference library's embed_tokens_kernel
// (an id or position that is non-finite, negative, too large or not integral,
// or a slot outside the table, gives a NaN row).
struct EmbedArgs {
  float* x;
  const float* wte;
  const float* wpe;
  const float* slot_tokens;
  int num_slots, vocab, n_positions, dim;
};

__device__ __forceinline__ bool bad_index(float raw, int limit) {
  return !isfinite(raw) || raw < 0.f || raw >= float(limit) || raw != floorf(raw);
}

// decode_prepare_kernel and the step's embeddings in one launch: workgroup 0
// builds the metadata; the others embed the rows. The embedding reads each
// slot's committed length itself (the position prepare writes), so the two
// parts do not wait for each other.
__global__ __launch_bounds__(kThreads) void decode_prepare_embed_kernel(Pool p, const int* slots, int b,
                                                                        int columns, int page_size,
                                                                        int limit, int* table,
                                                                        int* offsets, float* positions,
                                                                        int* cu_seqlens, int* new_page,
                                                                        EmbedArgs e) {
  if (blockIdx.x == 0) {
    decode_prepare_body(p, slots, b, columns, page_size, limit, table, offsets, positions, cu_seqlens,
                        new_page);
    return;
  }
  const int per_row = e.dim / 4;
  const int total = b * per_row;
  for (int i = (blockIdx.x - 1) * kThreads + threadIdx.x; i < total; i += (gridDim.x - 1) * kThreads) {
    const int t = i / per_row;
    const int col = (i - t * per_row) * 4;
    const int s = slots[t];
    const bool in = s >= 0 && s < e.num_slots;
    const float id = in ? e.slot_tokens[s] : NAN;
    const float pos = in ? float(p.slot_len[s]) : NAN;
    float4 v = make_float4(NAN, NAN, NAN, NAN);
    if (!bad_index(id, e.vocab) && !bad_index(pos, e.n_positions)) {
      const float4 a = *reinterpret_cast<const float4*>(e.wte + int64_t(id) * e.dim + col);
      const float4 w = *reinterpret_cast<const float4*>(e.wpe + int64_t(pos) * e.dim + col);
      v = make_float4(a.x + w.x, a.y + w.y, a.z + w.z, a.w + w.w);
    }
    *reinterpret_cast<float4*>(e.x + int64_t(t) * e.dim + col) = v;
  }
}

// Commit: lengths += tokens for every row.
__global__ __launch_bounds__(kThreads) void add_length_kernel(Pool p, const int* slots, int b, int tokens) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < b; i += gridDim.x * blockDim.x)
    p.slot_len[slots[i]] += tokens;
}

// Commit of n one-row caches: lengths[slots[i]] += tokens[i].
__global__ __launch_bounds__(kThreads) void add_lengths_kernel(Pool p, const int* slots, const int* tokens, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
    p.slot_len[slots[i]] += tokens[i];
}

// Abort of a decode step: push back the pages popped by decode_prepare_kernel,
// in row order (the reference aborts every prepared cache in batch order).
__global__ __launch_bounds__(kThreads) void decode_abort_kernel(Pool p, const int* slots, int b,
                                                                const int* new_page) {
  __shared__ int sh[33];
  int top = p.h->top, released = 0;
  for (int base = 0; base < b; base += blockDim.x) {
    const int i = base + threadIdx.x;
    const int page = i < b ? new_page[i] : -1;
    int total;
    const int at = block_exclusive_scan(page >= 0 ? 1 : 0, &total, sh);
    if (page >= 0) {
      const int slot = slots[i];
      p.stack[top + at] = page;
      p.owner[page] = -1;
      p.slot_npages[slot] -= 1;
      p.slot_pages[int64_t(slot) * p.max_cols + p.slot_npages[slot]] = -1;
    }
    top += total;
    released += total;
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    p.h->top = top;
    p.h->leased -= released;
    p.h->releases += released;
  }
}

bool valid_geometry(int max_pages, int max_slabs, int max_slots, int max_cols, int pps) {
  return max_pages > 0 && max_slabs > 0 && max_slots > 0 && max_cols > 0 && pps > 0 &&
         int64_t(max_slabs) * pps == max_pages && int64_t(max_slots) * max_cols <= INT32_MAX;
}

}  // namespace

#define MT_POOL_ARGS                                                                          \
  void *state, int max_pages, int max_slabs, int max_slots, int max_cols, int pages_per_slab, \
      unsigned long long pool_base, unsigned long long slab_bytes
#define MT_POOL make_pool(state, max_pages, max_slabs, max_slots, max_cols, pages_per_slab, pool_base, slab_bytes)
#define MT_POOL_CHECK                                                                   \
  if (!state || !valid_geometry(max_pages, max_slabs, max_slots, max_cols, pages_per_slab)) \
    return hipErrorInvalidValue;

extern "C" {

int mt_pool_layout(int max_pages, int max_slabs, int max_slots, int max_cols, size_t* offsets) {
  if (!offsets || max_pages < 1 || max_slabs < 1 || max_slots < 1 || max_cols < 1)
    return hipErrorInvalidValue;
  const Layout l = pool_layout(max_pages, max_slabs, max_slots, max_cols);
  const size_t v[9] = {l.header, l.stack, l.issued, l.owner, l.slab_table,
                       l.slot_len, l.slot_npages, l.slot_pages, l.total};
  for (int i = 0; i < 9; ++i) offsets[i] = v[i];
  return hipSuccess;
}

int mt_pool_init(MT_POOL_ARGS) {
  MT_POOL_CHECK
  init_kernel<<<256, 256>>>(MT_POOL);
  return hipGetLastError();
}

int mt_pool_pop(MT_POOL_ARGS, int count, int owner, int* out_pages) {
  MT_POOL_CHECK
  if (count < 0 || count > max_pages || (count > 0 && !out_pages)) return hipErrorInvalidValue;
  if (count) pop_kernel<<<1, kThreads>>>(MT_POOL, count, owner, out_pages);
  return hipGetLastError();
}

int mt_pool_push(MT_POOL_ARGS, const int* pages, int count, int owner) {
  MT_POOL_CHECK
  if (count < 0 || count > max_pages || (count > 0 && !pages)) return hipErrorInvalidValue;
  if (count) push_kernel<<<1, kThreads>>>(MT_POOL, pages, count, owner);
  return hipGetLastError();
}

int mt_pool_acquire_rows(MT_POOL_ARGS, const int* slots, int rows, int per_row, int* scratch) {
  MT_POOL_CHECK
  if (!slots || rows < 1 || per_row < 0 || int64_t(rows) * per_row > max_pages ||
      (per_row > 0 && !scratch))
    return hipErrorInvalidValue;
  if (per_row) acquire_rows_kernel<<<1, kThreads>>>(MT_POOL, slots, rows, per_row, scratch);
  return hipGetLastError();
}

int mt_pool_acquire_lists(MT_POOL_ARGS, const int* slots, const int* counts, int n, int* scratch) {
  MT_POOL_CHECK
  if (!slots || !counts || n < 1 || !scratch) return hipErrorInvalidValue;
  acquire_lists_kernel<<<1, kThreads>>>(MT_POOL, slots, counts, n, scratch);
  return hipGetLastError();
}

int mt_sched_add_lengths(MT_POOL_ARGS, const int* slots, const int* tokens, int n) {
  MT_POOL_CHECK
  if (!slots || !tokens || n < 1) return hipErrorInvalidValue;
  add_lengths_kernel<<<(n + kThreads - 1) / kThreads, kThreads>>>(MT_POOL, slots, tokens, n);
  return hipGetLastError();
}

int mt_pool_release_rows(MT_POOL_ARGS, const int* slots, int rows, int keep, int reset_length) {
  MT_POOL_CHECK
  if (!slots || rows < 1 || keep < 0) return hipErrorInvalidValue;
  release_rows_kernel<<<1, kThreads>>>(MT_POOL, slots, rows, keep, reset_length);
  return hipGetLastError();
}

int mt_sched_decode_prepare(MT_POOL_ARGS, const int* slots, int b, int columns, int page_size,
                            int limit, int* table, int* offsets, float* positions,
                            int* cu_seqlens, int* new_page) {
  MT_POOL_CHECK
  if (!slots || b < 1 || columns < 1 || columns > max_cols || limit < -1 || !table || !offsets ||
      !positions || !cu_seqlens || !new_page || !(page_size == 8 || page_size == 16 || page_size == 32) ||
      int64_t(b) * columns > INT32_MAX)
    return hipErrorInvalidValue;
  decode_prepare_kernel<<<1, kThreads>>>(MT_POOL, slots, b, columns, page_size, limit, table,
                                         offsets, positions, cu_seqlens, new_page);
  return hipGetLastError();
}

int mt_sched_decode_prepare_embed(MT_POOL_ARGS, const int* slots, int b, int columns, int page_size,
                                  int limit, int* table, int* offsets, float* positions,
                                  int* cu_seqlens, int* new_page, float* x, const float* wte,
                                  const float* wpe, const float* slot_tokens, int num_slots, int vocab,
                                  int n_positions, int dim) {
  MT_POOL_CHECK
  auto a16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; };
  if (!slots || b < 1 || columns < 1 || columns > max_cols || limit < -1 || !table || !offsets ||
      !positions || !cu_seqlens || !new_page || !(page_size == 8 || page_size == 16 || page_size == 32) ||
      int64_t(b) * columns > INT32_MAX || !x || !wte || !wpe || !slot_tokens || num_slots < 1 ||
      num_slots > max_slots || vocab < 1 || n_positions < 1 || dim < 4 || dim % 4 || !a16(x) || !a16(wte) || !a16(wpe) ||
      int64_t(b) * dim > INT32_MAX || int64_t(vocab) * dim > INT32_MAX || int64_t(n_positions) * dim > INT32_MAX)
    return hipErrorInvalidValue;
  EmbedArgs e{};
  e.x = x; e.wte = wte; e.wpe = wpe; e.slot_tokens = slot_tokens;
  e.num_slots = num_slots; e.vocab = vocab; e.n_positions = n_positions; e.dim = dim;
  const int64_t vecs = int64_t(b) * (dim / 4);
  const int64_t need = (vecs + kThreads - 1) / kThreads;
  const int embed_blocks = int(need < 64 ? need : 64);
  decode_prepare_embed_kernel<<<1 + embed_blocks, kThreads>>>(MT_POOL, slots, b, columns, page_size, limit,
                                                              table, offsets, positions, cu_seqlens,
                                                              new_page, e);
  return hipGetLastError();
}

int mt_sched_add_length(MT_POOL_ARGS, const int* slots, int b, int tokens) {
  MT_POOL_CHECK
  if (!slots || b < 1) return hipErrorInvalidValue;
  add_length_kernel<<<(b + kThreads - 1) / kThreads, kThreads>>>(MT_POOL, slots, b, tokens);
  return hipGetLastError();
}

int mt_sched_decode_abort(MT_POOL_ARGS, const int* slots, int b, const int* new_page) {
  MT_POOL_CHECK
  if (!slots || b < 1 || !new_page) return hipErrorInvalidValue;
  decode_abort_kernel<<<1, kThreads>>>(MT_POOL, slots, b, new_page);
  return hipGetLastError();
}

}  // extern "C"
