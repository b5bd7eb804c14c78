/* Device-side page allocator and decode-step scheduler metadata: C-ABI of
 * minitorch_amd/cuda_kernels/sched_kernels.so (gfx950).
 *
 * The reference keeps the page free list, per-cache page lists, block tables
 * and decode offsets on the host (minitorch/paged_kv_cache.py:27-263,
 * minitorch/paged_decode.py:10-93) and uploads them every step. Here they live
 * in one device "pool state" blob updated by kernels on the calling thread's default stream, with
 * page IDs identical to the reference's allocator: LIFO pops, new slabs'
 * page IDs pushed in reverse order on top of older free pages before a pop
 * that finds too few free pages, releases pushed in the given order.
 *
 * Every pool entry takes the same geometry arguments (MT_POOL_ARGS below):
 * state (device blob of the size mt_pool_layout reports), max_pages =
 * max_slabs * pages_per_slab, max_slots (cache rows the pool can track),
 * max_cols (page columns per row), pool_base (device address of slab 0;
 * slab s is at pool_base + s * slab_bytes). Status convention as in
 * mt_paged.h. Budget checks (MemoryError in the reference) are the caller's:
 * the host knows how many pages are leased without reading the device.
 */
#ifndef MT_SCHED_H
#define MT_SCHED_H
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Header at offset 0 of the state blob. */
typedef struct mt_pool_header {
  int top;          /* free pages on the stack */
  int slabs_opened; /* slabs whose pages have entered the free list */
  int leased;       /* pages owned by caches or API owners */
  int error;        /* bit 0: a release of pages the owner does not hold; bit 1: an
                       mt_pool_acquire_lists entry beyond its slot's columns or the budget */
  long long acquires, releases, reuses;
} mt_pool_header;

/* Byte offsets inside the state blob: [0] header, [1] free stack (int32
 * [max_pages]), [2] issued bitmap, [3] page owner (int32 [max_pages]),
 * [4] slab table (uint64 [max_slabs], 0 until a slab is opened), [5] slot
 * lengths (int32 [max_slots]), [6] slot page counts, [7] slot pages (int32
 * [max_slots, max_cols], -1 beyond a row's pages), [8] total bytes.
 * No reference counterpart (new device-side metadata). */
int mt_pool_layout(int max_pages, int max_slabs, int max_slots, int max_cols, size_t* offsets);

#define MT_POOL_ARGS                                                                          \
  void *state, int max_pages, int max_slabs, int max_slots, int max_cols, int pages_per_slab, \
      unsigned long long pool_base, unsigned long long slab_bytes

/* Empty pool: no slabs opened, every slot row empty.
 * Replaces the state set up by reference KVPagePool.__init__ (minitorch/paged_kv_cache.py:62-69). */
int mt_pool_init(MT_POOL_ARGS);

/* Pop `count` pages for `owner` into out_pages (device int32 [count]).
 * Replaces reference KVPagePool.acquire (minitorch/paged_kv_cache.py:71-94). */
int mt_pool_pop(MT_POOL_ARGS, int count, int owner, int* out_pages);

/* Push pages (device int32 [count]) held by `owner`, in order; a page the
 * owner does not hold sets header.error and is skipped.
 * Replaces reference KVPagePool.release (minitorch/paged_kv_cache.py:96-103). */
int mt_pool_push(MT_POOL_ARGS, const int* pages, int count, int owner);

/* Append per_row pages to each row slots[0..rows) from one pop of
 * rows * per_row pages (scratch: device int32 [rows * per_row]).
 * Replaces the page part of reference PagedKVCache.prepare_append
 * (minitorch/paged_kv_cache.py:171-186). */
int mt_pool_acquire_rows(MT_POOL_ARGS, const int* slots, int rows, int per_row, int* scratch);

/* prepare_append of n one-row caches in order: for i = 0..n-1, one pop of
 * counts[i] (device int32 [n]; host-checked against the budget and the
 * slot's columns, and checked again by the kernel: an entry with an invalid
 * slot, more pages than its slot's free columns or than the free budget is
 * skipped and sets bit 1 of header.error) pages appended to slot slots[i]'s
 * page list, the pops
 * opening slabs exactly as n mt_pool_acquire_rows calls of one row would
 * (scratch: device int32 [max counts[i]]). Replaces the page part of n
 * consecutive reference PagedKVCache.prepare_append calls
 * (minitorch/paged_kv_cache.py:171-186) with one launch. */
int mt_pool_acquire_lists(MT_POOL_ARGS, const int* slots, const int* counts, int n, int* scratch);

/* Release the pages [keep:] of each row slots[0..rows), row by row; with
 * reset_length the rows' lengths become 0. keep = 0 replaces reference
 * _release_cache / PagedKVCache.close (minitorch/paged_kv_cache.py:125-131);
 * keep = the page count before an append replaces PagedKVCache.abort_append
 * (minitorch/paged_kv_cache.py:228-234). */
int mt_pool_release_rows(MT_POOL_ARGS, const int* slots, int rows, int keep, int reset_length);

/* Decode-step metadata for the rows slots[0..b) (one new token each): every
 * row whose next token starts a new page takes one page, row by row (at most
 * `limit` pops); new_page[i] = that page or -1; offsets[i] = committed length;
 * positions[i] = (float)offsets[i]; cu_seqlens[0..b] = exclusive prefix sum
 * of offsets[i] + 1; table [b, columns] = each row's pages, -1 beyond them.
 * Replaces reference PagedDecodeBatch.prepare (minitorch/paged_decode.py:40-54). */
int mt_sched_decode_prepare(MT_POOL_ARGS, const int* slots, int b, int columns, int page_size,
                            int limit, int* table, int* offsets, float* positions,
                            int* cu_seqlens, int* new_page);

/* mt_sched_decode_prepare and the step's token embeddings in one launch:
 * also x[i, :] = wte[id_i, :] + wpe[pos_i, :] (fp32, [b, dim]) with id_i =
 * slot_tokens[slots[i]] (the slot's last token, num_slots <= max_slots entries) and
 * pos_i = its committed length, as mt_embed_tokens computes them from the
 * positions this call writes (same NaN rule: an id or position that is
 * non-finite, negative, too large or not integral, or a slot outside the
 * table, gives a NaN row). dim % 4 == 0, x/wte/wpe 16-byte aligned. One
 * workgroup builds the metadata while the others embed. No reference
 * counterpart (it saves the embedding's launch in a decode step). */
int mt_sched_decode_prepare_embed(MT_POOL_ARGS, const int* slots, int b, int columns, int page_size,
                                  int limit, int* table, int* offsets, float* positions,
                                  int* cu_seqlens, int* new_page, float* x, const float* wte,
                                  const float* wpe, const float* slot_tokens, int num_slots, int vocab,
                                  int n_positions, int dim);

/* lengths[slots[i]] += tokens. Replaces the length update of reference
 * CacheBase.commit_append (minitorch/kv_cache.py:142-147). */
int mt_sched_add_length(MT_POOL_ARGS, const int* slots, int b, int tokens);

/* lengths[slots[i]] += tokens[i] for i < n (device int32 arrays): the length
 * update of n reference CacheBase.commit_append calls
 * (minitorch/kv_cache.py:142-147) with one launch. */
int mt_sched_add_lengths(MT_POOL_ARGS, const int* slots, const int* tokens, int n);

/* Return the pages taken by mt_sched_decode_prepare (new_page >= 0), in row
 * order. Replaces reference PagedDecodeBatch.__exit__'s aborts
 * (minitorch/paged_decode.py:88-90). */
int mt_sched_decode_abort(MT_POOL_ARGS, const int* slots, int b, const int* new_page);

#undef MT_POOL_ARGS

#ifdef __cplusplus
}
#endif
#endif /* MT_SCHED_H */
