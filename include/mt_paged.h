/* Paged KV append and paged decode attention: C-ABI of
 * minitorch_amd/cuda_kernels/paged_attention_kernel.so (gfx950).
 *
 * Conventions (reference minitorch/cuda_resident_ops.py:41-47,
 * src/paged_attention_kernel.cu): every entry returns an int status, 0 on
 * success, otherwise a hipError_t value (1 = invalid value, 2 = out of
 * memory); pointers are device addresses; dtype 0 = float32, 1 = float16,
 * 2 = bfloat16; launches go to the calling thread's default stream (the
 * libraries are built with per-thread default streams) and never synchronize.
 *
 * Slab layout: [layers][2 (K,V)][pages_per_slab][heads][page_size][head_dim];
 * physical page p is slot p % pages_per_slab of slab p / pages_per_slab, whose
 * base address is slabs[p / pages_per_slab] (0 = absent). A table entry that
 * is negative, beyond the pool, or whose slab is absent is a missing page:
 * appends to it are skipped and attention reads it as NaN.
 */
#ifndef MT_PAGED_H
#define MT_PAGED_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Append n tokens per request at the common position `offset`:
 * K/V [b, h, n, d] -> pages through table [b, columns].
 * Replaces reference mt_paged_append (src/paged_attention_kernel.cu:96-106). */
int mt_paged_append(const void* k, const void* v, const uint64_t* slabs, const int* table, int b,
                    int h, int n, int d, int page_size, int pages_per_slab, int num_slabs,
                    int columns, int layer, int layers, int offset, int dtype);

/* Causal paged attention for nq >= 1 queries per request: out/q [b, h, nq, d];
 * query qi attends keys kj < nk with kj <= offset + qi (nk == offset + nq).
 * Replaces reference mt_paged_attention (src/paged_attention_kernel.cu:108-117). */
int mt_paged_attention(void* out, const void* q, const uint64_t* slabs, const int* table, int b,
                       int h, int nq, int nk, int d, int page_size, int pages_per_slab,
                       int num_slabs, int columns, int layer, int layers, int offset, int dtype);

/* Ragged batched decode: q/k/v/out [b, h, 1, d]; offsets[b] (device) are the
 * committed lengths. Appends k/v at position offsets[i] of request i, then
 * attends its offsets[i] + 1 keys. One fused append + attention launch, plus
 * a split-reduction launch when the table is longer than one context split
 * (1024 tokens). Rows are visited longest first, in the order
 * mt_paged_decode_split takes from a host work list, ranked on the device:
 * when no row can split and b <= 256 every workgroup ranks the rows by
 * offsets[] itself; otherwise, up to 2048 rows, a one-workgroup launch
 * (mt_paged_decode_order) writes the work list first and one residency
 * round of workgroups strides over it. Larger batches are visited in batch
 * order. The split partials and that list live in a library-owned
 * device workspace, one per (host thread, device) -- so calls from several
 * host threads, each on its own default stream, never share one -- kept
 * until the thread exits and grown stream-ordered on the calling thread's
 * default stream (hipMallocAsync / hipFreeAsync, no device synchronization)
 * when a table needs more; status 2 if it cannot grow. Batches of at most
 * 256 rows with tables of at most 1024 tokens allocate nothing.
 * Replaces reference mt_paged_decode_batch (src/paged_attention_kernel.cu:121-137). */
int mt_paged_decode_batch(void* out, const void* q, const void* k, const void* v,
                          const uint64_t* slabs, const int* table, const int* offsets, int b,
                          int h, int d, int page_size, int pages_per_slab, int num_slabs,
                          int columns, int layer, int layers, int dtype);

/* Bytes of device memory mt_paged_decode_batch_noalloc keeps for split
 * partials: a fixed array in the library, one copy per device, held until
 * the process ends. */
#define MT_PAGED_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)

/* mt_paged_decode_batch that allocates nothing: same arguments, kernels and
 * results, but the split partials of tables longer than one split (1024
 * tokens) live in the library's fixed device array of
 * MT_PAGED_NOALLOC_SCRATCH_BYTES instead of a workspace that may grow, and so
 * does the device-built visiting order. It returns 1 (invalid value) before
 * any launch when the partials, b * h * n * (d' + 2) * 4 bytes rounded up to
 * 256 (n = ceil(columns * page_size / split), d' = 64 for 16-byte-aligned
 * operands at d = 64, else 128; none when n = 1), plus the order,
 * (2 + (2 n + 1) b) * 4 bytes (none when n = 1 and b <= 256), exceed that
 * size. Calls on one device share the array: calls
 * that overlap (different streams) race; calls in stream order do not. The
 * first call on a device looks the array's device address up
 * (hipGetSymbolAddress) and keeps it; no call allocates or frees.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops and harnesses
 * that forbid hipMalloc). */
int mt_paged_decode_batch_noalloc(void* out, const void* q, const void* k, const void* v,
                                  const uint64_t* slabs, const int* table, const int* offsets,
                                  int b, int h, int d, int page_size, int pages_per_slab,
                                  int num_slabs, int columns, int layer, int layers, int dtype);

/* Number of launches since the library was loaded in which
 * mt_paged_attention / mt_paged_prefill split one long prompt's keys over
 * workgroups (query tiles x heads <= compute units, >= 6 key blocks in the
 * last tile). A diagnostic, e.g. for tests that must exercise that path.
 * No reference counterpart. */
int mt_paged_prefill_key_splits(long long* launches);

/* Bytes of workspace mt_paged_decode_split needs (0 when no row can be split).
 * split_tokens = 0 selects the automatic split length.
 * No reference counterpart: the split-context reduction is new in this build. */
int mt_paged_decode_workspace_bytes(int b, int h, int page_size, int columns, int split_tokens,
                                    size_t* bytes);

/* The split length mt_paged_decode_split uses for `requested` (0 = the
 * automatic choice: 1024 tokens, longer when a table of `columns` pages would
 * need more than 8 splits). No reference counterpart. */
int mt_paged_decode_split_tokens(int page_size, int columns, int requested, int* split_tokens);

/* The visiting order of a decode, built on the device from offsets[b]
 * (device, committed lengths as in mt_paged_decode_batch; 1 <= b <= 2048):
 * the work list mt_paged_decode_split takes, equal to the one a host caller
 * builds from the same lengths -- every (row, split) pair once, by tokens
 * descending, then row, then split, in passes of compute_units / h pairs
 * with every other pass reversed -- followed by the rows with more than one
 * split, ascending. A row past its table gets one pair (split 0). Writes
 * count[0] = pairs, count[1] = merge rows (device int[2]) and `list` (device,
 * 2 * b * n + b ints for n = ceil(columns * page_size / split)). split_tokens
 * and compute_units 0 = automatic (as mt_paged_decode_split; the device's
 * compute units). One launch of one workgroup on the calling thread's
 * default stream. No reference counterpart: mt_paged_decode_batch uses it to
 * order its rows. */
int mt_paged_decode_order(const int* offsets, int b, int h, int page_size, int columns,
                          int split_tokens, int compute_units, int* list, int* count);

/* mt_paged_decode_batch with a caller-owned workspace and tuning knobs:
 * split_tokens (a multiple of 64, at most 2048; 0 = automatic), unroll (1, 2
 * or 4 row-blocks per register stage, capped by the row size; 0 = automatic:
 * 2), waves per workgroup (2, 4 or 8; 0 = automatic: 8 when the whole grid is
 * resident at the 8-wave kernel's occupancy, 2 when the 2-wave kernel's grid
 * spans more than two residency rounds, else 4; 2 takes splits of at most
 * 1024 tokens, 512 for pages below 8, and runs 4 beyond), qkv_stride (elements between consecutive rows of q, k and
 * v, so that they can be column blocks of one fused [b, 3*h*d] projection
 * output; 0 = h*d, contiguous; out is always contiguous), and an optional
 * work list built by the caller from the
 * context lengths it knows on the host (device int32, 8-byte aligned): work_items pairs
 * (row, split), in the order they should be scheduled (e.g. longest first),
 * followed by merge_rows row indices, the rows with more than one split. A
 * work list requires an explicit split_tokens and must hold every (row,
 * split) of the batch; rows it omits are not written. With work == NULL every
 * (split, row) is scheduled in batch order and every row is merged as needed.
 * The workspace holds per-split partials; launches that share one workspace
 * must not overlap.
 * No reference counterpart (split-context variant of
 * src/paged_attention_kernel.cu:121-137). */
int mt_paged_decode_split(void* out, const void* q, const void* k, const void* v,
                          const uint64_t* slabs, const int* table, const int* offsets, int b,
                          int h, int d, int page_size, int pages_per_slab, int num_slabs,
                          int columns, int layer, int layers, int dtype, int split_tokens,
                          int unroll, int waves, int qkv_stride, const int* work,
                          int work_items, int merge_rows, void* workspace,
                          size_t workspace_bytes);

/* Prefill of n tokens per request at a common offset, in one call: appends
 * k/v (as mt_paged_append) and computes causal attention of the n queries
 * over keys [0, offset + n) (as mt_paged_attention), with token-major rows:
 * q, k and v are [b, n, qkv_stride] with head j at columns [j*d, (j+1)*d)
 * (qkv_stride = 3*h*d when they are column blocks of one fused projection;
 * 0 = h*d) and out is [b, n, out_stride] with heads merged the same way
 * (0 = h*d). The matrix-core kernel serves fp16/bf16 with d 64 or 128 and
 * n >= 16. No reference counterpart as one entry (reference
 * paged_kv_cache.py:205-221 calls mt_paged_append and mt_paged_attention on
 * head-split copies). */
int mt_paged_prefill(void* out, const void* q, const void* k, const void* v, const uint64_t* slabs,
                     const int* table, int b, int h, int n, int d, int page_size,
                     int pages_per_slab, int num_slabs, int columns, int layer, int layers,
                     int offset, int dtype, int qkv_stride, int out_stride);

/* mt_paged_prefill for `requests` prompts of different lengths in one call:
 * prompt r has tokens[r] token-major rows, concatenated in prompt order in
 * q/k/v (row stride qkv_stride, 0 = h*d) and out (out_stride, 0 = h*d), key
 * offset offsets[r] and its own block-table row tables[r] (a device pointer
 * to `columns` entries); tables, tokens and offsets are host arrays. Each
 * prompt's K/V are appended and its causal attention computed as
 * mt_paged_prefill would; with fp16/bf16, d 64/128 and 16-byte rows, up to 16
 * prompts (256 query tiles) share one append and one matrix-core launch.
 * No reference counterpart (the reference prefills one request per call). */
int mt_paged_prefill_ragged(void* out, const void* q, const void* k, const void* v,
                            const uint64_t* slabs, const int* const* tables, const int* tokens,
                            const int* offsets, int requests, int h, int d, int page_size,
                            int pages_per_slab, int num_slabs, int columns, int layer, int layers,
                            int dtype, int qkv_stride, int out_stride);

#ifdef __cplusplus
}
#endif
#endif /* MT_PAGED_H */
