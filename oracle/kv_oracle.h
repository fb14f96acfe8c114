/*
 * kv_oracle.h -- CPU oracle for the KV-cache transfer path.
 *
 * TEST INFRASTRUCTURE. This is the checker the HIP path is compared with:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it, and never as the thing measured or shipped. The product
 * (libsgl_rocm_kv.so) neither links nor calls it.
 *
 * It restates, in plain C and independently of the product code:
 *  - the page-major byte layout of PagedKvCacheLayout
 *    (crates/sglang-srt/src/kv_cache.rs:448-777);
 *  - the reference's byte-per-thread scatter/gather kernels, literally, one
 *    byte at a time (crates/sglang-kernel/src/cuda_kv_kernels.rs:11-99);
 *  - row-granular pack / unpack / pool-to-pool transfer for the generalised
 *    layouts (HND pages, page tables, single-tensor MLA rows). The reference
 *    has no such code; these are pinned by the closed-form definitions in
 *    the header of each function and by the checks in tests/.
 *  - transfer_page_indices (crates/sglang-srt/src/transfer.rs:679-720);
 *  - the f32 -> bf16 helper of the reference tests
 *    (crates/sglang-srt/tests/cuda_backend.rs:125-129).
 */
#ifndef KV_ORACLE_H
#define KV_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Error flag bits raised by the row-granular functions. */
#define ORA_FLAG_SLOT 1u /* a slot map entry >= slot_count */
#define ORA_FLAG_PAGE 2u /* a page-table index or entry out of range */
#define ORA_FLAG_SPAN 4u /* a row not covered by its span list */

/* Layout status codes (same numbering as the product's sgl_kv_status). */
#define ORA_OK 0
#define ORA_LAYOUT_ZERO_PAGE_COUNT 20
#define ORA_LAYOUT_ZERO_FIELD 21
#define ORA_LAYOUT_RUNTIME_PAGE_SIZE_MISMATCH 22
#define ORA_LAYOUT_UNEVEN_LAYER 23
#define ORA_LAYOUT_UNEVEN_TENSOR 24
#define ORA_LAYOUT_SIZE_OVERFLOW 25
#define ORA_LAYOUT_PAGE_OUT_OF_RANGE 26
#define ORA_LAYOUT_LAYER_OUT_OF_RANGE 27
#define ORA_LAYOUT_TENSOR_OUT_OF_RANGE 28
#define ORA_LAYOUT_TOKEN_OUT_OF_RANGE 29
#define ORA_LAYOUT_SLOT_OUT_OF_RANGE 30
#define ORA_PLAN_UNALIGNED_TOKEN_OFFSET 43
#define ORA_PLAN_UNALIGNED_CACHE_SLOT 44
#define ORA_PLAN_NON_CONTIGUOUS_CACHE_SLOTS 45

/* Uniform page-major layout (kv_cache.rs:448-478, Uniform geometry). */
typedef struct ora_layout {
    uint64_t page_size, num_layers, kv_tensors_per_token, bytes_per_token, page_size_bytes;
    uint64_t page_count;
} ora_layout;

/* tensor_token_byte_range (kv_cache.rs:653-700) for a Uniform layout. */
int ora_tensor_token_byte_range(const ora_layout *l, uint64_t page, uint64_t layer,
                                uint64_t tensor, uint64_t token, uint64_t *start, uint64_t *end);
/* tensor_slot_byte_range (kv_cache.rs:702-720). */
int ora_tensor_slot_byte_range(const ora_layout *l, uint64_t layer, uint64_t tensor,
                               uint64_t slot, uint64_t *start, uint64_t *end);
/* Explicit K/V pair layout (kv_cache.rs:480-529): token widths differ. */
int ora_pair_tensor_token_byte_range(const ora_layout *l, uint64_t key_token_bytes,
                                     uint64_t value_token_bytes, uint64_t page, uint64_t layer,
                                     uint64_t tensor, uint64_t token, uint64_t *start,
                                     uint64_t *end);

/* Literal restatement of sglang_gather_kv_pair_bytes (cuda_kv_kernels.rs:
 * 54-99): one iteration per (plane, row, byte). Returns the error flag
 * (1 when some slot >= slot_count; such bytes are skipped). */
uint32_t ora_ref_gather_kv_pair_bytes(const uint8_t *pool, const uint64_t *slots, uint8_t *keys,
                                      uint8_t *values, uint64_t row_count, uint64_t slot_count,
                                      uint64_t page_size, uint64_t page_stride_bytes,
                                      uint64_t key_in_page_offset, uint64_t value_in_page_offset,
                                      uint64_t row_bytes, uint64_t key_row_stride_bytes,
                                      uint64_t value_row_stride_bytes);
/* Literal restatement of sglang_scatter_kv_pair_bytes (cuda_kv_kernels.rs:11-52). */
uint32_t ora_ref_scatter_kv_pair_bytes(const uint8_t *keys, const uint8_t *values,
                                       const uint64_t *slots, uint8_t *pool, uint64_t row_count,
                                       uint64_t slot_count, uint64_t page_size,
                                       uint64_t page_stride_bytes, uint64_t key_in_page_offset,
                                       uint64_t value_in_page_offset, uint64_t row_bytes,
                                       uint64_t key_row_stride_bytes,
                                       uint64_t value_row_stride_bytes);

/* One layer of a pool. A (page, layer, tensor t) region starts at
 * page * page_stride + tensor_offset[t] and holds page_size rows of
 * rb_t bytes, rb_0 = row_bytes and rb_1 = value_row_bytes (0: row_bytes;
 * the tensor-pair layout of kv_cache.rs:480-529 has unequal widths).
 * NHD: token-major rows. HND: the region is [heads][page_size][rb_t / heads]. */
typedef struct ora_pool {
    uint64_t page_size, page_stride, page_count;
    uint64_t tensor_offset[2];
    uint64_t row_bytes;
    uint32_t tensors, heads, hnd, reserved;
    uint64_t value_row_bytes;
} ora_pool;

/* Bytes per (token, tensor t) of a pool. */
uint64_t ora_pool_row_bytes(const ora_pool *pool, uint32_t t);

typedef struct ora_span {
    uint32_t row_start, token_offset, token_count, page_table_start;
} ora_span;

/* Resolves the physical slot of rows [0, row_count): slots[r] when slots is
 * non-NULL, else from spans + page table (token k of a span -> page
 * page_table[page_table_start + k / page_size], position k % page_size).
 * Invalid rows get UINT64_MAX; the return value ORs the ORA_FLAG_* bits. */
uint32_t ora_resolve_slots(const ora_pool *pool, const uint64_t *slots, const int32_t *page_table,
                           uint64_t page_table_len, const ora_span *spans, uint32_t span_count,
                           uint64_t row_count, uint64_t *out_slots);

/* Byte offset of head chunk h of (slot, tensor t) in the pool. */
uint64_t ora_pool_chunk_offset(const ora_pool *pool, uint64_t slot, uint32_t t, uint32_t h);

/* Pack: rows[t] + r * stride[t] <- pool row (slot[r], t), rb_t bytes. Rows
 * whose slot is UINT64_MAX are left untouched. */
void ora_pack(const ora_pool *pool, const uint8_t *pool_bytes, const uint64_t *row_slots,
              uint64_t row_count, uint8_t *rows0, uint8_t *rows1, uint64_t stride0,
              uint64_t stride1, int threads);
/* Unpack: pool row (slot[r], t) <- rows[t] + r * stride[t]. */
void ora_unpack(const ora_pool *pool, uint8_t *pool_bytes, const uint64_t *row_slots,
                uint64_t row_count, const uint8_t *rows0, const uint8_t *rows1, uint64_t stride0,
                uint64_t stride1, int threads);
/* Pool to pool: dst row (dst_slot[r], t) <- src row (src_slot[r], t). */
void ora_transfer(const ora_pool *src, const uint8_t *src_bytes, const uint64_t *src_slots,
                  const ora_pool *dst, uint8_t *dst_bytes, const uint64_t *dst_slots,
                  uint64_t row_count, int threads);

/* transfer_page_indices (transfer.rs:679-720). Returns ORA_OK or an
 * ORA_PLAN_* code; *out_len = number of pages written. */
int ora_transfer_page_indices(uint64_t token_offset, const uint64_t *cache_slots,
                              uint64_t slot_len, uint64_t page_size, uint64_t *out_pages,
                              uint64_t *out_len);

/* f32 -> bf16 bits, round to nearest even, as cuda_backend.rs:125-129. */
void ora_f32_to_bf16(const float *in, uint16_t *out, uint64_t n);

#ifdef __cplusplus
}
#endif

#endif
