/*
 * kv_oracle.c -- CPU oracle for the KV-cache transfer path.
 *
 * TEST INFRASTRUCTURE: the checker, never the product. Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
 *
 * Pinning status (what checks each function; see tests/test_oracle.py):
 *  - ora_tensor_token_byte_range / ora_tensor_slot_byte_range /
 *    ora_pair_tensor_token_byte_range: reference goldens
 *    (crates/sglang-srt/tests/kv_cache.rs:64-217,
 *    crates/sglang-srt/tests/cuda_backend.rs:284-286) and a numpy
 *    reshape-view of the pool.
 *  - ora_ref_gather/scatter_kv_pair_bytes: the reference acceptance pattern
 *    (cuda_backend.rs:497-637: slots 1,15,16,31, strides +37/+53 and
 *    +11/+19, bytes (seed + 37 r + 13 b) % 251) and numpy fancy indexing.
 *  - ora_pack / ora_unpack / ora_transfer / ora_resolve_slots: numpy
 *    reshape views ([page][layer][tensor][pos][row] for NHD,
 *    [page][layer][tensor][head][pos][chunk] for HND; for a tensor pair of
 *    unequal widths, [page][layer] split at page_size * key bytes into a
 *    [pos][key] and a [pos][value] view), agreement with the literal
 *    byte-per-thread restatement on NHD pairs, the asymmetric tensor-pair
 *    goldens of crates/sglang-srt/tests/kv_cache.rs:180-217, and round trips.
 *  - ora_transfer_page_indices: transfer.rs:679-720 error cases and
 *    crates/sglang-srt/tests/pd_transfer_plan.rs:85-114.
 *  - ora_f32_to_bf16: torch's round-to-nearest-even float32 -> bfloat16.
 */
#include "kv_oracle.h"

#include <pthread.h>
#include <string.h>

/* ---------------------------------------------------------------------- */
/* Layout (kv_cache.rs:448-777)                                            */
/* ---------------------------------------------------------------------- */

/* The runtime checks both geometries share (kv_cache.rs:531-586). */
static int ora_runtime_check(const ora_layout *l, uint64_t *per_layer) {
    if (l->page_count == 0) return ORA_LAYOUT_ZERO_PAGE_COUNT;
    if (l->page_size == 0 || l->num_layers == 0 || l->kv_tensors_per_token == 0 ||
        l->bytes_per_token == 0 || l->page_size_bytes == 0)
        return ORA_LAYOUT_ZERO_FIELD;
    if (l->page_size * l->bytes_per_token != l->page_size_bytes)
        return ORA_LAYOUT_RUNTIME_PAGE_SIZE_MISMATCH;
    if (l->bytes_per_token % l->num_layers) return ORA_LAYOUT_UNEVEN_LAYER;
    *per_layer = l->bytes_per_token / l->num_layers;
    return ORA_OK;
}

/* Uniform geometry: every tensor takes an equal share (kv_cache.rs:448-478). */
static int ora_layout_check(const ora_layout *l, uint64_t *per_layer, uint64_t *token_bytes) {
    int rc = ora_runtime_check(l, per_layer);
    if (rc) return rc;
    if (*per_layer % l->kv_tensors_per_token) return ORA_LAYOUT_UNEVEN_TENSOR;
    *token_bytes = *per_layer / l->kv_tensors_per_token;
    return ORA_OK;
}

/* Byte start of (page, layer, tensor, token):
 *   page * page_size_bytes                     -- pages are outermost
 * + layer * (page_size * bytes_per_token_per_layer)
 * + tensor * (page_size * token_bytes)
 * + token * token_bytes                        (kv_cache.rs:675-697) */
int ora_tensor_token_byte_range(const ora_layout *l, uint64_t page, uint64_t layer,
                                uint64_t tensor, uint64_t token, uint64_t *start, uint64_t *end) {
    uint64_t per_layer, tb;
    int rc = ora_layout_check(l, &per_layer, &tb);
    if (rc) return rc;
    if (page >= l->page_count) return ORA_LAYOUT_PAGE_OUT_OF_RANGE;
    if (layer >= l->num_layers) return ORA_LAYOUT_LAYER_OUT_OF_RANGE;
    if (tensor >= l->kv_tensors_per_token) return ORA_LAYOUT_TENSOR_OUT_OF_RANGE;
    if (token >= l->page_size) return ORA_LAYOUT_TOKEN_OUT_OF_RANGE;
    *start = page * l->page_size_bytes + layer * (l->page_size * per_layer) +
             tensor * (l->page_size * tb) + token * tb;
    *end = *start + tb;
    return ORA_OK;
}

int ora_tensor_slot_byte_range(const ora_layout *l, uint64_t layer, uint64_t tensor,
                               uint64_t slot, uint64_t *start, uint64_t *end) {
    if (l->page_size == 0) return ORA_LAYOUT_ZERO_FIELD;
    if (slot >= l->page_count * l->page_size) return ORA_LAYOUT_SLOT_OUT_OF_RANGE;
    return ora_tensor_token_byte_range(l, slot / l->page_size, layer, tensor,
                                       slot % l->page_size, start, end);
}

/* Pair geometry: the key region of a (page, layer) is page_size * key bytes
 * long and the value region follows it (kv_cache.rs:808-818). */
int ora_pair_tensor_token_byte_range(const ora_layout *l, uint64_t key_token_bytes,
                                     uint64_t value_token_bytes, uint64_t page, uint64_t layer,
                                     uint64_t tensor, uint64_t token, uint64_t *start,
                                     uint64_t *end) {
    uint64_t per_layer;
    int rc = ora_runtime_check(l, &per_layer);
    if (rc) return rc;
    /* the pair's widths need not be equal, but must fill the layer
     * (TensorPairSizeMismatch, kv_cache.rs:499-508) */
    if (key_token_bytes + value_token_bytes != per_layer) return ORA_LAYOUT_UNEVEN_TENSOR;
    if (page >= l->page_count) return ORA_LAYOUT_PAGE_OUT_OF_RANGE;
    if (layer >= l->num_layers) return ORA_LAYOUT_LAYER_OUT_OF_RANGE;
    if (tensor >= 2) return ORA_LAYOUT_TENSOR_OUT_OF_RANGE;
    if (token >= l->page_size) return ORA_LAYOUT_TOKEN_OUT_OF_RANGE;
    uint64_t width = tensor == 0 ? key_token_bytes : value_token_bytes;
    uint64_t region = tensor == 0 ? 0 : l->page_size * key_token_bytes;
    *start = page * l->page_size_bytes + layer * (l->page_size * per_layer) + region +
             token * width;
    *end = *start + width;
    return ORA_OK;
}

/* ---------------------------------------------------------------------- */
/* Literal byte-per-thread kernels (cuda_kv_kernels.rs:11-99)              */
/* ---------------------------------------------------------------------- */

uint32_t ora_ref_gather_kv_pair_bytes(const uint8_t *pool, const uint64_t *slots, uint8_t *keys,
                                      uint8_t *values, uint64_t row_count, uint64_t slot_count,
                                      uint64_t page_size, uint64_t page_stride_bytes,
                                      uint64_t key_in_page_offset, uint64_t value_in_page_offset,
                                      uint64_t row_bytes, uint64_t key_row_stride_bytes,
                                      uint64_t value_row_stride_bytes) {
    uint32_t flag = 0;
    const uint64_t plane_bytes = row_count * row_bytes;
    for (uint64_t index = 0; index < plane_bytes * 2; ++index) {
        const int is_value = index >= plane_bytes;
        const uint64_t plane_index = is_value ? index - plane_bytes : index;
        const uint64_t row = plane_index / row_bytes;
        const uint64_t byte = plane_index % row_bytes;
        const uint64_t slot = slots[row];
        if (slot >= slot_count) {
            flag = 1;
            continue;
        }
        const uint64_t page = slot / page_size;
        const uint64_t token = slot % page_size;
        const uint64_t in_page = is_value ? value_in_page_offset : key_in_page_offset;
        const uint64_t source = page * page_stride_bytes + in_page + token * row_bytes + byte;
        const uint64_t destination =
            row * (is_value ? value_row_stride_bytes : key_row_stride_bytes) + byte;
        if (is_value)
            values[destination] = pool[source];
        else
            keys[destination] = pool[source];
    }
    return flag;
}

uint32_t ora_ref_scatter_kv_pair_bytes(const uint8_t *keys, const uint8_t *values,
                                       const uint64_t *slots, uint8_t *pool, uint64_t row_count,
                                       uint64_t slot_count, uint64_t page_size,
                                       uint64_t page_stride_bytes, uint64_t key_in_page_offset,
                                       uint64_t value_in_page_offset, uint64_t row_bytes,
                                       uint64_t key_row_stride_bytes,
                                       uint64_t value_row_stride_bytes) {
    uint32_t flag = 0;
    const uint64_t plane_bytes = row_count * row_bytes;
    for (uint64_t index = 0; index < plane_bytes * 2; ++index) {
        const int is_value = index >= plane_bytes;
        const uint64_t plane_index = is_value ? index - plane_bytes : index;
        const uint64_t row = plane_index / row_bytes;
        const uint64_t byte = plane_index % row_bytes;
        const uint64_t slot = slots[row];
        if (slot >= slot_count) {
            flag = 1;
            continue;
        }
        const uint64_t page = slot / page_size;
        const uint64_t token = slot % page_size;
        const uint64_t in_page = is_value ? value_in_page_offset : key_in_page_offset;
        const uint64_t destination = page * page_stride_bytes + in_page + token * row_bytes + byte;
        const uint64_t source =
            row * (is_value ? value_row_stride_bytes : key_row_stride_bytes) + byte;
        pool[destination] = is_value ? values[source] : keys[source];
    }
    return flag;
}

/* ---------------------------------------------------------------------- */
/* Generalised row-granular copies                                         */
/* ---------------------------------------------------------------------- */

uint32_t ora_resolve_slots(const ora_pool *pool, const uint64_t *slots, const int32_t *page_table,
                           uint64_t page_table_len, const ora_span *spans, uint32_t span_count,
                           uint64_t row_count, uint64_t *out_slots) {
    uint32_t flag = 0;
    const uint64_t slot_count = pool->page_count * pool->page_size;
    for (uint64_t r = 0; r < row_count; ++r) out_slots[r] = UINT64_MAX;
    if (slots) {
        for (uint64_t r = 0; r < row_count; ++r) {
            if (slots[r] < slot_count)
                out_slots[r] = slots[r];
            else
                flag |= ORA_FLAG_SLOT;
        }
        return flag;
    }
    /* Spans are walked in order; span s covers rows row_start .. +count.
     * A covered row whose page lookup fails is marked UINT64_MAX - 1 until
     * the end, so that it is not also reported as uncovered. */
    const uint64_t covered_bad = UINT64_MAX - 1;
    for (uint32_t s = 0; s < span_count; ++s) {
        const ora_span sp = spans[s];
        for (uint64_t j = 0; j < sp.token_count; ++j) {
            const uint64_t row = (uint64_t)sp.row_start + j;
            if (row >= row_count) break;
            const uint64_t token = (uint64_t)sp.token_offset + j;
            const uint64_t index = (uint64_t)sp.page_table_start + token / pool->page_size;
            if (index >= page_table_len || page_table[index] < 0 ||
                (uint64_t)page_table[index] >= pool->page_count) {
                flag |= ORA_FLAG_PAGE;
                out_slots[row] = covered_bad;
                continue;
            }
            out_slots[row] = (uint64_t)page_table[index] * pool->page_size + token % pool->page_size;
        }
    }
    for (uint64_t r = 0; r < row_count; ++r) {
        if (out_slots[r] == UINT64_MAX) flag |= ORA_FLAG_SPAN;
        if (out_slots[r] == covered_bad) out_slots[r] = UINT64_MAX;
    }
    return flag;
}

uint64_t ora_pool_row_bytes(const ora_pool *pool, uint32_t t) {
    return t == 1 && pool->value_row_bytes ? pool->value_row_bytes : pool->row_bytes;
}

uint64_t ora_pool_chunk_offset(const ora_pool *pool, uint64_t slot, uint32_t t, uint32_t h) {
    const uint64_t page = slot / pool->page_size;
    const uint64_t pos = slot % pool->page_size;
    const uint64_t rb = ora_pool_row_bytes(pool, t);
    const uint64_t chunk = rb / pool->heads;
    const uint64_t region = page * pool->page_stride + pool->tensor_offset[t];
    if (pool->hnd) return region + ((uint64_t)h * pool->page_size + pos) * chunk;
    return region + pos * rb + (uint64_t)h * chunk;
}

typedef struct ora_job {
    int kind; /* 0 pack, 1 unpack, 2 transfer */
    const ora_pool *src, *dst;
    const uint8_t *src_bytes;
    uint8_t *dst_bytes;
    const uint64_t *src_slots, *dst_slots;
    const uint8_t *rows_in[2];
    uint8_t *rows_out[2];
    uint64_t stride[2];
    uint64_t row_begin, row_end;
} ora_job;

static void *ora_run(void *arg) {
    const ora_job *j = (const ora_job *)arg;
    const ora_pool *pool = j->kind == 1 ? j->dst : j->src;
    const uint32_t tensors = pool->tensors;
    for (uint64_t r = j->row_begin; r < j->row_end; ++r) {
        if (j->kind == 0) {
            const uint64_t slot = j->src_slots[r];
            if (slot == UINT64_MAX) continue;
            for (uint32_t t = 0; t < tensors; ++t) {
                uint8_t *out = j->rows_out[t] + r * j->stride[t];
                const uint64_t rb = ora_pool_row_bytes(pool, t);
                if (!pool->hnd) {
                    memcpy(out, j->src_bytes + ora_pool_chunk_offset(pool, slot, t, 0), rb);
                } else {
                    const uint64_t chunk = rb / pool->heads;
                    for (uint32_t h = 0; h < pool->heads; ++h)
                        memcpy(out + h * chunk,
                               j->src_bytes + ora_pool_chunk_offset(pool, slot, t, h), chunk);
                }
            }
        } else if (j->kind == 1) {
            const uint64_t slot = j->dst_slots[r];
            if (slot == UINT64_MAX) continue;
            for (uint32_t t = 0; t < tensors; ++t) {
                const uint8_t *in = j->rows_in[t] + r * j->stride[t];
                const uint64_t rb = ora_pool_row_bytes(pool, t);
                if (!pool->hnd) {
                    memcpy(j->dst_bytes + ora_pool_chunk_offset(pool, slot, t, 0), in, rb);
                } else {
                    const uint64_t chunk = rb / pool->heads;
                    for (uint32_t h = 0; h < pool->heads; ++h)
                        memcpy(j->dst_bytes + ora_pool_chunk_offset(pool, slot, t, h),
                               in + h * chunk, chunk);
                }
            }
        } else {
            const uint64_t s = j->src_slots[r], d = j->dst_slots[r];
            if (s == UINT64_MAX || d == UINT64_MAX) continue;
            /* Heads are the common unit of both layouts. */
            const uint32_t heads = j->src->heads;
            for (uint32_t t = 0; t < tensors; ++t) {
                const uint64_t chunk = ora_pool_row_bytes(j->src, t) / heads;
                for (uint32_t h = 0; h < heads; ++h)
                    memcpy(j->dst_bytes + ora_pool_chunk_offset(j->dst, d, t, h),
                           j->src_bytes + ora_pool_chunk_offset(j->src, s, t, h), chunk);
            }
        }
    }
    return NULL;
}

static void ora_parallel(ora_job base, uint64_t row_count, int threads) {
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    if ((uint64_t)threads > row_count) threads = row_count ? (int)row_count : 1;
    if (threads == 1) {
        base.row_begin = 0;
        base.row_end = row_count;
        ora_run(&base);
        return;
    }
    pthread_t tid[256];
    ora_job jobs[256];
    for (int i = 0; i < threads; ++i) {
        jobs[i] = base;
        jobs[i].row_begin = row_count * (uint64_t)i / (uint64_t)threads;
        jobs[i].row_end = row_count * (uint64_t)(i + 1) / (uint64_t)threads;
        pthread_create(&tid[i], NULL, ora_run, &jobs[i]);
    }
    for (int i = 0; i < threads; ++i) pthread_join(tid[i], NULL);
}

void ora_pack(const ora_pool *pool, const uint8_t *pool_bytes, const uint64_t *row_slots,
              uint64_t row_count, uint8_t *rows0, uint8_t *rows1, uint64_t stride0,
              uint64_t stride1, int threads) {
    ora_job j;
    memset(&j, 0, sizeof j);
    j.kind = 0;
    j.src = pool;
    j.src_bytes = pool_bytes;
    j.src_slots = row_slots;
    j.rows_out[0] = rows0;
    j.rows_out[1] = rows1;
    j.stride[0] = stride0;
    j.stride[1] = stride1;
    ora_parallel(j, row_count, threads);
}

void ora_unpack(const ora_pool *pool, uint8_t *pool_bytes, const uint64_t *row_slots,
                uint64_t row_count, const uint8_t *rows0, const uint8_t *rows1, uint64_t stride0,
                uint64_t stride1, int threads) {
    ora_job j;
    memset(&j, 0, sizeof j);
    j.kind = 1;
    j.dst = pool;
    j.dst_bytes = pool_bytes;
    j.dst_slots = row_slots;
    j.rows_in[0] = rows0;
    j.rows_in[1] = rows1;
    j.stride[0] = stride0;
    j.stride[1] = stride1;
    ora_parallel(j, row_count, threads);
}

void ora_transfer(const ora_pool *src, const uint8_t *src_bytes, const uint64_t *src_slots,
                  const ora_pool *dst, uint8_t *dst_bytes, const uint64_t *dst_slots,
                  uint64_t row_count, int threads) {
    ora_job j;
    memset(&j, 0, sizeof j);
    j.kind = 2;
    j.src = src;
    j.dst = dst;
    j.src_bytes = src_bytes;
    j.dst_bytes = dst_bytes;
    j.src_slots = src_slots;
    j.dst_slots = dst_slots;
    ora_parallel(j, row_count, threads);
}

/* ---------------------------------------------------------------------- */
/* Transfer plan pages (transfer.rs:679-720)                               */
/* ---------------------------------------------------------------------- */

int ora_transfer_page_indices(uint64_t token_offset, const uint64_t *cache_slots,
                              uint64_t slot_len, uint64_t page_size, uint64_t *out_pages,
                              uint64_t *out_len) {
    *out_len = 0;
    if (slot_len == 0) return ORA_OK;
    if (token_offset % page_size) return ORA_PLAN_UNALIGNED_TOKEN_OFFSET;
    for (uint64_t first = 0; first < slot_len; first += page_size) {
        const uint64_t head = cache_slots[first];
        if (head % page_size) return ORA_PLAN_UNALIGNED_CACHE_SLOT;
        const uint64_t stop = first + page_size < slot_len ? first + page_size : slot_len;
        for (uint64_t i = first; i < stop; ++i)
            if (cache_slots[i] != head + (i - first)) return ORA_PLAN_NON_CONTIGUOUS_CACHE_SLOTS;
        out_pages[(*out_len)++] = head / page_size;
    }
    return ORA_OK;
}

/* ---------------------------------------------------------------------- */
/* Test-input helper                                                       */
/* ---------------------------------------------------------------------- */

void ora_f32_to_bf16(const float *in, uint16_t *out, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) {
        uint32_t bits;
        memcpy(&bits, &in[i], sizeof bits);
        const uint32_t bias = 0x7fffu + ((bits >> 16) & 1u);
        out[i] = (uint16_t)((bits + bias) >> 16);
    }
}
