// kv_plan.cpp -- host mirror of the scheduler-side producers of the transfer
// path's metadata: the KV page allocator that hands out slot indices
// (CachePageAllocator, crates/sglang-srt/src/cache.rs:340-473), the
// token-prefix cache whose match sets a span's token offset (RadixCache,
// cache.rs:475-547), the transfer plan of a prefill batch
// (KvCacheTransferPlan::from_prefill_worker_batch_with_page_size,
// crates/sglang-srt/src/transfer.rs:604-668) and the transfer span's
// descriptor checksum (KvCacheTransferSpan::descriptor_checksum,
// transfer.rs:548-570), with a SHA-256 written from FIPS 180-4. No HIP calls.
#include <string.h>

#include <deque>
#include <unordered_map>
#include <vector>

#include "kv_internal.h"

using namespace sglkv;

// --- page allocator ------------------------------------------------------------------------

struct sgl_kv_page_allocator {
    uint64_t slot_capacity;
    uint64_t page_size;
    std::deque<uint64_t> free_pages;  // front is handed out first
    std::vector<uint8_t> allocated;   // per page

    void reset() {
        const uint64_t pages = slot_capacity / page_size;
        free_pages.clear();
        for (uint64_t p = 0; p < pages; ++p) free_pages.push_back(p);
        allocated.assign(pages, 0);
    }
};

// CachePageAllocator::with_page_size (cache.rs:353-376).
extern "C" int32_t sgl_kv_page_allocator_new(uint64_t slot_capacity, uint64_t page_size,
                                             sgl_kv_page_allocator **out) {
    if (!out) return fail(SGL_KV_INVALID_ARGUMENT, "out", 0, 0, 0, "null argument");
    *out = nullptr;
    if (page_size == 0)
        return fail(SGL_KV_ALLOC_ZERO_PAGE_SIZE, nullptr, 0, 0, 0, "KV cache page size must be non-zero");
    if (slot_capacity == 0)
        return fail(SGL_KV_ALLOC_ZERO_SLOT_CAPACITY, nullptr, 0, 0, 0,
                    "KV cache slot capacity must be non-zero");
    if (slot_capacity % page_size)
        return fail(SGL_KV_ALLOC_SLOT_CAPACITY_NOT_PAGE_ALIGNED, nullptr, slot_capacity, page_size, 0,
                    "KV cache slot capacity %llu must be divisible by page size %llu",
                    (unsigned long long)slot_capacity, (unsigned long long)page_size);
    if (slot_capacity / page_size > (1ull << 32))
        return fail(SGL_KV_DIMENSION_TOO_LARGE, "page_count", slot_capacity / page_size, 1ull << 32, 0,
                    "allocator page count %llu exceeds %llu",
                    (unsigned long long)(slot_capacity / page_size), 1ull << 32);
    sgl_kv_page_allocator *a = new sgl_kv_page_allocator();
    a->slot_capacity = slot_capacity;
    a->page_size = page_size;
    a->reset();
    *out = a;
    return ok();
}

extern "C" int32_t sgl_kv_page_allocator_destroy(sgl_kv_page_allocator *a) {
    delete a;
    return SGL_KV_OK;
}

extern "C" uint64_t sgl_kv_page_allocator_available_pages(const sgl_kv_page_allocator *a) {
    return a ? a->free_pages.size() : 0;
}

extern "C" uint64_t sgl_kv_page_allocator_available_slots(const sgl_kv_page_allocator *a) {
    return a ? a->free_pages.size() * a->page_size : 0;
}

// CachePageAllocator::allocate_for_sequence (cache.rs:397-447): the free
// slots left in the sequence's last page are used first, then whole pages
// from the front of the free list. Nothing is taken when the request does
// not fit.
extern "C" int32_t sgl_kv_page_allocator_allocate_for_sequence(sgl_kv_page_allocator *a,
                                                               const uint64_t *sequence_slots,
                                                               uint64_t sequence_len,
                                                               uint64_t slot_count,
                                                               uint64_t *out_slots) {
    if (!a) return fail(SGL_KV_INVALID_ARGUMENT, "allocator", 0, 0, 0, "null allocator");
    if (slot_count == 0) return ok();
    if (!out_slots || (sequence_len && !sequence_slots))
        return fail(SGL_KV_INVALID_ARGUMENT, "out_slots/sequence_slots", 0, 0, 0, "null argument");
    const uint64_t P = a->page_size;
    uint64_t tail = 0;
    if (sequence_len) {
        const uint64_t last = sequence_slots[sequence_len - 1];
        const uint64_t page = last / P;
        if (page < a->allocated.size() && a->allocated[page]) tail = P - last % P - 1;
        if (tail > slot_count) tail = slot_count;
    }
    const uint64_t fresh = slot_count - tail;
    const uint64_t pages = fresh / P + (fresh % P ? 1 : 0);
    if (pages > a->free_pages.size())
        return fail(SGL_KV_ALLOC_OUT_OF_SLOTS, nullptr, slot_count, tail + a->free_pages.size() * P, 0,
                    "KV cache needs %llu slots but only %llu are available",
                    (unsigned long long)slot_count,
                    (unsigned long long)(tail + a->free_pages.size() * P));
    uint64_t n = 0;
    if (tail) {
        const uint64_t first = sequence_slots[sequence_len - 1] + 1;
        for (uint64_t i = 0; i < tail; ++i) out_slots[n++] = first + i;
    }
    uint64_t remaining = fresh;
    for (uint64_t i = 0; i < pages; ++i) {
        const uint64_t page = a->free_pages.front();
        a->free_pages.pop_front();
        a->allocated[page] = 1;
        const uint64_t in_page = remaining < P ? remaining : P;
        for (uint64_t s = 0; s < in_page; ++s) out_slots[n++] = page * P + s;
        remaining -= in_page;
    }
    return ok();
}

// CachePageAllocator::release (cache.rs:449-466): a page returns to the
// front of the free list when the slot that opens it (its first slot) is
// released; released pages keep their order.
extern "C" int32_t sgl_kv_page_allocator_release(sgl_kv_page_allocator *a, const uint64_t *cache_pages,
                                                 uint64_t count) {
    if (!a) return fail(SGL_KV_INVALID_ARGUMENT, "allocator", 0, 0, 0, "null allocator");
    if (count && !cache_pages) return fail(SGL_KV_INVALID_ARGUMENT, "cache_pages", 0, 0, 0, "null argument");
    std::vector<uint64_t> released;
    for (uint64_t i = 0; i < count; ++i) {
        const uint64_t slot = cache_pages[i];
        if (slot >= a->slot_capacity || slot % a->page_size) continue;
        const uint64_t page = slot / a->page_size;
        if (a->allocated[page]) {
            a->allocated[page] = 0;
            released.push_back(page);
        }
    }
    for (auto it = released.rbegin(); it != released.rend(); ++it) a->free_pages.push_front(*it);
    return ok();
}

extern "C" int32_t sgl_kv_page_allocator_reset(sgl_kv_page_allocator *a) {
    if (!a) return fail(SGL_KV_INVALID_ARGUMENT, "allocator", 0, 0, 0, "null allocator");
    a->reset();
    return ok();
}

// --- token-prefix cache --------------------------------------------------------------------

// RadixCache (cache.rs:475-547). Nodes live in one vector and name their
// children by index; node 0 is the root, which carries no page.
struct sgl_kv_radix_cache {
    struct Node {
        uint64_t page = 0;
        bool has_page = false;  // Option<CachePageId>: every u64 is a valid page
        std::unordered_map<uint32_t, uint32_t> children;
    };
    std::vector<Node> nodes;

    sgl_kv_radix_cache() { clear(); }
    void clear() {
        nodes.clear();
        nodes.emplace_back();
    }
};

extern "C" int32_t sgl_kv_radix_cache_new(sgl_kv_radix_cache **out) {
    if (!out) return fail(SGL_KV_INVALID_ARGUMENT, "out", 0, 0, 0, "null argument");
    *out = new sgl_kv_radix_cache();
    return ok();
}

extern "C" int32_t sgl_kv_radix_cache_destroy(sgl_kv_radix_cache *cache) {
    delete cache;
    return SGL_KV_OK;
}

extern "C" int32_t sgl_kv_radix_cache_clear(sgl_kv_radix_cache *cache) {
    if (!cache) return fail(SGL_KV_INVALID_ARGUMENT, "cache", 0, 0, 0, "null cache");
    cache->clear();
    return ok();
}

// RadixCache::insert (cache.rs:485-504).
extern "C" int32_t sgl_kv_radix_cache_insert(sgl_kv_radix_cache *cache, const uint32_t *input_ids,
                                             uint64_t token_count, const uint64_t *cache_pages,
                                             uint64_t cache_page_count) {
    if (!cache) return fail(SGL_KV_INVALID_ARGUMENT, "cache", 0, 0, 0, "null cache");
    if (token_count != cache_page_count)
        return fail(SGL_KV_RADIX_TOKEN_PAGE_LENGTH_MISMATCH, nullptr, token_count, cache_page_count, 0,
                    "token count (%llu) must match cache page count (%llu)", (unsigned long long)token_count,
                    (unsigned long long)cache_page_count);
    if (token_count && (!input_ids || !cache_pages))
        return fail(SGL_KV_INVALID_ARGUMENT, "input_ids/cache_pages", 0, 0, 0, "null argument");
    if (cache->nodes.size() + token_count > UINT32_MAX)
        return too_large_dim("radix_cache_nodes", cache->nodes.size() + token_count, UINT32_MAX);
    uint32_t node = 0;
    for (uint64_t i = 0; i < token_count; ++i) {
        auto it = cache->nodes[node].children.find(input_ids[i]);
        uint32_t child;
        if (it == cache->nodes[node].children.end()) {
            child = static_cast<uint32_t>(cache->nodes.size());
            cache->nodes[node].children.emplace(input_ids[i], child);
            cache->nodes.emplace_back();  // may move the vector: index, not reference, above
        } else {
            child = it->second;
        }
        cache->nodes[child].page = cache_pages[i];
        cache->nodes[child].has_page = true;
        node = child;
    }
    return ok();
}

// RadixCache::match_prefix (cache.rs:506-530): follow the prompt down the
// trie while the next token has a node and that node a page; with page_size
// > 1, match_prefix_page_aligned (:532-540) keeps the whole pages of it.
extern "C" int32_t sgl_kv_radix_cache_match_prefix(const sgl_kv_radix_cache *cache, const uint32_t *input_ids,
                                                   uint64_t token_count, uint64_t page_size,
                                                   uint64_t *matched_token_count, uint64_t *out_cache_pages) {
    if (!cache || !matched_token_count)
        return fail(SGL_KV_INVALID_ARGUMENT, "cache/matched_token_count", 0, 0, 0, "null argument");
    *matched_token_count = 0;
    if (page_size == 0)
        return fail(SGL_KV_INVALID_ARGUMENT, "page_size", 0, 0, 0, "KV cache page size must be non-zero");
    if (token_count && (!input_ids || !out_cache_pages))
        return fail(SGL_KV_INVALID_ARGUMENT, "input_ids/out_cache_pages", 0, 0, 0, "null argument");
    uint64_t m = 0;
    uint32_t node = 0;
    while (m < token_count) {
        const auto &children = cache->nodes[node].children;
        auto it = children.find(input_ids[m]);
        if (it == children.end()) break;
        const auto &child = cache->nodes[it->second];
        if (!child.has_page) break;
        out_cache_pages[m++] = child.page;
        node = it->second;
    }
    *matched_token_count = m / page_size * page_size;
    return ok();
}

// --- transfer plan from a prefill batch ----------------------------------------------------

// KvCacheTransferPlan::from_prefill_worker_batch_with_page_size
// (transfer.rs:604-668) over the batch's plan fields; each span's page
// indices come from transfer_page_indices (:679-720).
extern "C" int32_t sgl_kv_transfer_plan_from_prefill_batch(const sgl_kv_prefill_batch *batch,
                                                           uint64_t page_size, sgl_kv_plan_span *spans,
                                                           uint64_t span_capacity, uint64_t *page_indices,
                                                           uint64_t page_index_capacity, uint64_t *span_count,
                                                           uint64_t *page_index_count) {
    if (!batch || !span_count || !page_index_count)
        return fail(SGL_KV_INVALID_ARGUMENT, "batch/span_count/page_index_count", 0, 0, 0, "null argument");
    *span_count = *page_index_count = 0;
    if (batch->forward_mode != SGL_KV_FORWARD_PREFILL)
        return fail(SGL_KV_PLAN_NON_PREFILL_BATCH, nullptr, 0, 0, 0, "KV transfer plan requires prefill batch");
    if (page_size == 0)
        return fail(SGL_KV_PLAN_ZERO_PAGE_SIZE, nullptr, 0, 0, 0, "KV transfer page size must be non-zero");
    const uint64_t n = batch->request_count;
    if (n && (!batch->input_token_counts || !batch->cached_token_counts || !batch->has_disaggregated_params))
        return fail(SGL_KV_INVALID_ARGUMENT, "batch", 0, 0, 0, "null per-request array");
    if (batch->out_cache_page_count && !batch->out_cache_pages)
        return fail(SGL_KV_INVALID_ARGUMENT, "out_cache_pages", 0, 0, 0, "null argument");
    std::vector<sgl_kv_plan_span> out;
    std::vector<uint64_t> pages;
    uint64_t offset = 0;  // the next request's first cache page
    for (uint64_t r = 0; r < n; ++r) {
        const uint64_t count = batch->input_token_counts[r];
        const uint64_t left = batch->out_cache_page_count - offset;
        if (count > left)
            return fail(SGL_KV_PLAN_CACHE_PAGE_COUNT_MISMATCH, nullptr, r, count, left,
                        "request %llu has %llu input tokens but %llu cache pages available",
                        (unsigned long long)r, (unsigned long long)count, (unsigned long long)left);
        const uint64_t first = offset;
        offset += count;
        if (!batch->has_disaggregated_params[r]) continue;
        const uint64_t token_offset = batch->cached_token_counts[r];
        const uint64_t at = pages.size();
        pages.resize(at + count / page_size + (count % page_size ? 1 : 0));
        uint64_t got = 0;
        const int32_t rc = sgl_kv_transfer_page_indices(r, token_offset, batch->out_cache_pages + first, count,
                                                        page_size, pages.data() + at, &got);
        if (rc) return rc;
        pages.resize(at + got);
        out.push_back(sgl_kv_plan_span{r, token_offset, count, first, at, got});
    }
    if (offset != batch->out_cache_page_count)
        return fail(SGL_KV_PLAN_TRAILING_CACHE_PAGES, nullptr, offset, batch->out_cache_page_count, 0,
                    "KV transfer plan consumed %llu cache pages but batch has %llu",
                    (unsigned long long)offset, (unsigned long long)batch->out_cache_page_count);
    if (out.size() > span_capacity || (out.size() && !spans))
        return fail(SGL_KV_INVALID_ARGUMENT, "span_capacity", span_capacity, out.size(), 0,
                    "%llu span entries for %llu spans", (unsigned long long)span_capacity,
                    (unsigned long long)out.size());
    if (pages.size() > page_index_capacity || (pages.size() && !page_indices))
        return fail(SGL_KV_INVALID_ARGUMENT, "page_index_capacity", page_index_capacity, pages.size(), 0,
                    "%llu page-index entries for %llu pages", (unsigned long long)page_index_capacity,
                    (unsigned long long)pages.size());
    if (!out.empty()) memcpy(spans, out.data(), out.size() * sizeof(sgl_kv_plan_span));
    if (!pages.empty()) memcpy(page_indices, pages.data(), pages.size() * sizeof(uint64_t));
    *span_count = out.size();
    *page_index_count = pages.size();
    return ok();
}

// --- SHA-256 (FIPS 180-4) ---------------------------------------------------------------------

namespace {

class Sha256 {
  public:
    Sha256() {
        static const uint32_t init[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a,
                                         0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
        memcpy(h_, init, sizeof h_);
    }

    void update(const void *data, size_t len) {
        const uint8_t *p = static_cast<const uint8_t *>(data);
        total_ += len;
        while (len) {
            const size_t take = len < 64 - fill_ ? len : 64 - fill_;
            memcpy(block_ + fill_, p, take);
            fill_ += take;
            p += take;
            len -= take;
            if (fill_ == 64) {
                compress(block_);
                fill_ = 0;
            }
        }
    }

    void u64le(uint64_t v) {
        uint8_t b[8];
        for (int i = 0; i < 8; ++i) b[i] = (uint8_t)(v >> (8 * i));
        update(b, 8);
    }

    void hex(char out[65]) {
        const uint64_t bits = total_ * 8;
        const uint8_t one = 0x80, zero = 0;
        update(&one, 1);
        while (fill_ != 56) update(&zero, 1);
        uint8_t len_be[8];
        for (int i = 0; i < 8; ++i) len_be[i] = (uint8_t)(bits >> (56 - 8 * i));
        update(len_be, 8);
        static const char digits[] = "0123456789abcdef";
        for (int i = 0; i < 8; ++i)
            for (int j = 0; j < 4; ++j) {
                const uint8_t byte = (uint8_t)(h_[i] >> (24 - 8 * j));
                out[8 * i + 2 * j] = digits[byte >> 4];
                out[8 * i + 2 * j + 1] = digits[byte & 15];
            }
        out[64] = '\0';
    }

  private:
    static uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

    void compress(const uint8_t *b) {
        // First 32 bits of the fractional parts of the cube roots of the
        // first 64 primes (FIPS 180-4, 4.2.2).
        static const uint32_t k[64] = {
            0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4,
            0xab1c5ed5, 0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe,
            0x9bdc06a7, 0xc19bf174, 0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f,
            0x4a7484aa, 0x5cb0a9dc, 0x76f988da, 0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7,
            0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967, 0x27b70a85, 0x2e1b2138, 0x4d2c6dfc,
            0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85, 0xa2bfe8a1, 0xa81a664b,
            0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070, 0x19a4c116,
            0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
            0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7,
            0xc67178f2};
        uint32_t w[64];
        for (int i = 0; i < 16; ++i)
            w[i] = (uint32_t)b[4 * i] << 24 | (uint32_t)b[4 * i + 1] << 16 | (uint32_t)b[4 * i + 2] << 8 |
                   b[4 * i + 3];
        for (int i = 16; i < 64; ++i) {
            const uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
            const uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
            w[i] = w[i - 16] + s0 + w[i - 7] + s1;
        }
        uint32_t a = h_[0], bb = h_[1], c = h_[2], d = h_[3], e = h_[4], f = h_[5], g = h_[6], h = h_[7];
        for (int i = 0; i < 64; ++i) {
            const uint32_t t1 = h + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) + k[i] + w[i];
            const uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & bb) ^ (a & c) ^ (bb & c));
            h = g;
            g = f;
            f = e;
            e = d + t1;
            d = c;
            c = bb;
            bb = a;
            a = t1 + t2;
        }
        h_[0] += a;
        h_[1] += bb;
        h_[2] += c;
        h_[3] += d;
        h_[4] += e;
        h_[5] += f;
        h_[6] += g;
        h_[7] += h;
    }

    uint32_t h_[8];
    uint8_t block_[64];
    size_t fill_ = 0;
    uint64_t total_ = 0;
};

}  // namespace

extern "C" int32_t sgl_kv_sha256_hex(const void *data, uint64_t len, char out_hex[65]) {
    if (!out_hex || (len && !data)) return fail(SGL_KV_INVALID_ARGUMENT, "data/out_hex", 0, 0, 0, "null argument");
    Sha256 s;
    s.update(data, len);
    s.hex(out_hex);
    return ok();
}

// KvCacheTransferSpan::descriptor_checksum (transfer.rs:548-570): SHA-256 of
// a version tag, the length-prefixed request id and bootstrap host, the
// bootstrap port (u16 LE) and room (u64 LE), the DP rank (i32 LE), the
// token offset, token count and page size (u64 LE), then the cache slots and
// the page indices, each list prefixed by its length (u64 LE).
extern "C" int32_t sgl_kv_transfer_span_checksum(
    const char *request_id, uint64_t request_id_len, const char *bootstrap_host,
    uint64_t bootstrap_host_len, uint16_t bootstrap_port, uint64_t bootstrap_room,
    int32_t data_parallel_rank, uint64_t token_offset, uint64_t token_count, uint64_t page_size,
    const uint64_t *cache_pages, uint64_t cache_page_count, const uint64_t *page_indices,
    uint64_t page_index_count, char out_hex[65]) {
    if (!out_hex || (request_id_len && !request_id) || (bootstrap_host_len && !bootstrap_host) ||
        (cache_page_count && !cache_pages) || (page_index_count && !page_indices))
        return fail(SGL_KV_INVALID_ARGUMENT, "checksum input", 0, 0, 0, "null argument");
    Sha256 s;
    static const char tag[] = "sglang-rs.kv-transfer-span.v2";
    s.update(tag, sizeof tag);  // includes the terminating NUL, as the reference hashes it
    s.u64le(request_id_len);
    s.update(request_id, request_id_len);
    s.u64le(bootstrap_host_len);
    s.update(bootstrap_host, bootstrap_host_len);
    const uint8_t port[2] = {(uint8_t)(bootstrap_port & 0xFF), (uint8_t)(bootstrap_port >> 8)};
    s.update(port, 2);
    s.u64le(bootstrap_room);
    const uint32_t rank = (uint32_t)data_parallel_rank;
    const uint8_t rank_le[4] = {(uint8_t)rank, (uint8_t)(rank >> 8), (uint8_t)(rank >> 16),
                                (uint8_t)(rank >> 24)};
    s.update(rank_le, 4);
    s.u64le(token_offset);
    s.u64le(token_count);
    s.u64le(page_size);
    s.u64le(cache_page_count);
    for (uint64_t i = 0; i < cache_page_count; ++i) s.u64le(cache_pages[i]);
    s.u64le(page_index_count);
    for (uint64_t i = 0; i < page_index_count; ++i) s.u64le(page_indices[i]);
    s.hex(out_hex);
    return ok();
}
