// Host-only driver for the layout / plan mirror (kv_layout.cpp), built with
// AddressSanitizer and UndefinedBehaviorSanitizer by tests/test_host_sanitizers.py.
// It replays the reference goldens, then fuzzes every group-1 entry point
// with small, boundary and overflowing values and checks what must hold for
// any accepted input: every byte range lies inside the pool and the plan's
// required sizes cover the last row and the last slot.
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <random>
#include <vector>

#include "sgl_rocm_kv.h"

static int failures = 0;
#define CHECK(cond)                                                        \
    do {                                                                   \
        if (!(cond)) {                                                     \
            fprintf(stderr, "CHECK failed at line %d: %s\n", __LINE__, #cond); \
            ++failures;                                                    \
        }                                                                  \
    } while (0)

static uint64_t pick(std::mt19937_64 &rng) {
    switch (rng() % 8) {
    case 0: return 0;
    case 1: return 1 + rng() % 4;
    case 2: return 1 + rng() % 256;
    case 3: return 1ull << (rng() % 64);
    case 4: return UINT64_MAX - rng() % 4;
    case 5: return rng();
    case 6: return (1ull << 32) + rng() % 8;
    default: return 2 * (1 + rng() % 64);
    }
}

int main() {
    // Goldens: crates/sglang-srt/tests/kv_cache.rs:51-217.
    sgl_kv_runtime_layout rt;
    memset(&rt, 0, sizeof rt);
    rt.dtype = SGL_KV_DTYPE_BFLOAT16;
    rt.page_size = 4;
    rt.num_layers = 2;
    rt.kv_heads = 2;
    rt.head_dim = 8;
    rt.kv_tensors_per_token = 2;
    rt.bytes_per_token = 128;
    rt.page_size_bytes = 512;
    sgl_kv_paged_layout l;
    CHECK(sgl_kv_paged_layout_new(&rt, 3, &l) == SGL_KV_OK);
    uint64_t s = 0, e = 0;
    CHECK(sgl_kv_paged_layout_tensor_token_byte_range(&l, 1, 1, 1, 3, &s, &e) == SGL_KV_OK);
    CHECK(s == 992 && e == 1024);
    CHECK(sgl_kv_paged_layout_tensor_slot_byte_range(&l, 1, 1, 12, &s, &e) ==
          SGL_KV_LAYOUT_SLOT_OUT_OF_RANGE);
    sgl_kv_pair_copy_layout pl = {4, 512, 256, 384, 32};
    sgl_kv_pair_copy_plan plan;
    CHECK(sgl_kv_pair_copy_plan_new(3, 12, &pl, 40, 48, &plan) == SGL_KV_OK);
    CHECK(plan.key_rows_required_bytes == 112 && plan.pool_required_bytes == 1536);

    std::mt19937_64 rng(20261201);
    for (int it = 0; it < 200000; ++it) {
        sgl_kv_runtime_layout r;
        memset(&r, 0, sizeof r);
        r.dtype = (int32_t)(rng() % 6);
        r.page_size = pick(rng);
        r.num_layers = pick(rng);
        r.kv_heads = pick(rng);
        r.head_dim = pick(rng);
        r.kv_tensors_per_token = rng() % 2 ? 2 : pick(rng);
        // Mostly self-consistent runtimes so that the range functions run.
        if (rng() % 4) {
            r.bytes_per_token = r.num_layers * r.kv_tensors_per_token * (1 + rng() % 64);
            r.page_size_bytes = r.page_size * r.bytes_per_token;
        } else {
            r.bytes_per_token = pick(rng);
            r.page_size_bytes = pick(rng);
        }
        const uint64_t pages = pick(rng);
        sgl_kv_paged_layout lay;
        int32_t rc;
        if (rng() % 3)
            rc = sgl_kv_paged_layout_new(&r, pages, &lay);
        else
            rc = sgl_kv_paged_layout_new_with_tensor_pair(&r, pages, pick(rng), pick(rng), &lay);
        if (rc != SGL_KV_OK) continue;
        for (int k = 0; k < 8; ++k) {
            const uint64_t layer = rng() % 2 ? rng() % (r.num_layers + 1) : pick(rng);
            const uint64_t tensor = rng() % 3;
            const uint64_t slot = rng() % 2 ? rng() % (lay.slot_count + 2) : pick(rng);
            if (sgl_kv_paged_layout_tensor_slot_byte_range(&lay, layer, tensor, slot, &s, &e) ==
                SGL_KV_OK) {
                CHECK(s < e);
                CHECK(e <= lay.total_byte_len);
                CHECK(slot < lay.slot_count && layer < r.num_layers);
            }
            sgl_kv_pair_copy_layout g;
            if (sgl_kv_paged_layout_kv_pair_copy_geometry(&lay, layer, &g) == SGL_KV_OK) {
                CHECK(g.key_in_page_offset + g.page_size * g.row_bytes <= g.page_stride_bytes);
                CHECK(g.value_in_page_offset + g.page_size * g.row_bytes <= g.page_stride_bytes);
            }
        }
    }

    for (int it = 0; it < 200000; ++it) {
        sgl_kv_pair_copy_layout g = {pick(rng), pick(rng), pick(rng), pick(rng), pick(rng)};
        const uint64_t rows = pick(rng), slots = pick(rng), ks = pick(rng), vs = pick(rng);
        sgl_kv_pair_copy_plan p;
        if (sgl_kv_pair_copy_plan_new(rows, slots, &g, ks, vs, &p) != SGL_KV_OK) continue;
        // Every accepted plan covers its last row and its last slot.
        CHECK(p.key_rows_required_bytes >= g.row_bytes && p.value_rows_required_bytes >= g.row_bytes);
        CHECK(p.slot_indices_required_bytes == rows * 8);
        const uint64_t last = slots - 1;
        const uint64_t key_end = (last / g.page_size) * g.page_stride_bytes + g.key_in_page_offset +
                                 (last % g.page_size + 1) * g.row_bytes;
        const uint64_t val_end = (last / g.page_size) * g.page_stride_bytes +
                                 g.value_in_page_offset + (last % g.page_size + 1) * g.row_bytes;
        CHECK(p.pool_required_bytes >= key_end && p.pool_required_bytes >= val_end);
    }

    for (int it = 0; it < 100000; ++it) {
        const uint64_t page_size = rng() % 5;
        std::vector<uint64_t> cache(rng() % 12);
        uint64_t base = (rng() % 6) * (page_size ? page_size : 1);
        for (size_t i = 0; i < cache.size(); ++i) cache[i] = rng() % 8 ? base + i : rng() % 64;
        std::vector<uint64_t> out(cache.size() + 1);
        uint64_t n = 0;
        const int32_t rc = sgl_kv_transfer_page_indices(0, (rng() % 3) * 2, cache.data(), cache.size(),
                                                        page_size, out.data(), &n);
        if (rc == SGL_KV_OK) CHECK(n <= cache.size());
    }
    // Page allocator under random traffic: allocations never overlap live
    // slots and stay in range; the allocator never leaks or double-frees.
    for (int round = 0; round < 20; ++round) {
        const uint64_t P = 1 + rng() % 16, pages = 1 + rng() % 64;
        sgl_kv_page_allocator *a = nullptr;
        CHECK(sgl_kv_page_allocator_new(P * pages, P, &a) == SGL_KV_OK);
        std::vector<std::vector<uint64_t>> live;
        std::vector<uint8_t> used(P * pages, 0);
        for (int it = 0; it < 2000; ++it) {
            if (!live.empty() && rng() % 3 == 0) {
                const size_t v = rng() % live.size();
                for (uint64_t slot : live[v]) used[slot] = 0;
                CHECK(sgl_kv_page_allocator_release(a, live[v].data(), live[v].size()) == SGL_KV_OK);
                live.erase(live.begin() + v);
                continue;
            }
            const uint64_t n = 1 + rng() % (3 * P);
            std::vector<uint64_t> out(n);
            const int32_t rc = sgl_kv_page_allocator_allocate_for_sequence(a, nullptr, 0, n, out.data());
            if (rc != SGL_KV_OK) {
                CHECK(rc == SGL_KV_ALLOC_OUT_OF_SLOTS);
                continue;
            }
            for (uint64_t slot : out) {
                CHECK(slot < P * pages && !used[slot]);
                used[slot] = 1;
            }
            live.push_back(out);
        }
        // release garbage, then everything
        const uint64_t junk[4] = {UINT64_MAX, P * pages, 1, P * pages + P};
        CHECK(sgl_kv_page_allocator_release(a, junk, 4) == SGL_KV_OK);
        for (auto &v : live) sgl_kv_page_allocator_release(a, v.data(), v.size());
        CHECK(sgl_kv_page_allocator_available_pages(a) <= pages);
        sgl_kv_page_allocator_destroy(a);
    }
    char hex[65];
    const uint64_t pages2[2] = {0, 1};
    CHECK(sgl_kv_transfer_span_checksum("http-pd-poll", 12, "10.0.0.8", 8, 8200, 42, 0, 0, 2, 1, pages2, 2,
                                        pages2, 2, hex) == SGL_KV_OK);
    CHECK(strcmp(hex, "e37f348404de723244ca004c09d05fccfdcad793f9013bd1f882c332d1c50b5d") == 0);
    std::vector<uint8_t> blob(5000);
    for (auto &x : blob) x = (uint8_t)rng();
    for (size_t n = 0; n < blob.size(); n += 1 + rng() % 97)
        CHECK(sgl_kv_sha256_hex(blob.data(), n, hex) == SGL_KV_OK && strlen(hex) == 64);

    // The token-prefix cache under random inserts and matches: a match never
    // exceeds the query, is a multiple of the page size, and reports pages
    // for exactly the matched tokens (the rest of out_pages is untouched).
    {
        sgl_kv_radix_cache *c = nullptr;
        CHECK(sgl_kv_radix_cache_new(&c) == SGL_KV_OK);
        for (int it = 0; it < 3000; ++it) {
            const uint64_t n = rng() % 24;
            std::vector<uint32_t> toks(n);
            std::vector<uint64_t> pages(n);
            for (uint64_t i = 0; i < n; ++i) {
                toks[i] = (uint32_t)(rng() % 3);
                pages[i] = pick(rng);
            }
            if (rng() % 3 == 0) {
                CHECK(sgl_kv_radix_cache_insert(c, toks.data(), n, pages.data(), n) == SGL_KV_OK);
                if (n) CHECK(sgl_kv_radix_cache_insert(c, toks.data(), n, pages.data(), n - 1) ==
                             SGL_KV_RADIX_TOKEN_PAGE_LENGTH_MISMATCH);
            } else {
                const uint64_t P = rng() % 5;
                std::vector<uint64_t> out(n + 1, 0xA5A5A5A5A5A5A5A5ull);
                uint64_t m = UINT64_MAX;
                const int32_t rc = sgl_kv_radix_cache_match_prefix(c, toks.data(), n, P, &m, out.data());
                if (P == 0) {
                    CHECK(rc == SGL_KV_INVALID_ARGUMENT && m == 0);
                } else {
                    CHECK(rc == SGL_KV_OK && m <= n && m % P == 0);
                    CHECK(out[n] == 0xA5A5A5A5A5A5A5A5ull);
                }
            }
            if (rng() % 500 == 0) CHECK(sgl_kv_radix_cache_clear(c) == SGL_KV_OK);
        }
        sgl_kv_radix_cache_destroy(c);
    }
    // The prefill-batch plan on random (mostly malformed) batches: it returns
    // a status and never writes past the capacities it was given.
    for (int it = 0; it < 3000; ++it) {
        const uint64_t reqs = rng() % 6, P = rng() % 5;
        std::vector<uint64_t> inputs(reqs), cached(reqs);
        std::vector<uint8_t> pd(reqs);
        uint64_t total = 0;
        for (uint64_t r = 0; r < reqs; ++r) {
            inputs[r] = rng() % 3 == 0 ? pick(rng) : rng() % 9;
            cached[r] = rng() % 2 ? (P ? P * (rng() % 3) : 0) : pick(rng);
            pd[r] = (uint8_t)(rng() % 2);
            if (inputs[r] < 64) total += inputs[r];
        }
        std::vector<uint64_t> slots(total + rng() % 3);
        for (uint64_t i = 0; i < slots.size(); ++i) slots[i] = rng() % 2 ? i : pick(rng);
        sgl_kv_prefill_batch b = {(int32_t)(rng() % 4 == 0), reqs, inputs.data(), cached.data(),
                                  pd.data(), slots.data(), slots.size()};
        const uint64_t span_cap = rng() % (reqs + 2), page_cap = rng() % (slots.size() + 3);
        std::vector<sgl_kv_plan_span> spans(span_cap + 1);
        std::vector<uint64_t> idx(page_cap + 1, 77);
        spans[span_cap].request_index = 99;
        uint64_t ns = 5, ni = 5;
        const int32_t rc = sgl_kv_transfer_plan_from_prefill_batch(&b, P, spans.data(), span_cap, idx.data(),
                                                                   page_cap, &ns, &ni);
        CHECK(rc == SGL_KV_OK ? ns <= span_cap && ni <= page_cap : ns == 0 && ni == 0);
        CHECK(spans[span_cap].request_index == 99 && idx[page_cap] == 77);
    }

    if (failures) {
        fprintf(stderr, "%d checks failed\n", failures);
        return 1;
    }
    printf("layout fuzz ok\n");
    return 0;
}
