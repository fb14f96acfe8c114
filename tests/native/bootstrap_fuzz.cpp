// Host-only driver for the bootstrap wire format (kv_bootstrap.cpp), built
// with AddressSanitizer and UndefinedBehaviorSanitizer by
// tests/test_host_sanitizers.py. Three parts:
//  1. encoder -> decoder round trip over random valid records: every field
//     read back equals the one written;
//  2. mutations of valid frames (truncated, extended, flipped bytes, parts
//     dropped or added) and fully random frames go through ingest: no
//     access outside the parts, and an accepted frame yields views whose
//     counts and offsets are consistent;
//  3. the state keeps its invariants (a room's status is WaitingForInput
//     exactly when it once held required_dst_info_num sessions).
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <random>
#include <string>
#include <vector>

#include "sgl_rocm_kv.h"

static int failures = 0;
#define CHECK(cond)                                                            \
    do {                                                                       \
        if (!(cond)) {                                                         \
            fprintf(stderr, "CHECK failed at line %d: %s\n", __LINE__, #cond); \
            ++failures;                                                        \
        }                                                                      \
    } while (0)

typedef std::vector<std::vector<uint8_t>> Frame;

static Frame to_frame(const std::vector<uint8_t> &buf, const sgl_kv_frame_part *parts, uint32_t n) {
    Frame f;
    for (uint32_t i = 0; i < n; ++i) f.emplace_back(parts[i].data, parts[i].data + parts[i].len);
    (void)buf;
    return f;
}

// Ingests a frame through parts that point at exactly-sized heap copies, so
// that ASan sees any read past a part.
static int32_t ingest(sgl_kv_bootstrap *s, const Frame &f) {
    std::vector<uint8_t *> copies;
    std::vector<sgl_kv_frame_part> parts;
    for (const auto &p : f) {
        uint8_t *c = p.empty() ? nullptr : (uint8_t *)malloc(p.size());
        if (c) memcpy(c, p.data(), p.size());
        copies.push_back(c);
        parts.push_back({c, p.size()});
    }
    const int32_t rc = sgl_kv_bootstrap_ingest(s, parts.data(), (uint32_t)parts.size());
    for (uint8_t *c : copies) free(c);
    return rc;
}

static std::string rand_text(std::mt19937_64 &rng) {
    std::string s;
    const int n = (int)(rng() % 12) + 1;
    for (int i = 0; i < n; ++i) s.push_back((char)('a' + rng() % 26));
    return s;
}

template <typename T>
static void rand_lists(std::mt19937_64 &rng, std::vector<T> &values, std::vector<uint64_t> &offsets) {
    values.clear();
    offsets.assign(1, 0);
    const int lists = (int)(rng() % 4);
    for (int i = 0; i < lists; ++i) {
        const int n = (int)(rng() % 4);
        for (int k = 0; k < n; ++k) values.push_back((T)rng());
        offsets.push_back(values.size());
    }
}

static void check_views(sgl_kv_bootstrap *s, const char *session) {
    sgl_kv_bootstrap_kv_args a;
    if (sgl_kv_bootstrap_get_kv_args(s, session, &a) != SGL_KV_OK) return;
    volatile uint64_t sink = 0;
    for (uint64_t i = 0; i < a.dst_kv_ptr_count; ++i) sink += a.dst_kv_ptrs[i];
    for (uint64_t i = 0; i < a.dst_aux_ptr_count; ++i) sink += a.dst_aux_ptrs[i];
    const sgl_kv_u64_lists &l = a.dst_state_data_ptrs;
    for (uint64_t i = 0; i < l.count; ++i) {
        CHECK(l.offsets[i] <= l.offsets[i + 1]);
        for (uint64_t k = l.offsets[i]; k < l.offsets[i + 1]; ++k) sink += l.values[k];
    }
    (void)sink;
}

int main() {
    std::mt19937_64 rng(20261201);
    sgl_kv_bootstrap *s = nullptr;
    CHECK(sgl_kv_bootstrap_create(&s) == SGL_KV_OK);
    std::vector<Frame> valid;

    // 1. round trips
    for (int it = 0; it < 3000; ++it) {
        const std::string endpoint = rand_text(rng), session = rand_text(rng);
        std::vector<uint64_t> kv_ptrs(rng() % 5), aux(rng() % 3);
        for (auto &v : kv_ptrs) v = rng();
        for (auto &v : aux) v = rng();
        std::vector<uint64_t> sd, sdo, ilo, dio;
        std::vector<uint32_t> il, di;
        rand_lists(rng, sd, sdo);
        rand_lists(rng, il, ilo);
        rand_lists(rng, di, dio);
        sgl_kv_bootstrap_kv_args a;
        memset(&a, 0, sizeof a);
        a.endpoint = endpoint.c_str();
        a.mooncake_session_id = session.c_str();
        a.dst_port = (uint32_t)(rng() % 65536);
        a.dst_tp_rank = (int32_t)rng();
        a.dst_attn_tp_size = rng();
        a.dst_kv_item_len = rng();
        a.dst_kv_ptrs = kv_ptrs.data();
        a.dst_kv_ptr_count = kv_ptrs.size();
        a.dst_aux_ptrs = aux.data();
        a.dst_aux_ptr_count = aux.size();
        a.dst_state_data_ptrs = {sd.data(), sdo.data(), sdo.size() - 1};
        a.dst_state_item_lens = {il.data(), ilo.data(), ilo.size() - 1};
        a.dst_state_dim_per_tensor = {di.data(), dio.data(), dio.size() - 1};
        uint64_t need = 0;
        uint32_t n = 0;
        sgl_kv_frame_part parts[SGL_KV_BOOTSTRAP_MAX_PARTS];
        CHECK(sgl_kv_bootstrap_encode_kv_args(&a, nullptr, 0, parts, &n, &need) == SGL_KV_OK);
        std::vector<uint8_t> buf(need + 1);
        CHECK(sgl_kv_bootstrap_encode_kv_args(&a, buf.data(), need, parts, &n, &need) == SGL_KV_OK);
        const Frame f = to_frame(buf, parts, n);
        CHECK(ingest(s, f) == SGL_KV_OK);
        sgl_kv_bootstrap_kv_args b;
        CHECK(sgl_kv_bootstrap_get_kv_args(s, session.c_str(), &b) == SGL_KV_OK);
        CHECK(b.dst_port == a.dst_port && b.dst_tp_rank == a.dst_tp_rank);
        CHECK(b.dst_attn_tp_size == a.dst_attn_tp_size && b.dst_kv_item_len == a.dst_kv_item_len);
        CHECK(b.dst_kv_ptr_count == kv_ptrs.size() && b.dst_aux_ptr_count == aux.size());
        for (size_t i = 0; i < kv_ptrs.size(); ++i) CHECK(b.dst_kv_ptrs[i] == kv_ptrs[i]);
        CHECK(b.dst_state_data_ptrs.count == sdo.size() - 1 && b.dst_state_item_lens.count == ilo.size() - 1);
        for (size_t i = 0; i < sd.size(); ++i) CHECK(b.dst_state_data_ptrs.values[i] == sd[i]);
        for (size_t i = 0; i < sdo.size(); ++i) CHECK(b.dst_state_data_ptrs.offsets[i] == sdo[i]);
        for (size_t i = 0; i < di.size(); ++i) CHECK(b.dst_state_dim_per_tensor.values[i] == di[i]);
        valid.push_back(f);

        std::vector<int32_t> idx(rng() % 6);
        for (auto &v : idx) v = (int32_t)rng();
        std::vector<int32_t> st;
        std::vector<uint64_t> sto;
        rand_lists(rng, st, sto);
        sgl_kv_bootstrap_transfer t;
        memset(&t, 0, sizeof t);
        t.room = rng() >> 1;
        t.endpoint = endpoint.c_str();
        t.mooncake_session_id = session.c_str();
        t.dst_port = a.dst_port;
        t.is_dummy = rng() % 5 == 0;
        t.dst_kv_indices = idx.data();
        t.dst_kv_index_count = idx.size();
        t.has_dst_aux_index = 1;
        t.dst_aux_index = (int32_t)rng();
        t.dst_state_indices = {st.data(), sto.data(), sto.size() - 1};
        t.required_dst_info_num = 1 + rng() % 3;
        t.has_decode_prefix_len = rng() % 2;
        t.decode_prefix_len = rng() >> 1;
        CHECK(sgl_kv_bootstrap_encode_transfer(&t, nullptr, 0, parts, &n, &need) == SGL_KV_OK);
        buf.assign(need + 1, 0);
        CHECK(sgl_kv_bootstrap_encode_transfer(&t, buf.data(), need, parts, &n, &need) == SGL_KV_OK);
        const Frame tf = to_frame(buf, parts, n);
        CHECK(ingest(s, tf) == SGL_KV_OK);
        sgl_kv_bootstrap_transfer u;
        CHECK(sgl_kv_bootstrap_get_transfer(s, t.room, session.c_str(), &u) == SGL_KV_OK);
        CHECK(u.is_dummy == t.is_dummy && u.required_dst_info_num == t.required_dst_info_num);
        if (!t.is_dummy) {
            CHECK(u.dst_kv_index_count == idx.size() && u.dst_aux_index == t.dst_aux_index);
            for (size_t i = 0; i < idx.size(); ++i) CHECK(u.dst_kv_indices[i] == idx[i]);
            CHECK(u.dst_state_indices.count == sto.size() - 1);
        }
        CHECK(u.decode_prefix_len == (t.has_decode_prefix_len ? t.decode_prefix_len : 0));
        valid.push_back(tf);
    }

    // 2. mutations and random frames
    for (int it = 0; it < 200000; ++it) {
        Frame f = valid[rng() % valid.size()];
        switch (rng() % 6) {
        case 0:
            if (!f.empty()) f.resize(rng() % f.size());
            break;
        case 1:
            f.push_back(std::vector<uint8_t>(rng() % 20, (uint8_t)rng()));
            break;
        case 2: {
            auto &p = f[rng() % f.size()];
            if (!p.empty()) p[rng() % p.size()] ^= (uint8_t)(1u << (rng() % 8));
            break;
        }
        case 3: {
            auto &p = f[rng() % f.size()];
            p.resize(rng() % (p.size() + 9), (uint8_t)rng());
            break;
        }
        case 4: {
            auto &p = f[rng() % f.size()];
            p.resize(rng() % 40);
            for (auto &b : p) b = (uint8_t)rng();
            break;
        }
        default: {
            f.assign(rng() % 17, {});
            for (auto &p : f) {
                p.resize(rng() % 24);
                for (auto &b : p) b = (uint8_t)(rng() % 3 == 0 ? '0' + rng() % 10 : rng());
            }
            if (!f.empty() && rng() % 2) f[0] = {'N', 'o', 'n', 'e'};
        }
        }
        const int32_t rc = ingest(s, f);
        CHECK(rc == SGL_KV_OK || (rc >= SGL_KV_BOOT_MISSING_FIELD && rc <= SGL_KV_BOOT_DECODE_LAYOUT) ||
              (rc >= SGL_KV_LAYOUT_ZERO_PAGE_COUNT && rc <= SGL_KV_LAYOUT_UNEVEN_KV_PAIR_COPY) ||
              rc == SGL_KV_INVALID_ARGUMENT);
        if (rc == SGL_KV_OK && f.size() > 3) {
            const std::string session(f[3].begin(), f[3].end());
            check_views(s, session.c_str());
        }
    }

    // 3. room invariants on a fresh state
    sgl_kv_bootstrap *r = nullptr;
    CHECK(sgl_kv_bootstrap_create(&r) == SGL_KV_OK);
    for (int it = 0; it < 2000; ++it) {
        const uint64_t room = rng() % 50;
        const std::string session = "s" + std::to_string(rng() % 4);
        const uint64_t required = 1 + rng() % 4;
        const std::string ep = "e";
        int32_t idx[1] = {1};
        sgl_kv_bootstrap_transfer t;
        memset(&t, 0, sizeof t);
        t.room = room;
        t.endpoint = ep.c_str();
        t.mooncake_session_id = session.c_str();
        t.dst_kv_indices = idx;
        t.dst_kv_index_count = 1;
        t.has_dst_aux_index = 1;
        t.required_dst_info_num = required;
        sgl_kv_frame_part parts[SGL_KV_BOOTSTRAP_MAX_PARTS];
        uint64_t need = 0;
        uint32_t n = 0;
        std::vector<uint8_t> buf(256);
        CHECK(sgl_kv_bootstrap_encode_transfer(&t, buf.data(), buf.size(), parts, &n, &need) == SGL_KV_OK);
        int32_t before = 0;
        CHECK(sgl_kv_bootstrap_transfer_status(r, room, &before) == SGL_KV_OK);
        CHECK(sgl_kv_bootstrap_ingest(r, parts, n) == SGL_KV_OK);
        uint64_t req = 0, sessions = 0, prefix = 0;
        uint32_t has = 0;
        int32_t after = 0;
        CHECK(sgl_kv_bootstrap_room(r, room, &req, &has, &prefix, &sessions) == SGL_KV_OK);
        CHECK(sgl_kv_bootstrap_transfer_status(r, room, &after) == SGL_KV_OK);
        CHECK(req == required && has == 1 && prefix == 0);
        // WaitingForInput once reached is kept; otherwise it follows the count.
        if (before == 2) CHECK(after == 2);
        else CHECK(after == (sessions == required ? 2 : 1));
    }
    sgl_kv_bootstrap_destroy(r);
    sgl_kv_bootstrap_destroy(s);
    if (failures) {
        fprintf(stderr, "%d checks failed\n", failures);
        return 1;
    }
    printf("bootstrap fuzz ok\n");
    return 0;
}
