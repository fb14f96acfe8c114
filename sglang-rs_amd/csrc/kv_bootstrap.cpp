// kv_bootstrap.cpp -- the bootstrap wire format that carries the decode
// side's page table (and, as an extension, its page layout) to the prefill
// side: decoding and ingesting Mooncake bootstrap frames the way
// PrefillBootstrapState does (crates/sglang-srt/src/pd_bootstrap.rs:150-270,
// 416-494, 1421-1636) and encoding them the way the decode publisher does
// (:671-749, 1209-1270). Host only; no GPU call.
#include <stdio.h>
#include <string.h>

#include <map>
#include <new>
#include <string>
#include <vector>

#include "kv_internal.h"

using namespace sglkv;

namespace {

constexpr int32_t kKvPollBootstrapping = 1, kKvPollWaitingForInput = 2;  // transfer.rs:355-361
constexpr uint64_t kI64Max = 0x7FFFFFFFFFFFFFFFull;

template <typename T>
struct Lists {  // a flattened list of lists
    std::vector<T> values;
    std::vector<uint64_t> offsets{0};
    uint64_t count() const { return offsets.size() - 1; }
};

struct KvArgs {
    std::string room, endpoint, session;
    uint16_t dst_port = 0;
    int32_t dst_tp_rank = 0;
    uint64_t dst_attn_tp_size = 0, dst_kv_item_len = 0;
    std::vector<uint64_t> dst_kv_ptrs, dst_aux_ptrs;
    Lists<uint64_t> dst_state_data_ptrs;
    Lists<uint32_t> dst_state_item_lens, dst_state_dim_per_tensor;
    bool has_layout = false;
    sgl_kv_decode_layout layout;
};

struct Transfer {
    uint64_t room = 0;
    std::string endpoint, session;
    uint16_t dst_port = 0;
    bool is_dummy = false;
    std::vector<int32_t> dst_kv_indices;
    bool has_aux = false;
    int32_t aux = 0;
    Lists<int32_t> dst_state_indices;
    uint64_t required = 0;
    bool has_prefix = false;
    uint64_t prefix = 0;
};

struct Room {
    uint64_t required = 0;
    int32_t status = kKvPollBootstrapping;
    bool has_prefix = false;
    uint64_t prefix = 0;
    std::map<std::string, Transfer> transfers;
};

// ---- field access and parsing (pd_bootstrap.rs:1421-1547) ----

struct Frame {
    const sgl_kv_frame_part *parts;
    uint32_t count;
};

int32_t missing_field(const char *frame, uint64_t expected, uint64_t actual) {
    return fail(SGL_KV_BOOT_MISSING_FIELD, frame, expected, actual, 0,
                "%s frame requires at least %llu fields, got %llu", frame, (unsigned long long)expected,
                (unsigned long long)actual);
}

int32_t require_min_fields(const Frame &f, uint32_t expected, const char *frame) {
    return f.count < expected ? missing_field(frame, expected, f.count) : SGL_KV_OK;
}

int32_t field(const Frame &f, uint32_t index, const char *name, const uint8_t **data, uint64_t *len) {
    if (index >= f.count) return missing_field(name, (uint64_t)index + 1, f.count);
    *data = f.parts[index].data;
    *len = f.parts[index].len;
    if (*len && !*data) return fail(SGL_KV_INVALID_ARGUMENT, name, 0, 0, 0, "frame part %s has no data", name);
    return SGL_KV_OK;
}

// std::str::from_utf8: well-formed UTF-8 (no overlong forms, surrogates or
// code points past U+10FFFF).
bool valid_utf8(const uint8_t *s, uint64_t n) {
    uint64_t i = 0;
    while (i < n) {
        const uint8_t c = s[i];
        if (c < 0x80) {
            ++i;
            continue;
        }
        uint32_t need, cp;
        if (c >= 0xC2 && c <= 0xDF) {
            need = 1;
            cp = c & 0x1F;
        } else if (c >= 0xE0 && c <= 0xEF) {
            need = 2;
            cp = c & 0x0F;
        } else if (c >= 0xF0 && c <= 0xF4) {
            need = 3;
            cp = c & 0x07;
        } else {
            return false;
        }
        if (n - i <= need) return false;
        for (uint32_t k = 1; k <= need; ++k) {
            if ((s[i + k] & 0xC0) != 0x80) return false;
            cp = (cp << 6) | (s[i + k] & 0x3F);
        }
        if ((need == 2 && (cp < 0x800 || (cp >= 0xD800 && cp <= 0xDFFF))) ||
            (need == 3 && (cp < 0x10000 || cp > 0x10FFFF)))
            return false;
        i += need + 1;
    }
    return true;
}

int32_t ascii_field(const Frame &f, uint32_t index, const char *name, std::string *out) {
    const uint8_t *d;
    uint64_t n;
    int32_t rc = field(f, index, name, &d, &n);
    if (rc) return rc;
    if (!valid_utf8(d, n)) return fail(SGL_KV_BOOT_UTF8_FIELD, name, 0, 0, 0, "%s must be ASCII/UTF-8", name);
    out->assign(reinterpret_cast<const char *>(d), n);
    return SGL_KV_OK;
}

int32_t integer_error(const char *name, const std::string &value) {
    return fail(SGL_KV_BOOT_INTEGER_FIELD, name, 0, 0, 0, "%s must be an integer, got %.200s", name,
                value.c_str());
}

// The FromStr of Rust's integers: an optional sign ('+', or '-' for signed
// types) then at least one ASCII digit, nothing else, no overflow. The
// magnitude limit is max_pos (or max_neg after a '-').
bool parse_decimal(const std::string &s, bool is_signed, uint64_t max_pos, uint64_t max_neg, bool *negative,
                   uint64_t *magnitude) {
    size_t i = 0;
    *negative = false;
    if (!s.empty() && (s[0] == '+' || (is_signed && s[0] == '-'))) {
        *negative = s[0] == '-';
        i = 1;
    }
    if (i >= s.size()) return false;
    const uint64_t limit = *negative ? max_neg : max_pos;
    uint64_t v = 0;
    for (; i < s.size(); ++i) {
        const char c = s[i];
        if (c < '0' || c > '9') return false;
        if (v > (limit - (uint64_t)(c - '0')) / 10) return false;
        v = v * 10 + (uint64_t)(c - '0');
    }
    *magnitude = v;
    return true;
}

int32_t parse_unsigned(const Frame &f, uint32_t index, const char *name, uint64_t max, uint64_t *out) {
    std::string s;
    int32_t rc = ascii_field(f, index, name, &s);
    if (rc) return rc;
    bool neg;
    if (!parse_decimal(s, false, max, 0, &neg, out)) return integer_error(name, s);
    return SGL_KV_OK;
}

int32_t parse_i32(const Frame &f, uint32_t index, const char *name, int32_t *out) {
    std::string s;
    int32_t rc = ascii_field(f, index, name, &s);
    if (rc) return rc;
    bool neg;
    uint64_t m;
    if (!parse_decimal(s, true, 0x7FFFFFFFull, 0x80000000ull, &neg, &m)) return integer_error(name, s);
    *out = neg ? (int32_t)(0 - (uint32_t)m) : (int32_t)m;
    return SGL_KV_OK;
}

// parse_bootstrap_room (:1474-1495): a u64 no larger than i64::MAX.
int32_t parse_room(const Frame &f, uint32_t index, const char *name, uint64_t *out) {
    std::string s;
    int32_t rc = ascii_field(f, index, name, &s);
    if (rc) return rc;
    bool neg;
    if (!parse_decimal(s, false, UINT64_MAX, 0, &neg, out) || *out > kI64Max) return integer_error(name, s);
    return SGL_KV_OK;
}

// ---- binary fields (:1549-1636) ----

template <typename T>
int32_t unpack_fixed(const uint8_t *d, uint64_t n, const char *name, std::vector<T> *out) {
    if (n % sizeof(T))
        return fail(SGL_KV_BOOT_BINARY_LENGTH, name, sizeof(T), n, 0, "%s byte length %llu must be divisible by %u",
                    name, (unsigned long long)n, (unsigned)sizeof(T));
    out->resize(n / sizeof(T));
    if (n) memcpy(out->data(), d, n);  // little-endian host
    return SGL_KV_OK;
}

uint32_t le32(const uint8_t *p) { return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24; }
uint64_t le64(const uint8_t *p) { return (uint64_t)le32(p) | (uint64_t)le32(p + 4) << 32; }

struct Span {
    const uint8_t *data;
    uint64_t len;
};

int32_t unpack_list_of_buffers(const uint8_t *d, uint64_t n, const char *name, std::vector<Span> *out) {
    out->clear();
    if (n == 0) return SGL_KV_OK;
    if (n < 4) return fail(SGL_KV_BOOT_PACKED_LIST_HEADER, name, 0, 0, 0, "%s packed list header is incomplete", name);
    const uint64_t count = le32(d);
    const uint64_t header = 4 + count * 4;
    if (n < header) return fail(SGL_KV_BOOT_PACKED_LIST_HEADER, name, 0, 0, 0, "%s packed list header is incomplete", name);
    uint64_t offset = header;
    for (uint64_t i = 0; i < count; ++i) {
        const uint64_t len = le32(d + 4 + 4 * i);
        if (n - offset < len)
            return fail(SGL_KV_BOOT_PACKED_LIST_LENGTH, name, 0, 0, 0, "%s packed list payload is incomplete", name);
        out->push_back(Span{d + offset, len});
        offset += len;
    }
    return SGL_KV_OK;
}

template <typename T>
int32_t unpack_lists(const uint8_t *d, uint64_t n, const char *list_name, const char *value_name, Lists<T> *out) {
    std::vector<Span> bufs;
    int32_t rc = unpack_list_of_buffers(d, n, list_name, &bufs);
    if (rc) return rc;
    *out = Lists<T>();
    std::vector<T> one;
    for (const Span &b : bufs) {
        if ((rc = unpack_fixed<T>(b.data, b.len, value_name, &one))) return rc;
        out->values.insert(out->values.end(), one.begin(), one.end());
        out->offsets.push_back(out->values.size());
    }
    return SGL_KV_OK;
}

// ---- the decode-layout extension ----

int32_t layout_error(const char *what, uint64_t a, uint64_t b) {
    return fail(SGL_KV_BOOT_DECODE_LAYOUT, what, a, b, 0, "decode layout extension: %s (%llu, %llu)", what,
                (unsigned long long)a, (unsigned long long)b);
}

int32_t decode_layout(const uint8_t *d, uint64_t n, sgl_kv_decode_layout *out) {
    if (n != SGL_KV_DECODE_LAYOUT_BYTES) return layout_error("length", SGL_KV_DECODE_LAYOUT_BYTES, n);
    if (le32(d) != SGL_KV_DECODE_LAYOUT_MAGIC) return layout_error("magic", SGL_KV_DECODE_LAYOUT_MAGIC, le32(d));
    if (le32(d + 4) != 1) return layout_error("version", 1, le32(d + 4));
    sgl_kv_runtime_layout rt;
    memset(&rt, 0, sizeof rt);
    rt.dtype = (int32_t)le32(d + 8);
    const uint32_t head_layout = le32(d + 12);
    const uint8_t *q = d + 16;
    rt.page_size = le64(q);
    rt.num_layers = le64(q + 8);
    rt.kv_heads = le64(q + 16);
    rt.head_dim = le64(q + 24);
    rt.kv_tensors_per_token = le64(q + 32);
    rt.bytes_per_token = le64(q + 40);
    rt.page_size_bytes = le64(q + 48);
    const uint64_t page_count = le64(q + 56), pair = le64(q + 64), key_bytes = le64(q + 72),
                   value_bytes = le64(q + 80), heads = le64(q + 88);
    if (head_layout > SGL_KV_HND) return layout_error("head_layout", head_layout, SGL_KV_HND);
    if (pair > 1) return layout_error("tensor_pair", pair, 1);
    memset(out, 0, sizeof *out);
    int32_t rc = pair ? sgl_kv_paged_layout_new_with_tensor_pair(&rt, page_count, key_bytes, value_bytes, &out->layout)
                      : sgl_kv_paged_layout_new(&rt, page_count, &out->layout);
    if (rc) return rc;
    const uint64_t h = heads ? heads : rt.kv_heads;
    if (head_layout == SGL_KV_HND && (h == 0 || out->layout.token_bytes[0] % h || out->layout.token_bytes[1] % h))
        return layout_error("heads", h, out->layout.token_bytes[0]);
    out->head_layout = head_layout;
    out->heads = heads;
    return SGL_KV_OK;
}

void put32(std::vector<uint8_t> &b, uint32_t v) {
    for (int i = 0; i < 4; ++i) b.push_back((uint8_t)(v >> (8 * i)));
}
void put64(std::vector<uint8_t> &b, uint64_t v) {
    for (int i = 0; i < 8; ++i) b.push_back((uint8_t)(v >> (8 * i)));
}

std::vector<uint8_t> encode_layout(const sgl_kv_decode_layout &l) {
    std::vector<uint8_t> b;
    const sgl_kv_runtime_layout &rt = l.layout.runtime;
    put32(b, SGL_KV_DECODE_LAYOUT_MAGIC);
    put32(b, 1);
    put32(b, (uint32_t)rt.dtype);
    put32(b, l.head_layout);
    for (uint64_t v : {rt.page_size, rt.num_layers, rt.kv_heads, rt.head_dim, rt.kv_tensors_per_token,
                       rt.bytes_per_token, rt.page_size_bytes, l.layout.page_count, l.layout.tensor_pair,
                       l.layout.token_bytes[0], l.layout.token_bytes[1], l.heads})
        put64(b, v);
    return b;
}

// ---- frames -> records (:431-449, :465-494) ----

int32_t parse_kv_args(const Frame &f, KvArgs *a) {
    int32_t rc;
    const uint8_t *d;
    uint64_t n, v;
    if ((rc = require_min_fields(f, 10, "Mooncake KVArgs registration"))) return rc;
    if ((rc = ascii_field(f, 0, "room", &a->room)) || (rc = ascii_field(f, 1, "endpoint", &a->endpoint)))
        return rc;
    if ((rc = parse_unsigned(f, 2, "dst_port", 0xFFFF, &v))) return rc;
    a->dst_port = (uint16_t)v;
    if ((rc = ascii_field(f, 3, "mooncake_session_id", &a->session))) return rc;
    if ((rc = field(f, 4, "dst_kv_ptrs", &d, &n)) || (rc = unpack_fixed<uint64_t>(d, n, "u64 values", &a->dst_kv_ptrs)))
        return rc;
    if ((rc = field(f, 5, "dst_aux_ptrs", &d, &n)) || (rc = unpack_fixed<uint64_t>(d, n, "u64 values", &a->dst_aux_ptrs)))
        return rc;
    if ((rc = field(f, 6, "dst_state_data_ptrs", &d, &n)) ||
        (rc = unpack_lists<uint64_t>(d, n, "u64 lists", "u64 values", &a->dst_state_data_ptrs)))
        return rc;
    if ((rc = parse_i32(f, 7, "dst_tp_rank", &a->dst_tp_rank))) return rc;
    if ((rc = parse_unsigned(f, 8, "dst_attn_tp_size", UINT64_MAX, &a->dst_attn_tp_size))) return rc;
    if ((rc = parse_unsigned(f, 9, "dst_kv_item_len", UINT64_MAX, &a->dst_kv_item_len))) return rc;
    // optional_u32_lists (:1539-1547): a missing part is an empty list.
    if (f.count > 10 && ((rc = field(f, 10, "dst_state_item_lens", &d, &n)) ||
                         (rc = unpack_lists<uint32_t>(d, n, "u32 lists", "u32 values", &a->dst_state_item_lens))))
        return rc;
    if (f.count > 11 && ((rc = field(f, 11, "dst_state_dim_per_tensor", &d, &n)) ||
                         (rc = unpack_lists<uint32_t>(d, n, "u32 lists", "u32 values", &a->dst_state_dim_per_tensor))))
        return rc;
    // Parts 12 and 13 are written by the reference's encoder and read by no
    // decoder; part 14, when present and non-empty, is the decode layout.
    if (f.count > 14) {
        if ((rc = field(f, 14, "dst_kv_layout", &d, &n))) return rc;
        if (n) {
            if ((rc = decode_layout(d, n, &a->layout))) return rc;
            a->has_layout = true;
        }
    }
    return SGL_KV_OK;
}

int32_t parse_transfer(const Frame &f, Transfer *t) {
    int32_t rc;
    const uint8_t *d4, *d5, *d6;
    uint64_t n4, n5, n6, v;
    if ((rc = require_min_fields(f, 8, "Mooncake transfer metadata"))) return rc;
    if ((rc = field(f, 4, "dst_kv_indices", &d4, &n4)) || (rc = field(f, 5, "dst_aux_index", &d5, &n5)))
        return rc;
    t->is_dummy = n4 == 0 && n5 == 0;
    if (!t->is_dummy) {
        if ((rc = unpack_fixed<int32_t>(d4, n4, "i32 values", &t->dst_kv_indices))) return rc;
        if ((rc = parse_i32(f, 5, "dst_aux_index", &t->aux))) return rc;
        t->has_aux = true;
        if ((rc = field(f, 6, "dst_state_indices", &d6, &n6)) ||
            (rc = unpack_lists<int32_t>(d6, n6, "i32 lists", "i32 values", &t->dst_state_indices)))
            return rc;
    }
    if ((rc = parse_room(f, 0, "room", &t->room)) || (rc = ascii_field(f, 1, "endpoint", &t->endpoint))) return rc;
    if ((rc = parse_unsigned(f, 2, "dst_port", 0xFFFF, &v))) return rc;
    t->dst_port = (uint16_t)v;
    if ((rc = ascii_field(f, 3, "mooncake_session_id", &t->session))) return rc;
    if ((rc = parse_unsigned(f, 7, "required_dst_info_num", UINT64_MAX, &t->required))) return rc;
    // optional_usize (:1525-1537): missing or empty is None.
    if (f.count > 8 && f.parts[8].len) {  // parse_unsigned checks the part's data
        if ((rc = parse_unsigned(f, 8, "decode_prefix_len", UINT64_MAX, &t->prefix))) return rc;
        t->has_prefix = true;
    }
    return SGL_KV_OK;
}

// ---- records -> frames (:685-749, 1209-1270) ----

std::vector<uint8_t> text(const std::string &s) { return std::vector<uint8_t>(s.begin(), s.end()); }
std::vector<uint8_t> text_u64(uint64_t v) { return text(std::to_string(v)); }
std::vector<uint8_t> text_i64(int64_t v) { return text(std::to_string(v)); }

template <typename T>
std::vector<uint8_t> pack_values(const T *v, uint64_t n) {
    std::vector<uint8_t> b(n * sizeof(T));
    if (n) memcpy(b.data(), v, n * sizeof(T));  // little-endian host
    return b;
}

// pack_list_of_buffers (:1255-1270): nothing for an empty list.
template <typename T>
int32_t pack_lists(const T *values, const uint64_t *offsets, uint64_t count, const char *name,
                   std::vector<uint8_t> *out) {
    out->clear();
    if (count == 0) return SGL_KV_OK;
    if (!offsets) return fail(SGL_KV_INVALID_ARGUMENT, name, 0, 0, 0, "list %s has no offsets", name);
    if (count > UINT32_MAX) return too_large_dim(name, count, UINT32_MAX);
    put32(*out, (uint32_t)count);
    for (uint64_t i = 0; i < count; ++i) {
        if (offsets[i + 1] < offsets[i] || (offsets[i + 1] - offsets[i]) * sizeof(T) > UINT32_MAX)
            return fail(SGL_KV_INVALID_ARGUMENT, name, i, offsets[i], offsets[i + 1], "list %s has bad offsets", name);
        put32(*out, (uint32_t)((offsets[i + 1] - offsets[i]) * sizeof(T)));
    }
    if (offsets[count] > offsets[0] && !values)
        return fail(SGL_KV_INVALID_ARGUMENT, name, 0, 0, 0, "list %s has no values", name);
    for (uint64_t i = 0; i < count; ++i) {
        const std::vector<uint8_t> b = pack_values(values + offsets[i], offsets[i + 1] - offsets[i]);
        out->insert(out->end(), b.begin(), b.end());
    }
    return SGL_KV_OK;
}

int32_t emit(const std::vector<std::vector<uint8_t>> &frame, uint8_t *buf, uint64_t capacity,
             sgl_kv_frame_part *parts, uint32_t *part_count, uint64_t *bytes_needed) {
    uint64_t total = 0;
    for (const auto &p : frame) total += p.size();
    if (bytes_needed) *bytes_needed = total;
    if (part_count) *part_count = (uint32_t)frame.size();
    if (!buf) return ok();
    if (capacity < total)
        return fail(SGL_KV_ALLOCATION_OUT_OF_BOUNDS, "buffer", 0, total, capacity,
                    "frame needs %llu bytes, buffer holds %llu", (unsigned long long)total,
                    (unsigned long long)capacity);
    if (!parts) return fail(SGL_KV_INVALID_ARGUMENT, "parts", 0, 0, 0, "null parts");
    uint64_t off = 0;
    for (size_t i = 0; i < frame.size(); ++i) {
        if (!frame[i].empty()) memcpy(buf + off, frame[i].data(), frame[i].size());
        parts[i].data = buf + off;
        parts[i].len = frame[i].size();
        off += frame[i].size();
    }
    return ok();
}

bool has_string(const char *s) { return s != nullptr; }

}  // namespace

struct sgl_kv_bootstrap {
    std::map<std::string, KvArgs> kv_args;
    uint64_t registrations = 0;
    std::map<uint64_t, Room> rooms;
};

extern "C" int32_t sgl_kv_bootstrap_create(sgl_kv_bootstrap **out) {
    if (!out) return fail(SGL_KV_INVALID_ARGUMENT, "out", 0, 0, 0, "null argument");
    *out = new (std::nothrow) sgl_kv_bootstrap();
    if (!*out) return fail(SGL_KV_INVALID_ARGUMENT, "out", 0, 0, 0, "out of host memory");
    return ok();
}

extern "C" int32_t sgl_kv_bootstrap_destroy(sgl_kv_bootstrap *state) {
    delete state;
    return ok();
}

extern "C" int32_t sgl_kv_bootstrap_ingest(sgl_kv_bootstrap *state, const sgl_kv_frame_part *parts,
                                           uint32_t part_count) {
    if (!state || (part_count && !parts)) return fail(SGL_KV_INVALID_ARGUMENT, "state/parts", 0, 0, 0, "null argument");
    const Frame f{parts, part_count};
    std::string room;
    int32_t rc = ascii_field(f, 0, "room", &room);
    if (rc) return rc;
    if (room == "WATERMARK" || room == "STAGING_RSP") return ok();
    if (room == "None") {
        KvArgs a;
        if ((rc = parse_kv_args(f, &a))) return rc;
        const std::string session = a.session;
        state->kv_args[session] = std::move(a);
        ++state->registrations;
        return ok();
    }
    Transfer t;
    if ((rc = parse_transfer(f, &t))) return rc;
    auto it = state->rooms.find(t.room);
    if (it == state->rooms.end()) {
        Room r;
        r.required = t.required;
        it = state->rooms.emplace(t.room, std::move(r)).first;
    }
    Room &r = it->second;
    r.required = t.required;
    if (!r.has_prefix && t.has_prefix) {
        r.has_prefix = true;
        r.prefix = t.prefix;
    }
    const std::string session = t.session;
    r.transfers[session] = std::move(t);
    if (r.transfers.size() == r.required) r.status = kKvPollWaitingForInput;
    return ok();
}

extern "C" int32_t sgl_kv_bootstrap_registration_count(const sgl_kv_bootstrap *state, uint64_t *count) {
    if (!state || !count) return fail(SGL_KV_INVALID_ARGUMENT, "state/count", 0, 0, 0, "null argument");
    *count = state->registrations;
    return ok();
}

namespace {

int32_t missing_kv_args(uint64_t room, const char *session) {
    return fail(SGL_KV_BOOT_MISSING_KV_ARGS, nullptr, room, 0, 0,
                "missing Mooncake KVArgs registration for room %llu session %.200s", (unsigned long long)room,
                session);
}

}  // namespace

extern "C" int32_t sgl_kv_bootstrap_get_kv_args(const sgl_kv_bootstrap *state, const char *session,
                                            sgl_kv_bootstrap_kv_args *out) {
    if (!state || !session || !out) return fail(SGL_KV_INVALID_ARGUMENT, "state/session/out", 0, 0, 0, "null argument");
    auto it = state->kv_args.find(session);
    if (it == state->kv_args.end()) return missing_kv_args(0, session);
    const KvArgs &a = it->second;
    memset(out, 0, sizeof *out);
    out->endpoint = a.endpoint.c_str();
    out->mooncake_session_id = a.session.c_str();
    out->dst_port = a.dst_port;
    out->dst_tp_rank = a.dst_tp_rank;
    out->dst_attn_tp_size = a.dst_attn_tp_size;
    out->dst_kv_item_len = a.dst_kv_item_len;
    out->dst_kv_ptrs = a.dst_kv_ptrs.data();
    out->dst_kv_ptr_count = a.dst_kv_ptrs.size();
    out->dst_aux_ptrs = a.dst_aux_ptrs.data();
    out->dst_aux_ptr_count = a.dst_aux_ptrs.size();
    out->dst_state_data_ptrs = {a.dst_state_data_ptrs.values.data(), a.dst_state_data_ptrs.offsets.data(),
                                a.dst_state_data_ptrs.count()};
    out->dst_state_item_lens = {a.dst_state_item_lens.values.data(), a.dst_state_item_lens.offsets.data(),
                                a.dst_state_item_lens.count()};
    out->dst_state_dim_per_tensor = {a.dst_state_dim_per_tensor.values.data(),
                                     a.dst_state_dim_per_tensor.offsets.data(), a.dst_state_dim_per_tensor.count()};
    out->decode_layout = a.has_layout ? &a.layout : nullptr;
    return ok();
}

extern "C" int32_t sgl_kv_bootstrap_transfer_status(const sgl_kv_bootstrap *state, uint64_t room, int32_t *status) {
    if (!state || !status) return fail(SGL_KV_INVALID_ARGUMENT, "state/status", 0, 0, 0, "null argument");
    auto it = state->rooms.find(room);
    *status = it == state->rooms.end() ? -1 : it->second.status;
    return ok();
}

extern "C" int32_t sgl_kv_bootstrap_room(const sgl_kv_bootstrap *state, uint64_t room, uint64_t *required,
                                         uint32_t *has_prefix, uint64_t *prefix, uint64_t *sessions) {
    if (!state) return fail(SGL_KV_INVALID_ARGUMENT, "state", 0, 0, 0, "null argument");
    auto it = state->rooms.find(room);
    if (it == state->rooms.end())
        return fail(SGL_KV_BOOT_MISSING_TRANSFER_ROOM, nullptr, room, 0, 0, "missing Mooncake transfer room: %llu",
                    (unsigned long long)room);
    const Room &r = it->second;
    if (required) *required = r.required;
    if (has_prefix) *has_prefix = r.has_prefix ? 1 : 0;
    if (prefix) *prefix = r.prefix;
    if (sessions) *sessions = r.transfers.size();
    return ok();
}

extern "C" int32_t sgl_kv_bootstrap_get_transfer(const sgl_kv_bootstrap *state, uint64_t room, const char *session,
                                             sgl_kv_bootstrap_transfer *out) {
    if (!state || !session || !out) return fail(SGL_KV_INVALID_ARGUMENT, "state/session/out", 0, 0, 0, "null argument");
    auto it = state->rooms.find(room);
    if (it == state->rooms.end())
        return fail(SGL_KV_BOOT_MISSING_TRANSFER_ROOM, nullptr, room, 0, 0, "missing Mooncake transfer room: %llu",
                    (unsigned long long)room);
    auto tt = it->second.transfers.find(session);
    if (tt == it->second.transfers.end())
        return fail(SGL_KV_INVALID_ARGUMENT, "mooncake_session_id", room, 0, 0,
                    "room %llu has no transfer metadata from session %.200s", (unsigned long long)room, session);
    const Transfer &t = tt->second;
    memset(out, 0, sizeof *out);
    out->room = t.room;
    out->endpoint = t.endpoint.c_str();
    out->mooncake_session_id = t.session.c_str();
    out->dst_port = t.dst_port;
    out->is_dummy = t.is_dummy ? 1 : 0;
    out->dst_kv_indices = t.dst_kv_indices.data();
    out->dst_kv_index_count = t.dst_kv_indices.size();
    out->has_dst_aux_index = t.has_aux ? 1 : 0;
    out->dst_aux_index = t.aux;
    out->dst_state_indices = {t.dst_state_indices.values.data(), t.dst_state_indices.offsets.data(),
                              t.dst_state_indices.count()};
    out->required_dst_info_num = t.required;
    out->has_decode_prefix_len = t.has_prefix ? 1 : 0;
    out->decode_prefix_len = t.prefix;
    return ok();
}

extern "C" int32_t sgl_kv_bootstrap_remote_layouts(const sgl_kv_bootstrap *state, uint64_t room,
                                                   sgl_kv_remote_kv_layout *out, uint64_t capacity,
                                                   uint64_t *count) {
    if (!state || !count || (capacity && !out))
        return fail(SGL_KV_INVALID_ARGUMENT, "state/out/count", 0, 0, 0, "null argument");
    auto it = state->rooms.find(room);
    if (it == state->rooms.end())
        return fail(SGL_KV_BOOT_MISSING_TRANSFER_ROOM, nullptr, room, 0, 0, "missing Mooncake transfer room: %llu",
                    (unsigned long long)room);
    uint64_t n = 0;
    for (const auto &kv : it->second.transfers) {
        const Transfer &t = kv.second;
        if (t.is_dummy) continue;
        auto a = state->kv_args.find(t.session);
        if (a == state->kv_args.end()) return missing_kv_args(room, t.session.c_str());
        if (n < capacity) {
            sgl_kv_remote_kv_layout &l = out[n];
            memset(&l, 0, sizeof l);
            l.mooncake_session_id = t.session.c_str();
            l.dst_kv_ptrs = a->second.dst_kv_ptrs.data();
            l.dst_kv_ptr_count = a->second.dst_kv_ptrs.size();
            l.dst_kv_indices = t.dst_kv_indices.data();
            l.dst_kv_index_count = t.dst_kv_indices.size();
            l.dst_kv_item_len = a->second.dst_kv_item_len;
            l.decode_layout = a->second.has_layout ? &a->second.layout : nullptr;
        }
        ++n;
    }
    *count = n;
    return ok();
}

extern "C" int32_t sgl_kv_bootstrap_encode_kv_args(const sgl_kv_bootstrap_kv_args *a, uint8_t *buf,
                                                   uint64_t capacity, sgl_kv_frame_part *parts,
                                                   uint32_t *part_count, uint64_t *bytes_needed) {
    if (!a || !has_string(a->endpoint) || !has_string(a->mooncake_session_id))
        return fail(SGL_KV_INVALID_ARGUMENT, "args", 0, 0, 0, "null argument");
    if ((a->dst_kv_ptr_count && !a->dst_kv_ptrs) || (a->dst_aux_ptr_count && !a->dst_aux_ptrs))
        return fail(SGL_KV_INVALID_ARGUMENT, "ptrs", 0, 0, 0, "pointer list without values");
    if (a->dst_port > 0xFFFF) return too_large_dim("dst_port", a->dst_port, 0xFFFF);
    std::vector<std::vector<uint8_t>> frame;
    frame.push_back(text("None"));
    frame.push_back(text(a->endpoint));
    frame.push_back(text_u64(a->dst_port));
    frame.push_back(text(a->mooncake_session_id));
    frame.push_back(pack_values(a->dst_kv_ptrs, a->dst_kv_ptr_count));
    frame.push_back(pack_values(a->dst_aux_ptrs, a->dst_aux_ptr_count));
    std::vector<uint8_t> p;
    int32_t rc;
    if ((rc = pack_lists(a->dst_state_data_ptrs.values, a->dst_state_data_ptrs.offsets, a->dst_state_data_ptrs.count,
                         "dst_state_data_ptrs", &p)))
        return rc;
    frame.push_back(p);
    frame.push_back(text_i64(a->dst_tp_rank));
    frame.push_back(text_u64(a->dst_attn_tp_size));
    frame.push_back(text_u64(a->dst_kv_item_len));
    if ((rc = pack_lists(a->dst_state_item_lens.values, a->dst_state_item_lens.offsets, a->dst_state_item_lens.count,
                         "dst_state_item_lens", &p)))
        return rc;
    frame.push_back(p);
    if ((rc = pack_lists(a->dst_state_dim_per_tensor.values, a->dst_state_dim_per_tensor.offsets,
                         a->dst_state_dim_per_tensor.count, "dst_state_dim_per_tensor", &p)))
        return rc;
    frame.push_back(p);
    frame.push_back({});
    frame.push_back(text("0"));
    if (a->decode_layout) {
        // Round-trip the descriptor through the decoder so that only a layout
        // the prefill side will accept is ever sent.
        const std::vector<uint8_t> l = encode_layout(*a->decode_layout);
        sgl_kv_decode_layout check;
        if ((rc = decode_layout(l.data(), l.size(), &check))) return rc;
        frame.push_back(l);
    }
    return emit(frame, buf, capacity, parts, part_count, bytes_needed);
}

extern "C" int32_t sgl_kv_bootstrap_encode_transfer(const sgl_kv_bootstrap_transfer *t, uint8_t *buf,
                                                    uint64_t capacity, sgl_kv_frame_part *parts,
                                                    uint32_t *part_count, uint64_t *bytes_needed) {
    if (!t || !has_string(t->endpoint) || !has_string(t->mooncake_session_id))
        return fail(SGL_KV_INVALID_ARGUMENT, "transfer", 0, 0, 0, "null argument");
    if (t->dst_port > 0xFFFF) return too_large_dim("dst_port", t->dst_port, 0xFFFF);
    std::vector<uint8_t> indices, aux, state;
    if (!t->is_dummy) {
        if (!t->has_dst_aux_index)
            return fail(SGL_KV_BOOT_MISSING_AUX_INDEX, nullptr, 0, 0, 0,
                        "Mooncake transfer metadata for %.200s needs aux index", t->mooncake_session_id);
        if (t->dst_kv_index_count && !t->dst_kv_indices)
            return fail(SGL_KV_INVALID_ARGUMENT, "dst_kv_indices", 0, 0, 0, "index list without values");
        indices = pack_values(t->dst_kv_indices, t->dst_kv_index_count);
        aux = text_i64(t->dst_aux_index);
        int32_t rc = pack_lists(t->dst_state_indices.values, t->dst_state_indices.offsets, t->dst_state_indices.count,
                                "dst_state_indices", &state);
        if (rc) return rc;
    }
    std::vector<std::vector<uint8_t>> frame;
    frame.push_back(text_u64(t->room));
    frame.push_back(text(t->endpoint));
    frame.push_back(text_u64(t->dst_port));
    frame.push_back(text(t->mooncake_session_id));
    frame.push_back(indices);
    frame.push_back(aux);
    frame.push_back(state);
    frame.push_back(text_u64(t->required_dst_info_num));
    // The reference writes decode_prefix_len.unwrap_or(0) (:746).
    frame.push_back(text_u64(t->has_decode_prefix_len ? t->decode_prefix_len : 0));
    return emit(frame, buf, capacity, parts, part_count, bytes_needed);
}
