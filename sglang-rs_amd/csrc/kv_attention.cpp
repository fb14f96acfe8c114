// kv_attention.cpp -- host side of the paged-attention reader: the plan
// (CudaBf16PagedAttentionPlan::new, crates/sglang-kernel/src/
// cuda_attention.rs:277-430, same validation order and error variants),
// the plan derived from a pool layout (build_plan,
// crates/sglang-srt/src/cuda_attention.rs:505-572) and the launch
// (CudaBf16PagedAttentionKernels::forward, cuda_attention.rs:681-850:
// device and range checks, clear the error word, launch, synchronise, read
// the word).
#include <hip/hip_runtime.h>

#include <mutex>
#include <math.h>
#include <string.h>

#include "kv_internal.h"

using namespace sglkv;

namespace {

// The plan flags: EXACT_WEIGHTS (the default, kept for callers that set it)
// and FAST_WEIGHTS exclude each other; other bits are unknown.
int32_t check_flags(uint32_t flags) {
    constexpr uint32_t known = SGL_KV_ATTN_EXACT_WEIGHTS | SGL_KV_ATTN_FAST_WEIGHTS;
    if (flags & ~known)
        return fail(SGL_KV_INVALID_ARGUMENT, "flags", flags, known, 0, "unknown attention plan flags 0x%x", flags);
    if ((flags & known) == known)
        return fail(SGL_KV_INVALID_ARGUMENT, "flags", flags, known, 0,
                    "attention plan flags 0x%x ask for exact and fast weights at once", flags);
    return SGL_KV_OK;
}

int32_t attn_overflow() {
    return fail(SGL_KV_SHAPE_OVERFLOW, nullptr, 0, 0, 0, "CUDA paged attention shape overflowed");
}

int32_t region_end(const char *tensor, uint64_t offset, uint64_t page_bytes, uint64_t stride,
                   uint64_t *end) {
    if (add_ovf(offset, page_bytes, end)) return attn_overflow();
    if (*end > stride)
        return fail(SGL_KV_TENSOR_PAGE_REGION_OUT_OF_BOUNDS, tensor, offset, page_bytes, stride,
                    "CUDA paged attention %s page region [%llu, %llu) exceeds page stride %llu", tensor,
                    (unsigned long long)offset, (unsigned long long)*end, (unsigned long long)stride);
    return SGL_KV_OK;
}

}  // namespace

// Device error word bits of the attention kernels ->
// DeviceMetadataInvalid with the reference's bit values (request 0x1,
// sequence 0x2, slot 0x4; cuda_attention.rs:59-99).
int32_t sglkv::attention_flag_status(uint32_t flag) {
    const uint32_t bad = ((flag & SGLKV_FLAG_ATTN_REQUEST) ? 1u : 0u) |
                         ((flag & SGLKV_FLAG_ATTN_SEQUENCE) ? 2u : 0u) |
                         ((flag & SGLKV_FLAG_ATTN_SLOT) ? 4u : 0u);
    if (bad)
        return fail(SGL_KV_ATTN_DEVICE_METADATA_INVALID, nullptr, bad, 0, 0,
                    "CUDA paged attention rejected device metadata with error flags 0x%x "
                    "(request=0x1, sequence=0x2, slot=0x4)",
                    bad);
    return ok();
}

extern "C" int32_t sgl_kv_attention_plan_new(const sgl_kv_attention_plan_config *c,
                                             sgl_kv_attention_plan *out) {
    if (!c || !out) return fail(SGL_KV_INVALID_ARGUMENT, "config/out", 0, 0, 0, "null argument");
    const sgl_kv_attention_layout &lay = c->layout;
    const struct {
        const char *name;
        uint64_t value;
    } dims[] = {{"query_count", c->query_count},
                {"request_count", c->request_count},
                {"sequence_slot_count", c->sequence_slot_count},
                {"slot_count", c->slot_count},
                {"query_head_count", c->query_head_count},
                {"kv_head_count", c->kv_head_count},
                {"query_key_head_dim", c->query_key_head_dim},
                {"value_head_dim", c->value_head_dim},
                {"page_size", lay.page_size},
                {"page_stride_bytes", lay.page_stride_bytes},
                {"key_row_bytes", lay.key_row_bytes},
                {"value_row_bytes", lay.value_row_bytes}};
    for (const auto &d : dims)
        if (d.value == 0)
            return fail(SGL_KV_ZERO_DIMENSION, d.name, 0, 0, 0,
                        "CUDA paged attention dimension %s must be non-zero", d.name);
    if (!isfinite(c->scale) || c->scale <= 0.0f) {
        uint32_t bits;
        memcpy(&bits, &c->scale, sizeof bits);
        return fail(SGL_KV_ATTN_INVALID_SCALE, nullptr, bits, 0, 0,
                    "CUDA paged attention scale must be finite and positive, got %g", (double)c->scale);
    }
    if (c->query_head_count % c->kv_head_count)
        return fail(SGL_KV_ATTN_QUERY_HEADS_NOT_DIVISIBLE, nullptr, c->query_head_count,
                    c->kv_head_count, 0,
                    "CUDA paged attention query head count %llu is not divisible by KV head count %llu",
                    (unsigned long long)c->query_head_count, (unsigned long long)c->kv_head_count);
    uint64_t want;
    if (mul_ovf(c->kv_head_count, c->query_key_head_dim, &want) || mul_ovf(want, 2, &want))
        return attn_overflow();
    if (lay.key_row_bytes != want)
        return fail(SGL_KV_ATTN_KEY_ROW_BYTES_MISMATCH, nullptr, want, lay.key_row_bytes, 0,
                    "CUDA BF16 paged attention requires %llu bytes per KV row, layout has %llu",
                    (unsigned long long)want, (unsigned long long)lay.key_row_bytes);
    if (mul_ovf(c->kv_head_count, c->value_head_dim, &want) || mul_ovf(want, 2, &want))
        return attn_overflow();
    if (lay.value_row_bytes != want)
        return fail(SGL_KV_ATTN_VALUE_ROW_BYTES_MISMATCH, nullptr, want, lay.value_row_bytes, 0,
                    "CUDA BF16 paged attention requires %llu bytes per value row, layout has %llu",
                    (unsigned long long)want, (unsigned long long)lay.value_row_bytes);
    uint64_t key_page, value_page, key_end, value_end;
    if (mul_ovf(lay.page_size, lay.key_row_bytes, &key_page) ||
        mul_ovf(lay.page_size, lay.value_row_bytes, &value_page))
        return attn_overflow();
    int32_t rc;
    if ((rc = region_end("key", lay.key_in_page_offset, key_page, lay.page_stride_bytes, &key_end)) ||
        (rc = region_end("value", lay.value_in_page_offset, value_page, lay.page_stride_bytes, &value_end)))
        return rc;
    if (lay.key_in_page_offset < value_end && lay.value_in_page_offset < key_end) {
        rc = fail(SGL_KV_ATTN_TENSOR_PAGE_REGIONS_OVERLAP, nullptr, lay.key_in_page_offset,
                  lay.value_in_page_offset, key_page,
                  "CUDA paged attention key/value page regions overlap: key offset %llu (%llu bytes), "
                  "value offset %llu (%llu bytes)",
                  (unsigned long long)lay.key_in_page_offset, (unsigned long long)key_page,
                  (unsigned long long)lay.value_in_page_offset, (unsigned long long)value_page);
        set_detail_d(value_page);
        return rc;
    }
    if (lay.head_layout > SGL_KV_HND)
        return fail(SGL_KV_INVALID_ARGUMENT, "head_layout", lay.head_layout, 0, 0,
                    "unknown head layout %u", lay.head_layout);
    if ((rc = check_flags(c->flags))) return rc;

    sgl_kv_attention_plan p;
    memset(&p, 0, sizeof p);
    p.config = *c;
    uint64_t v;
    if (mul_ovf(c->query_count, c->query_head_count, &v) || mul_ovf(v, c->query_key_head_dim, &v) ||
        mul_ovf(v, 2, &p.query_required_bytes))
        return attn_overflow();
    if (mul_ovf(c->query_count, 4, &p.query_request_indices_required_bytes) ||
        mul_ovf(c->query_count, 8, &p.query_sequence_lengths_required_bytes) ||
        add_ovf(c->request_count, 1, &v) || mul_ovf(v, 8, &p.request_slot_offsets_required_bytes) ||
        mul_ovf(c->sequence_slot_count, 8, &p.sequence_slots_required_bytes))
        return attn_overflow();
    // The pool must reach the last slot's key and value rows (NHD, as the
    // reference computes it) or, for head-major pages, the last page's
    // whole key and value regions.
    const uint64_t last_slot = c->slot_count - 1;
    const uint64_t last_page = last_slot / lay.page_size, last_token = last_slot % lay.page_size;
    uint64_t kend, vend;
    if (lay.head_layout == SGL_KV_HND) {
        kend = key_end;
        vend = value_end;
    } else if (mul_ovf(last_token, lay.key_row_bytes, &kend) ||
               add_ovf(kend, lay.key_in_page_offset, &kend) || add_ovf(kend, lay.key_row_bytes, &kend) ||
               mul_ovf(last_token, lay.value_row_bytes, &vend) ||
               add_ovf(vend, lay.value_in_page_offset, &vend) ||
               add_ovf(vend, lay.value_row_bytes, &vend)) {
        return attn_overflow();
    }
    if (mul_ovf(last_page, lay.page_stride_bytes, &v) ||
        add_ovf(v, kend > vend ? kend : vend, &p.pool_required_bytes))
        return attn_overflow();
    if (mul_ovf(c->query_count, c->query_head_count, &v) || mul_ovf(v, c->value_head_dim, &v) ||
        mul_ovf(v, 2, &p.output_required_bytes))
        return attn_overflow();
    // The reference sizes its block's shared memory as (256 + dv) floats and
    // launches one block per (query, head); keep its limits.
    if (add_ovf(256, c->value_head_dim, &v) || mul_ovf(v, 4, &v) || v > UINT32_MAX) return attn_overflow();
    if (c->query_count > UINT32_MAX)
        return too_large_dim("query_count", c->query_count, UINT32_MAX);
    if (c->query_head_count > UINT32_MAX)
        return too_large_dim("query_head_count", c->query_head_count, UINT32_MAX);
    *out = p;
    return ok();
}

// build_plan (crates/sglang-srt/src/cuda_attention.rs:505-572): the
// attention geometry of one layer of a bf16 pool.
extern "C" int32_t sgl_kv_attention_plan_for_layer(const sgl_kv_paged_layout *layout, uint64_t layer,
                                                   uint64_t query_count, uint64_t request_count,
                                                   uint64_t sequence_slot_count,
                                                   uint64_t query_head_count, float scale,
                                                   uint32_t head_layout, sgl_kv_attention_plan *out) {
    if (!layout || !out) return fail(SGL_KV_INVALID_ARGUMENT, "layout/out", 0, 0, 0, "null argument");
    const sgl_kv_runtime_layout &rt = layout->runtime;
    if (rt.dtype != SGL_KV_DTYPE_BFLOAT16) {
        static const char *const names[] = {"Auto", "Float32", "Bfloat16", "Fp8E4M3", "Fp8E5M2", "Fp4E2M1"};
        const char *name = rt.dtype >= 0 && rt.dtype <= 5 ? names[rt.dtype] : "unknown";
        return fail(SGL_KV_ATTN_UNSUPPORTED_KV_DTYPE, nullptr, (uint64_t)(int64_t)rt.dtype,
                    SGL_KV_DTYPE_BFLOAT16, 0,
                    "CUDA paged attention requires KV cache dtype Bfloat16, found %s", name);
    }
    uint64_t start, end, key_row, value_row;
    int32_t rc;
    if ((rc = sgl_kv_paged_layout_tensor_token_byte_range(layout, 0, layer, 0, 0, &start, &end)))
        return rc;
    key_row = end - start;
    const uint64_t key_offset = start;
    if ((rc = sgl_kv_paged_layout_tensor_token_byte_range(layout, 0, layer, 1, 0, &start, &end)))
        return rc;
    value_row = end - start;
    const uint64_t value_offset = start;
    uint64_t denom;
    if (mul_ovf(rt.kv_heads, 2, &denom) || key_row % denom)
        return fail(SGL_KV_ATTN_TENSOR_ROW_GEOMETRY_MISMATCH, "key", key_row, rt.kv_heads, 2,
                    "CUDA paged attention key row has %llu bytes, which cannot be divided across %llu "
                    "heads of 2-byte elements",
                    (unsigned long long)key_row, (unsigned long long)rt.kv_heads);
    if (value_row % denom)
        return fail(SGL_KV_ATTN_TENSOR_ROW_GEOMETRY_MISMATCH, "value", value_row, rt.kv_heads, 2,
                    "CUDA paged attention value row has %llu bytes, which cannot be divided across %llu "
                    "heads of 2-byte elements",
                    (unsigned long long)value_row, (unsigned long long)rt.kv_heads);
    sgl_kv_attention_plan_config c;
    memset(&c, 0, sizeof c);
    c.query_count = query_count;
    c.request_count = request_count;
    c.sequence_slot_count = sequence_slot_count;
    c.slot_count = layout->slot_count;
    c.query_head_count = query_head_count;
    c.kv_head_count = rt.kv_heads;
    c.query_key_head_dim = key_row / denom;
    c.value_head_dim = value_row / denom;
    c.scale = scale;
    c.layout.page_size = rt.page_size;
    c.layout.page_stride_bytes = rt.page_size_bytes;
    c.layout.key_in_page_offset = key_offset;
    c.layout.value_in_page_offset = value_offset;
    c.layout.key_row_bytes = key_row;
    c.layout.value_row_bytes = value_row;
    c.layout.head_layout = head_layout;
    return sgl_kv_attention_plan_new(&c, out);
}

namespace {

int32_t attn_ptr(const char *name, const sgl_kv_device_buffer &b, uint64_t offset, uint64_t need,
                 uint64_t *addr) {
    if (!b.ptr) return fail(SGL_KV_INVALID_ARGUMENT, name, 0, 0, 0, "null buffer %s", name);
    uint64_t end;
    if (add_ovf(offset, need, &end) || end > b.byte_len)
        return fail(SGL_KV_ALLOCATION_OUT_OF_BOUNDS, name, offset, need, b.byte_len,
                    "allocation %s range [%llu, +%llu) exceeds its %llu bytes", name,
                    (unsigned long long)offset, (unsigned long long)need,
                    (unsigned long long)b.byte_len);
    *addr = (uint64_t)(uintptr_t)b.ptr + offset;
    return SGL_KV_OK;
}

uint64_t ceil_div(uint64_t a, uint64_t b) { return (a + b - 1) / b; }

// Validates, sizes the split and launches the attention (and, with
// several splits, the combine pass) on `stream`; nothing waits. Metadata
// errors raise `flag_word`. `workspace` (fixed, `workspace_bytes` long)
// holds the split records when given; otherwise the context's buffer,
// grown on demand.
int32_t attention_enqueue(sgl_rocm_kv_ctx *ctx, const sgl_kv_attention_plan *plan,
                          const sgl_kv_attention_buffers *b, uint64_t max_sequence_length,
                          hipStream_t s, uint32_t *flag_word, void *workspace = nullptr,
                          uint64_t workspace_bytes = 0) {
    if (!ctx || !plan || !b)
        return fail(SGL_KV_INVALID_ARGUMENT, "ctx/plan/buffers", 0, 0, 0, "null argument");
    const sgl_kv_attention_plan_config &c = plan->config;
    const sgl_kv_attention_layout &lay = c.layout;
    const struct {
        const char *name;
        const sgl_kv_device_buffer *buf;
    } all[] = {{"queries", &b->queries},
               {"query_request_indices", &b->query_request_indices},
               {"query_sequence_lengths", &b->query_sequence_lengths},
               {"request_slot_offsets", &b->request_slot_offsets},
               {"sequence_slots", &b->sequence_slots},
               {"pool", &b->pool},
               {"output", &b->output}};
    int32_t rc;
    for (const auto &a : all)
        if ((rc = check_device(ctx, a.name, *a.buf))) return rc;
    // A plan is a plain struct the caller may have edited since plan_new.
    if ((rc = check_flags(c.flags))) return rc;
    uint64_t qp, rip, slp, rop, ssp, poolp, outp;
    if ((rc = attn_ptr("queries", b->queries, b->queries_offset, plan->query_required_bytes, &qp)) ||
        (rc = attn_ptr("query_request_indices", b->query_request_indices, b->query_request_indices_offset,
                       plan->query_request_indices_required_bytes, &rip)) ||
        (rc = attn_ptr("query_sequence_lengths", b->query_sequence_lengths,
                       b->query_sequence_lengths_offset, plan->query_sequence_lengths_required_bytes,
                       &slp)) ||
        (rc = attn_ptr("request_slot_offsets", b->request_slot_offsets, b->request_slot_offsets_offset,
                       plan->request_slot_offsets_required_bytes, &rop)) ||
        (rc = attn_ptr("sequence_slots", b->sequence_slots, b->sequence_slots_offset,
                       plan->sequence_slots_required_bytes, &ssp)) ||
        (rc = attn_ptr("pool", b->pool, b->pool_offset, plan->pool_required_bytes, &poolp)) ||
        (rc = attn_ptr("output", b->output, b->output_offset, plan->output_required_bytes, &outp)))
        return rc;
    if (c.query_key_head_dim > SGLKV_ATTN_MAX_DK)
        return too_large_dim("query_key_head_dim", c.query_key_head_dim, SGLKV_ATTN_MAX_DK);
    // Every element access is naturally aligned.
    const bool aligned = qp % 2 == 0 && outp % 2 == 0 && rip % 4 == 0 && slp % 8 == 0 && rop % 8 == 0 &&
                         ssp % 8 == 0 &&
                         ((poolp | lay.key_in_page_offset | lay.value_in_page_offset |
                           lay.page_stride_bytes | lay.key_row_bytes | lay.value_row_bytes) & 1) == 0;
    if (!aligned)
        return fail(SGL_KV_INVALID_ARGUMENT, "alignment", 0, 0, 0,
                    "paged attention buffers must be aligned to their element sizes");

    sglkv_attn_params p;
    memset(&p, 0, sizeof p);
    p.queries = reinterpret_cast<const uint16_t *>(qp);
    p.query_request_indices = reinterpret_cast<const uint32_t *>(rip);
    p.query_sequence_lengths = reinterpret_cast<const uint64_t *>(slp);
    p.request_slot_offsets = reinterpret_cast<const uint64_t *>(rop);
    p.sequence_slots = reinterpret_cast<const uint64_t *>(ssp);
    p.pool = reinterpret_cast<const uint8_t *>(poolp);
    p.output = reinterpret_cast<uint16_t *>(outp);
    p.flag = flag_word;
    p.query_count = c.query_count;
    p.request_count = c.request_count;
    p.sequence_slot_count = c.sequence_slot_count;
    p.slot_count = c.slot_count;
    p.page_size = lay.page_size;
    p.page_stride = lay.page_stride_bytes;
    p.key_offset = lay.key_in_page_offset;
    p.value_offset = lay.value_in_page_offset;
    const uint64_t kh = c.query_key_head_dim * 2, vh = c.value_head_dim * 2;
    if (lay.head_layout == SGL_KV_HND) {
        p.key_head_stride = lay.page_size * kh;
        p.key_token_stride = kh;
        p.value_head_stride = lay.page_size * vh;
        p.value_token_stride = vh;
    } else {
        p.key_head_stride = kh;
        p.key_token_stride = lay.key_row_bytes;
        p.value_head_stride = vh;
        p.value_token_stride = lay.value_row_bytes;
    }
    p.query_heads = (uint32_t)c.query_head_count;
    p.kv_heads = (uint32_t)c.kv_head_count;
    p.group = (uint32_t)(c.query_head_count / c.kv_head_count);
    p.head_groups = (uint32_t)ceil_div(p.group, SGLKV_ATTN_HEADS);
    p.dk = (uint32_t)c.query_key_head_dim;
    p.dk_pad = (uint32_t)ceil_div(p.dk, 32) * 32;
    p.dv = (uint32_t)c.value_head_dim;
    p.dv_blocks = (uint32_t)ceil_div(p.dv, SGLKV_ATTN_DV);
    p.scale_log2 = c.scale * 1.4426950408889634f;
    p.page_shift = 32;
    if ((lay.page_size & (lay.page_size - 1)) == 0) {
        p.page_shift = 0;
        while ((1ull << p.page_shift) < lay.page_size) ++p.page_shift;
    }

    const bool vec = (p.dk % 8 == 0) && (p.dv % 8 == 0) &&
                     ((poolp + lay.key_in_page_offset) % 16 == 0) &&
                     ((poolp + lay.value_in_page_offset) % 16 == 0) &&
                     ((lay.page_stride_bytes | p.key_head_stride | p.key_token_stride | p.value_head_stride |
                       p.value_token_stride) % 16 == 0);
    // 16-byte rows, power-of-two pages and strides that fit 32 bits admit
    // the pipelined and wide bodies (32-bit slots, shift-and-mask pages);
    // head dims up to 128 take the software-pipelined body.
    const bool fast = vec && p.page_shift < 32 && c.slot_count < (1ull << 32) &&
                      lay.page_stride_bytes <= UINT32_MAX && p.key_token_stride <= UINT32_MAX &&
                      p.value_token_stride <= UINT32_MAX;
    const bool pipe = fast && p.dk_pad <= 128 && p.dv <= SGLKV_ATTN_DV;
    int which = !vec ? 1 : !pipe ? 0 : (p.dk == 128 && p.dv == 128) ? 2 : 3;
    // Many query heads per KV head (more than one 16-head group) or wide
    // values: the wide bodies share each K/V block among 4 head groups
    // instead of every group and value block reading it again. They hold
    // the queries in registers as 16-byte vectors.
    unsigned threads = 64;
    unsigned lds = (unsigned)((SGLKV_ATTN_HEADS * (p.dk_pad + 8) + SGLKV_ATTN_DV * SGLKV_ATTN_VT_STRIDE) *
                              sizeof(uint16_t));
    uint64_t max_len = max_sequence_length ? max_sequence_length : c.sequence_slot_count;
    if (max_len > c.sequence_slot_count) max_len = c.sequence_slot_count;
    // (Their chunks fit the slot table, so the grid's 65535 splits bound
    // the length they take.)
    if (fast && qp % 16 == 0 && (p.head_groups > 1 || p.dv > SGLKV_ATTN_DV) &&
        max_len <= 65535ull * SGLKV_ATTN_WIDE_SLOTS) {
        const unsigned narrow = SGLKV_ATTN_WIDE_LDS_BYTES(4u, 8u), wide = SGLKV_ATTN_WIDE_LDS_BYTES(18u, 32u);
        if (p.dk_pad <= 128 && p.dv <= 128 && narrow <= (unsigned)ctx->max_lds_per_block) {
            which = 5;
            lds = narrow;
            threads = 64 * SGLKV_ATTN_WIDE_WAVES;
        } else if (p.dk > 512 && p.dk <= 576 && p.dv == 512 &&
                   SGLKV_ATTN_LATENT_LDS_BYTES <= (unsigned)ctx->max_lds_per_block) {
            // MLA's latent rows (K 576 = 512 + 64 rope dims, V 512): 32 heads
            // per wave, rows loaded straight into LDS.
            which = 6;
            lds = SGLKV_ATTN_LATENT_LDS_BYTES;
            threads = 64 * SGLKV_ATTN_LATENT_WAVES;
        } else if (p.dk_pad <= 576 && p.dv <= 512 && wide <= (unsigned)ctx->max_lds_per_block) {
            which = 4;
            lds = wide;
            threads = 64 * SGLKV_ATTN_WIDE_WAVES;
        }
    }
    // Dims 128 or 64 with one head group per KV head (the Llama/Qwen GQA
    // decodes): the staged bodies, rows loaded straight into LDS. They
    // share one in-page offset between a token's K and V rows and form it
    // with a 24-bit multiply.
    // Dims 256 (Qwen3.5's full-attention layers) take the staged body too,
    // one wave covering all 256 value dims.
    const bool d64 = which == 3 && p.dk == 64 && p.dv == 64;
    const bool d256 = fast && p.dk == 256 && p.dv == 256;
    if ((which == 2 || d64 || d256) && qp % 16 == 0 && p.head_groups == 1 &&
        p.key_token_stride == p.value_token_stride && p.key_token_stride < (1u << 24) &&
        lay.page_size <= (1u << 24) &&
        max_len <= 65535ull * SGLKV_ATTN_STAGED_SLOTS &&
        SGLKV_ATTN_STAGED_LDS_BYTES(p.dk) <= (unsigned)ctx->max_lds_per_block) {
        which = d64 ? 8 : d256 ? 10 : 7;
        lds = SGLKV_ATTN_STAGED_LDS_BYTES(p.dk);
        // Head-major pages at dims 128: K in registers, V alone in LDS.
        // (Dims 64 keep K in LDS: the same body with K in registers,
        // 125 VGPRs, measured no faster on head-major pages.)
        if (which == 7 && lay.head_layout == SGL_KV_HND) {
            which = 11;
            lds = SGLKV_ATTN_KREG_LDS_BYTES(p.dk);
        }
        threads = 64;
        p.dv_blocks = 1;
    }
    p.zero_row = ctx->zero_row;
    p.page_stride32 = (uint32_t)lay.page_stride_bytes;
    p.key_token_stride32 = (uint32_t)p.key_token_stride;
    p.value_token_stride32 = (uint32_t)p.value_token_stride;
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");

    // Workgroups before splitting; split each query's sequence so that the
    // launch fills every CU with as many workgroups as stay resident at
    // once (the kernel's occupancy at this LDS size), in one round.
    const bool wide = which >= 4 && which <= 6;  // the wide and latent bodies (7, 8, 10, 11: staged)
    const uint64_t hblocks = which == 6 ? ceil_div(p.group, SGLKV_ATTN_LATENT_HEADS)
                                        : (p.head_groups + SGLKV_ATTN_WIDE_GROUPS - 1) / SGLKV_ATTN_WIDE_GROUPS;
    uint64_t base = c.query_count;
    if (mul_ovf(base, p.kv_heads, &base) || (wide && mul_ovf(base, hblocks, &base)) ||
        (!wide && (mul_ovf(base, p.head_groups, &base) || mul_ovf(base, p.dv_blocks, &base))) ||
        base > UINT32_MAX / threads)  // a dispatch counts its work-items in 32 bits
        return too_large_dim("workgroups", base, UINT32_MAX / threads);
    // The latent body has two functions: hi + lo weights (the default, as
    // precise as the other bodies) and, on request, bf16 weights.
    const int fn = which == 6 && !(c.flags & SGL_KV_ATTN_FAST_WEIGHTS) ? 9 : which;
    if (ctx->attention_occupancy_lds[fn] != lds) {
        int per_cu = 0;
        SGLKV_CHECK_HIP(hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, ctx->attention[fn],
                                                                           (int)threads, lds));
        ctx->attention_occupancy[fn] = per_cu > 0 ? (uint32_t)per_cu : 1;
        ctx->attention_occupancy_lds[fn] = lds;
    }
    const uint64_t target =
        (uint64_t)ctx->attention_occupancy[fn] * (uint64_t)(ctx->cu_count > 0 ? ctx->cu_count : 256);
    const uint64_t want = base >= target ? 1 : target / base;
    uint64_t chunk = ceil_div(max_len, want);
    // The shortest chunk a split takes. Small batches split further when
    // the combine merges many splits per memory round (both combines spread
    // a query's split groups over several waves or thread sets), which puts
    // more CUs to work. Measured:
    //  - staged bodies (GQA dims 128 / 64, 32 heads over 8 KV heads, 4,096
    //    tokens): 1 query 23.3 -> 15.5 us / 16.7 -> 11.8 us at 64 tokens
    //    against 256, 2 queries 24.6 -> 17.8 / 17.5 -> 12.2, 4 queries 26.4
    //    -> 23.3 / 18.8 -> 15.9; from 16 queries on the split count is set
    //    by the occupancy target, not by this minimum. The dims-128 body
    //    with K in registers (eight waves per CU) takes 128: at 64, 4
    //    queries took 22.4 us against 20.6;
    //  - latent body (MLA over 8,192 tokens): 64 tokens for one workgroup
    //    before splitting, 128 for two or three (1 query 40.0 -> 33.2 us,
    //    2 queries 41.0 -> 35.2 us), 256 from four on (best there);
    //  - the other bodies keep 256 (not measured otherwise).
    const uint64_t min_chunk = which == 11                 ? 128
                               : which >= 7                ? 64
                               : which == 6 && base < 4    ? (base <= 1 ? 64 : 128)
                                                           : 256;
    chunk = ceil_div(chunk < min_chunk ? min_chunk : chunk, SGLKV_ATTN_TOKENS) * SGLKV_ATTN_TOKENS;
    uint64_t splits = ceil_div(max_len, chunk);
    const uint64_t table = wide ? SGLKV_ATTN_WIDE_SLOTS : which >= 7 ? SGLKV_ATTN_STAGED_SLOTS : 0;
    if (table && chunk > table) {  // the slot table of the wide, latent and staged bodies
        chunk = table;
        splits = ceil_div(max_len, chunk);
    }
    if (splits > 65535) {  // grid y limit
        chunk = ceil_div(ceil_div(max_len, 65535), SGLKV_ATTN_TOKENS) * SGLKV_ATTN_TOKENS;
        splits = ceil_div(max_len, chunk);
    }
    p.chunk_tokens = chunk;
    p.splits = (uint32_t)splits;

    // The latent body writes scaled fp16 records (SGLKV_ATTN_HPAD), the
    // others fp32 ones (SGLKV_ATTN_OPAD).
    const bool half_records = which == 6;
    // The fp16 records and their combine are laid out for the latent body's
    // 512-wide values (SGLKV_ATTN_HPAD); nothing else selects that body.
    if (half_records && p.dv != 512)
        return fail(SGL_KV_INVALID_ARGUMENT, "value_head_dim", p.dv, 512, 0,
                    "the latent body's fp16 split records need 512-wide values, not %u", (unsigned)p.dv);
    if (splits > 1) {
        uint64_t bytes;
        const uint64_t per_record = half_records ? 2ull * SGLKV_ATTN_HPAD(p.dv) + 16 : 4ull * (SGLKV_ATTN_OPAD(p.dv) + 2);
        if (mul_ovf(c.query_count * c.query_head_count, splits, &bytes) || mul_ovf(bytes, per_record, &bytes))
            return attn_overflow();
        if (workspace) {
            if (bytes > workspace_bytes)
                return fail(SGL_KV_DIMENSION_TOO_LARGE, "workspace", bytes, workspace_bytes, 0,
                            "paged attention needs %llu bytes of split records, more than the "
                            "%llu-byte workspace",
                            (unsigned long long)bytes, (unsigned long long)workspace_bytes);
        } else if (bytes > ctx->attention_partial_bytes) {
            if (ctx->attention_partial) {
                SGLKV_CHECK_HIP(hipDeviceSynchronize());
                SGLKV_CHECK_HIP(hipFree(ctx->attention_partial));
                ctx->attention_partial = nullptr;
                ctx->attention_partial_bytes = 0;
            }
            SGLKV_CHECK_HIP(hipMalloc(&ctx->attention_partial, bytes));
            ctx->attention_partial_bytes = bytes;
        }
        p.partial = static_cast<float *>(workspace ? workspace : ctx->attention_partial);
    }
    // The combine pass: one workgroup per (query, head); the fp16 one in
    // blocks of 64 per 8 groups of 8 heads (its XCD map), padded.
    uint64_t combine_grid = 0;
    if (splits > 1) {
        uint64_t heads;
        if (mul_ovf(c.query_count, c.query_head_count, &heads)) return attn_overflow();
        combine_grid = half_records ? 64 * ceil_div(c.query_count * ceil_div(c.query_head_count, 8), 8) : heads;
        const uint64_t limit = UINT32_MAX / (half_records ? 256 : 128);  // work-items in 32 bits
        if (heads > limit / 2 || combine_grid > limit)
            return too_large_dim("combine workgroups", heads, limit / 2);
    }
    void *args[] = {&p};
    SGLKV_CHECK_HIP(hipModuleLaunchKernel(ctx->attention[fn], (unsigned)base, (unsigned)splits, 1, threads,
                                          1, 1, lds, s, args, nullptr));
    // The fp16 combine: one wave per group of eight splits, up to four.
    const unsigned combine_threads = half_records ? 64 * (unsigned)(splits > 24 ? 4 : ceil_div(splits, 8)) : 128;
    if (splits > 1)
        SGLKV_CHECK_HIP(hipModuleLaunchKernel(half_records ? ctx->attention_combine_h : ctx->attention_combine,
                                              (unsigned)combine_grid, 1, 1, combine_threads, 1, 1, 0, s, args,
                                              nullptr));
    return SGL_KV_OK;
}

}  // namespace

extern "C" int32_t sgl_rocm_kv_paged_attention(sgl_rocm_kv_ctx *ctx, const sgl_kv_attention_plan *plan,
                                               const sgl_kv_attention_buffers *b,
                                               uint64_t max_sequence_length, void *stream) {
    if (!ctx) return fail(SGL_KV_INVALID_ARGUMENT, "ctx", 0, 0, 0, "null argument");
    hipStream_t s = static_cast<hipStream_t>(stream);
    // The synchronous forward has an error word of its own, as the
    // reference's kernels object has its flag (cuda_attention.rs:667,
    // 706-707): asynchronous launches still running on other streams raise
    // the asynchronous word, so nothing here can take or clear their bits.
    // Calls on one context do not overlap, so the word is clean on entry:
    // every synchronous call leaves it zero.
    int32_t rc = attention_enqueue(ctx, plan, b, max_sequence_length, s, ctx->sync_attn_flag);
    if (rc) return rc;
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    SGLKV_CHECK_HIP(hipStreamSynchronize(s));
    uint32_t flag = 0;
    SGLKV_CHECK_HIP(hipMemcpy(&flag, ctx->sync_attn_flag, sizeof flag, hipMemcpyDeviceToHost));
    if (flag) SGLKV_CHECK_HIP(hipMemset(ctx->sync_attn_flag, 0, sizeof(uint32_t)));
    return attention_flag_status(flag);
}

extern "C" int32_t sgl_rocm_kv_paged_attention_async(sgl_rocm_kv_ctx *ctx,
                                                     const sgl_kv_attention_plan *plan,
                                                     const sgl_kv_attention_buffers *b,
                                                     uint64_t max_sequence_length, void *stream) {
    if (!ctx) return fail(SGL_KV_INVALID_ARGUMENT, "ctx", 0, 0, 0, "null argument");
    const int32_t rc =
        attention_enqueue(ctx, plan, b, max_sequence_length, static_cast<hipStream_t>(stream), ctx->attn_flag);
    return rc ? rc : ok();
}

extern "C" int32_t sgl_rocm_kv_paged_attention_async_noalloc(sgl_rocm_kv_ctx *ctx,
                                                             const sgl_kv_attention_plan *plan,
                                                             const sgl_kv_attention_buffers *b,
                                                             uint64_t max_sequence_length, void *stream) {
    if (!ctx) return fail(SGL_KV_INVALID_ARGUMENT, "ctx", 0, 0, 0, "null argument");
    if (!ctx->noalloc_workspace || !ctx->noalloc_order)
        return fail(SGL_KV_MODULE, "workspace", 0, 0, 0, "the context has no workspace address");
    hipStream_t s = static_cast<hipStream_t>(stream);
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    // Every call on this device shares the workspace. The device's event
    // marks the end of the last call that used it: this call's launches
    // wait for it on `s`, and the event then moves past this call's
    // combine. The lock makes wait, launch and record one step for all
    // host threads and contexts, so calls on any streams run in the order
    // they were made. Under stream capture the graph's own dependencies
    // order its launches (an event recorded outside the capture cannot be
    // waited on there), so the event is left alone.
    NoallocOrder *order = ctx->noalloc_order;
    std::lock_guard<std::mutex> guard(order->lock);
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    SGLKV_CHECK_HIP(hipStreamIsCapturing(s, &capture));
    const bool ordered = capture == hipStreamCaptureStatusNone;
    if (ordered) SGLKV_CHECK_HIP(hipStreamWaitEvent(s, order->last, 0));
    const int32_t rc = attention_enqueue(ctx, plan, b, max_sequence_length, s, ctx->attn_flag,
                                         ctx->noalloc_workspace, SGL_KV_NOALLOC_WORKSPACE_BYTES);
    // Recorded whatever the enqueue returned: a failure after its first
    // launch still leaves work on `s` that uses the workspace.
    const hipError_t rec = ordered ? hipEventRecord(order->last, s) : hipSuccess;
    if (rc) return rc;
    if (rec != hipSuccess) return hip_fail(rec, "hipEventRecord");
    return ok();
}
