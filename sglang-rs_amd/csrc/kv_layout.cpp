// kv_layout.cpp -- host mirror of the reference's KV layout arithmetic and
// copy plan (group 1 of sgl_rocm_kv.h). No HIP calls: these run on any host.
//
// Each function follows the reference item cited beside it: the same
// validation order, the same error variants (as sgl_kv_status codes with the
// variant's fields in a/b/c) and the same checked arithmetic.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "kv_internal.h"

namespace sglkv {

static thread_local sgl_kv_error_detail t_last;

int32_t fail(int32_t code, const char *name, uint64_t a, uint64_t b, uint64_t c, const char *fmt,
             ...) {
    memset(&t_last, 0, sizeof t_last);
    t_last.code = code;
    t_last.a = a;
    t_last.b = b;
    t_last.c = c;
    if (name) snprintf(t_last.name, sizeof t_last.name, "%s", name);
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(t_last.message, sizeof t_last.message, fmt, ap);
    va_end(ap);
    return code;
}

int32_t ok() {
    memset(&t_last, 0, sizeof t_last);
    return SGL_KV_OK;
}

void set_detail_d(uint64_t d) { t_last.d = d; }

}  // namespace sglkv

using namespace sglkv;

extern "C" void sgl_kv_last_error(sgl_kv_error_detail *out) {
    if (out) *out = t_last;
}

extern "C" const char *sgl_kv_status_name(int32_t code) {
    switch (code) {
    case SGL_KV_OK: return "Ok";
    case SGL_KV_ZERO_DIMENSION: return "ZeroDimension";
    case SGL_KV_SHAPE_OVERFLOW: return "ShapeOverflow";
    case SGL_KV_DIMENSION_TOO_LARGE: return "DimensionTooLarge";
    case SGL_KV_ROW_STRIDE_TOO_SMALL: return "RowStrideTooSmall";
    case SGL_KV_TENSOR_PAGE_REGION_OUT_OF_BOUNDS: return "TensorPageRegionOutOfBounds";
    case SGL_KV_TENSOR_PAGE_REGIONS_OVERLAP: return "TensorPageRegionsOverlap";
    case SGL_KV_DEVICE_MISMATCH: return "DeviceMismatch";
    case SGL_KV_DEVICE_SLOT_INDEX_OUT_OF_RANGE: return "DeviceSlotIndexOutOfRange";
    case SGL_KV_HIP: return "Hip";
    case SGL_KV_MODULE: return "Module";
    case SGL_KV_ALLOCATION_OUT_OF_BOUNDS: return "AllocationOutOfBounds";
    case SGL_KV_INVALID_ARGUMENT: return "InvalidArgument";
    case SGL_KV_LAYOUT_ZERO_PAGE_COUNT: return "ZeroPageCount";
    case SGL_KV_LAYOUT_ZERO_FIELD: return "ZeroLayoutField";
    case SGL_KV_LAYOUT_RUNTIME_PAGE_SIZE_MISMATCH: return "RuntimePageSizeMismatch";
    case SGL_KV_LAYOUT_UNEVEN_LAYER: return "UnevenLayerLayout";
    case SGL_KV_LAYOUT_UNEVEN_TENSOR: return "UnevenTensorLayout";
    case SGL_KV_LAYOUT_SIZE_OVERFLOW: return "SizeOverflow";
    case SGL_KV_LAYOUT_PAGE_OUT_OF_RANGE: return "PageOutOfRange";
    case SGL_KV_LAYOUT_LAYER_OUT_OF_RANGE: return "LayerOutOfRange";
    case SGL_KV_LAYOUT_TENSOR_OUT_OF_RANGE: return "TensorOutOfRange";
    case SGL_KV_LAYOUT_TOKEN_OUT_OF_RANGE: return "TokenOutOfRange";
    case SGL_KV_LAYOUT_SLOT_OUT_OF_RANGE: return "SlotOutOfRange";
    case SGL_KV_LAYOUT_EMPTY_SLOT_MAP: return "EmptySlotMap";
    case SGL_KV_LAYOUT_BATCH_SLOT_OUT_OF_RANGE: return "BatchSlotOutOfRange";
    case SGL_KV_ATTN_INVALID_SCALE: return "InvalidScale";
    case SGL_KV_ATTN_QUERY_HEADS_NOT_DIVISIBLE: return "QueryHeadsNotDivisibleByKvHeads";
    case SGL_KV_ATTN_KEY_ROW_BYTES_MISMATCH: return "KvRowByteSizeMismatch";
    case SGL_KV_ATTN_VALUE_ROW_BYTES_MISMATCH: return "ValueRowByteSizeMismatch";
    case SGL_KV_ATTN_TENSOR_PAGE_REGIONS_OVERLAP: return "TensorPageRegionsOverlap";
    case SGL_KV_ATTN_DEVICE_METADATA_INVALID: return "DeviceMetadataInvalid";
    case SGL_KV_ATTN_UNSUPPORTED_KV_DTYPE: return "UnsupportedKvDtype";
    case SGL_KV_ATTN_TENSOR_ROW_GEOMETRY_MISMATCH: return "TensorRowGeometryMismatch";
    case SGL_KV_BOOT_MISSING_FIELD: return "MissingField";
    case SGL_KV_BOOT_UTF8_FIELD: return "Utf8Field";
    case SGL_KV_BOOT_INTEGER_FIELD: return "IntegerField";
    case SGL_KV_BOOT_BINARY_LENGTH: return "BinaryLength";
    case SGL_KV_BOOT_PACKED_LIST_HEADER: return "PackedListHeader";
    case SGL_KV_BOOT_PACKED_LIST_LENGTH: return "PackedListLength";
    case SGL_KV_BOOT_MISSING_TRANSFER_ROOM: return "MissingTransferRoom";
    case SGL_KV_BOOT_MISSING_KV_ARGS: return "MissingKvArgsRegistration";
    case SGL_KV_BOOT_MISSING_AUX_INDEX: return "MissingAuxIndex";
    case SGL_KV_BOOT_DECODE_LAYOUT: return "DecodeLayout";
    case SGL_KV_MODEL_DTYPE_REQUIRES_MODEL_METADATA: return "DtypeRequiresModelMetadata";
    case SGL_KV_MODEL_INVALID_PACKED_MLA_NOPE_HEAD_DIM: return "InvalidPackedMlaNopeHeadDim";
    case SGL_KV_MODEL_ZERO_TENSOR_WIDTH: return "ZeroTensorWidth";
    case SGL_KV_MODEL_SIZE_OVERFLOW: return "SizeOverflow";
    case SGL_KV_MODEL_MISSING_CAPABILITY: return "MissingCapabilities";
    case SGL_KV_LAYOUT_KV_PAIR_REQUIRES_TWO_TENSORS: return "KvPairRequiresTwoTensors";
    case SGL_KV_LAYOUT_TENSOR_PAIR_REQUIRES_TWO_TENSORS: return "TensorPairRequiresTwoTensors";
    case SGL_KV_LAYOUT_TENSOR_PAIR_SIZE_MISMATCH: return "TensorPairSizeMismatch";
    case SGL_KV_LAYOUT_UNEVEN_KV_PAIR_COPY: return "UnevenKvPairCopy";
    case SGL_KV_PLAN_ZERO_PAGE_SIZE: return "ZeroPageSize";
    case SGL_KV_PLAN_CACHE_PAGE_COUNT_MISMATCH: return "CachePageCountMismatch";
    case SGL_KV_PLAN_TRAILING_CACHE_PAGES: return "TrailingCachePages";
    case SGL_KV_PLAN_UNALIGNED_TOKEN_OFFSET: return "UnalignedTokenOffset";
    case SGL_KV_PLAN_UNALIGNED_CACHE_SLOT: return "UnalignedCacheSlot";
    case SGL_KV_PLAN_NON_CONTIGUOUS_CACHE_SLOTS: return "NonContiguousCacheSlots";
    case SGL_KV_PLAN_NON_PREFILL_BATCH: return "NonPrefillBatch";
    case SGL_KV_DEVICE_PAGE_INDEX_OUT_OF_RANGE: return "DevicePageIndexOutOfRange";
    case SGL_KV_DEVICE_SPAN_OUT_OF_RANGE: return "DeviceSpanOutOfRange";
    case SGL_KV_DEVICE_REQUEST_OUT_OF_RANGE: return "DeviceRequestOutOfRange";
    case SGL_KV_REQ_ZERO_PAGE_SIZE: return "ZeroPageSize";
    case SGL_KV_REQ_ZERO_REMOTE_ITEM_SIZE: return "ZeroRemoteKvItemSize";
    case SGL_KV_REQ_MISSING_REMOTE_POINTERS: return "MissingRemoteKvPointers";
    case SGL_KV_REQ_SPAN_PAGE_COUNT_MISMATCH: return "SpanPageCountMismatch";
    case SGL_KV_REQ_REMOTE_INDEX_COUNT_MISMATCH: return "RemoteKvIndexCountMismatch";
    case SGL_KV_REQ_REMOTE_ITEM_LAYOUT_MISMATCH: return "RemoteKvItemLayoutMismatch";
    case SGL_KV_REQ_NEGATIVE_REMOTE_INDEX: return "NegativeRemoteKvIndex";
    case SGL_KV_REQ_ADDRESS_OVERFLOW: return "AddressOverflow";
    case SGL_KV_REQ_OFFSET_OVERFLOW: return "OffsetOverflow";
    case SGL_KV_ALLOC_ZERO_PAGE_SIZE: return "ZeroPageSize";
    case SGL_KV_ALLOC_ZERO_SLOT_CAPACITY: return "ZeroSlotCapacity";
    case SGL_KV_ALLOC_SLOT_CAPACITY_NOT_PAGE_ALIGNED: return "SlotCapacityNotPageAligned";
    case SGL_KV_ALLOC_OUT_OF_SLOTS: return "OutOfSlots";
    case SGL_KV_RADIX_TOKEN_PAGE_LENGTH_MISMATCH: return "TokenPageLengthMismatch";
    case SGL_KV_STORAGE_SIZE_MISMATCH: return "StorageSizeMismatch";
    case SGL_KV_STORAGE_SLOT_MAP_CAPACITY_MISMATCH: return "SlotMapCapacityMismatch";
    case SGL_KV_STORAGE_PAGE_BUFFER_SIZE_MISMATCH: return "PageBufferSizeMismatch";
    case SGL_KV_STORAGE_SIZE_OVERFLOW: return "SizeOverflow";
    case SGL_KV_ZERO_ALLOCATION: return "ZeroAllocation";
    case SGL_KV_UNSUPPORTED_MEMORY_LOCATION: return "UnsupportedMemoryLocation";
    case SGL_KV_STORAGE_DESCRIPTOR: return "Descriptor";
    default: return "Unknown";
    }
}

// KvCacheDtype::bytes_per_element (crates/sglang-srt/src/kv_cache.rs:39-46).
extern "C" size_t sgl_kv_dtype_bytes_per_element(int32_t dtype) {
    switch (dtype) {
    case SGL_KV_DTYPE_AUTO:
    case SGL_KV_DTYPE_BFLOAT16: return 2;
    case SGL_KV_DTYPE_FLOAT32: return 4;
    case SGL_KV_DTYPE_FP8_E4M3:
    case SGL_KV_DTYPE_FP8_E5M2: return 1;
    default: return 0;
    }
}

// --- KvCacheModelLayout (crates/sglang-srt/src/kv_cache.rs:68-225) ---

static const char *dtype_name(int32_t dtype) {
    // KvCacheDtype::as_str (kv_cache.rs:28-37)
    switch (dtype) {
    case SGL_KV_DTYPE_AUTO: return "auto";
    case SGL_KV_DTYPE_FLOAT32: return "float32";
    case SGL_KV_DTYPE_BFLOAT16: return "bfloat16";
    case SGL_KV_DTYPE_FP8_E4M3: return "fp8_e4m3";
    case SGL_KV_DTYPE_FP8_E5M2: return "fp8_e5m2";
    case SGL_KV_DTYPE_FP4_E2M1: return "fp4_e2m1";
    default: return "unknown";
    }
}

static int32_t model_overflow() {
    return fail(SGL_KV_MODEL_SIZE_OVERFLOW, nullptr, 0, 0, 0, "KV cache layout byte size overflowed");
}

static int32_t model_dtype_width(int32_t dtype, uint64_t *width) {
    *width = sgl_kv_dtype_bytes_per_element(dtype);
    if (*width == 0)
        return fail(SGL_KV_MODEL_DTYPE_REQUIRES_MODEL_METADATA, nullptr, (uint64_t)(int64_t)dtype, 0, 0,
                    "KV cache dtype %s requires model metadata for byte width", dtype_name(dtype));
    return SGL_KV_OK;
}

extern "C" int32_t sgl_kv_model_layout_multi_tensor(uint64_t num_layers, uint64_t kv_heads, uint64_t head_dim,
                                                    uint64_t kv_tensors_per_token, sgl_kv_model_layout *out) {
    if (!out) return fail(SGL_KV_INVALID_ARGUMENT, "out", 0, 0, 0, "null argument");
    memset(out, 0, sizeof *out);
    out->num_layers = num_layers;
    out->kv_heads = kv_heads;
    out->head_dim = head_dim;
    out->kv_tensors_per_token = kv_tensors_per_token;
    out->geometry = SGL_KV_GEOMETRY_UNIFORM;
    return ok();
}

extern "C" int32_t sgl_kv_model_layout_tensor_pair(uint64_t num_layers, uint64_t key_heads, uint64_t key_head_dim,
                                                   uint64_t value_heads, uint64_t value_head_dim,
                                                   sgl_kv_model_layout *out) {
    if (!out) return fail(SGL_KV_INVALID_ARGUMENT, "out", 0, 0, 0, "null argument");
    uint64_t key_elements, value_elements;
    if (mul_ovf(key_heads, key_head_dim, &key_elements) || mul_ovf(value_heads, value_head_dim, &value_elements))
        return model_overflow();
    if (key_elements == 0 || value_elements == 0)
        return fail(SGL_KV_MODEL_ZERO_TENSOR_WIDTH, nullptr, 0, 0, 0, "KV cache tensor width must be non-zero");
    memset(out, 0, sizeof *out);
    out->num_layers = num_layers;
    out->kv_heads = key_heads;
    out->head_dim = key_head_dim;
    out->kv_tensors_per_token = 2;
    out->geometry = SGL_KV_GEOMETRY_PAIR;
    out->key_elements = key_elements;
    out->value_elements = value_elements;
    return ok();
}

extern "C" int32_t sgl_kv_model_layout_packed_bytes_per_layer(uint64_t num_layers, uint64_t bytes_per_token_per_layer,
                                                              sgl_kv_model_layout *out) {
    if (!out) return fail(SGL_KV_INVALID_ARGUMENT, "out", 0, 0, 0, "null argument");
    memset(out, 0, sizeof *out);
    out->num_layers = num_layers;
    out->kv_heads = 1;
    out->head_dim = bytes_per_token_per_layer;
    out->kv_tensors_per_token = 1;
    out->bytes_per_token_per_layer = bytes_per_token_per_layer;
    out->geometry = SGL_KV_GEOMETRY_PACKED_BYTES;
    return ok();
}

extern "C" int32_t sgl_kv_model_layout_packed_mla(uint64_t num_layers, uint64_t qk_nope_head_dim,
                                                  uint64_t qk_rope_head_dim, sgl_kv_model_layout *out) {
    if (!out) return fail(SGL_KV_INVALID_ARGUMENT, "out", 0, 0, 0, "null argument");
    if (qk_nope_head_dim % 64)
        return fail(SGL_KV_MODEL_INVALID_PACKED_MLA_NOPE_HEAD_DIM, nullptr, qk_nope_head_dim, 0, 0,
                    "qk_nope_head_dim must be divisible by 64 for packed MLA KV layout: %llu",
                    (unsigned long long)qk_nope_head_dim);
    // nope + 2 * rope + nope / 64 + 1 bytes, checked as the reference adds them
    uint64_t bytes;
    if (mul_ovf(qk_rope_head_dim, 2, &bytes) || add_ovf(qk_nope_head_dim, bytes, &bytes) ||
        add_ovf(bytes, qk_nope_head_dim / 64, &bytes) || add_ovf(bytes, 1, &bytes))
        return model_overflow();
    return sgl_kv_model_layout_packed_bytes_per_layer(num_layers, bytes, out);
}

extern "C" int32_t sgl_kv_model_layout_elements_per_token(const sgl_kv_model_layout *l, uint64_t *out,
                                                          uint32_t *has) {
    if (!l || !out || !has) return fail(SGL_KV_INVALID_ARGUMENT, "layout/out/has", 0, 0, 0, "null argument");
    *out = 0;
    *has = 0;
    uint64_t per_layer;
    if (l->geometry == SGL_KV_GEOMETRY_UNIFORM) {
        if (mul_ovf(l->kv_tensors_per_token, l->kv_heads, &per_layer) || mul_ovf(per_layer, l->head_dim, &per_layer))
            return ok();
    } else if (l->geometry == SGL_KV_GEOMETRY_PAIR) {
        if (add_ovf(l->key_elements, l->value_elements, &per_layer)) return ok();
    } else {
        return ok();
    }
    if (mul_ovf(l->num_layers, per_layer, out)) {
        *out = 0;
        return ok();
    }
    *has = 1;
    return ok();
}

extern "C" int32_t sgl_kv_model_layout_token_size_bytes(const sgl_kv_model_layout *l, int32_t dtype, uint64_t *out) {
    if (!l || !out) return fail(SGL_KV_INVALID_ARGUMENT, "layout/out", 0, 0, 0, "null argument");
    *out = 0;
    if (l->geometry == SGL_KV_GEOMETRY_PACKED_BYTES || l->bytes_per_token_per_layer) {
        if (mul_ovf(l->num_layers, l->bytes_per_token_per_layer, out)) return model_overflow();
        return ok();
    }
    uint64_t elements;
    uint32_t has;
    sgl_kv_model_layout_elements_per_token(l, &elements, &has);
    if (!has) return model_overflow();
    uint64_t width;
    int32_t rc = model_dtype_width(dtype, &width);
    if (rc) return rc;
    if (mul_ovf(elements, width, out)) return model_overflow();
    return ok();
}

extern "C" int32_t sgl_kv_model_layout_tensor_pair_size_bytes(const sgl_kv_model_layout *l, int32_t dtype,
                                                              uint64_t out[2], uint32_t *is_pair) {
    if (!l || !out || !is_pair) return fail(SGL_KV_INVALID_ARGUMENT, "layout/out/is_pair", 0, 0, 0, "null argument");
    out[0] = out[1] = 0;
    *is_pair = 0;
    if (l->geometry != SGL_KV_GEOMETRY_PAIR) return ok();
    uint64_t width;
    int32_t rc = model_dtype_width(dtype, &width);
    if (rc) return rc;
    if (mul_ovf(l->key_elements, width, &out[0]) || mul_ovf(l->value_elements, width, &out[1])) {
        out[0] = out[1] = 0;
        return model_overflow();
    }
    *is_pair = 1;
    return ok();
}

static int32_t layout_overflow() {
    return fail(SGL_KV_LAYOUT_SIZE_OVERFLOW, nullptr, 0, 0, 0, "KV cache layout size overflowed");
}

// PagedKvCacheLayout::validate_runtime (kv_cache.rs:531-586).
static int32_t validate_runtime(const sgl_kv_runtime_layout *rt, uint64_t page_count,
                                sgl_kv_paged_layout *out) {
    if (page_count == 0)
        return fail(SGL_KV_LAYOUT_ZERO_PAGE_COUNT, nullptr, 0, 0, 0,
                    "KV cache page count must be non-zero");
    const struct {
        const char *field;
        uint64_t value;
    } fields[] = {{"page_size", rt->page_size},
                  {"num_layers", rt->num_layers},
                  {"kv_heads", rt->kv_heads},
                  {"head_dim", rt->head_dim},
                  {"kv_tensors_per_token", rt->kv_tensors_per_token},
                  {"bytes_per_token", rt->bytes_per_token},
                  {"page_size_bytes", rt->page_size_bytes}};
    for (const auto &f : fields)
        if (f.value == 0)
            return fail(SGL_KV_LAYOUT_ZERO_FIELD, f.field, 0, 0, 0,
                        "KV cache layout field %s must be non-zero", f.field);
    uint64_t expected;
    if (mul_ovf(rt->page_size, rt->bytes_per_token, &expected)) return layout_overflow();
    if (rt->page_size_bytes != expected)
        return fail(SGL_KV_LAYOUT_RUNTIME_PAGE_SIZE_MISMATCH, nullptr, expected, rt->page_size_bytes, 0,
                    "KV cache runtime page size is %llu bytes but page_size * bytes_per_token "
                    "requires %llu bytes",
                    (unsigned long long)rt->page_size_bytes, (unsigned long long)expected);
    if (rt->bytes_per_token % rt->num_layers)
        return fail(SGL_KV_LAYOUT_UNEVEN_LAYER, nullptr, rt->bytes_per_token, rt->num_layers, 0,
                    "KV cache token size %llu bytes is not divisible by %llu layers",
                    (unsigned long long)rt->bytes_per_token, (unsigned long long)rt->num_layers);
    memset(out, 0, sizeof *out);
    out->runtime = *rt;
    out->page_count = page_count;
    out->bytes_per_token_per_layer = rt->bytes_per_token / rt->num_layers;
    if (mul_ovf(rt->page_size, out->bytes_per_token_per_layer, &out->bytes_per_layer_page) ||
        mul_ovf(page_count, rt->page_size_bytes, &out->total_byte_len) ||
        mul_ovf(page_count, rt->page_size, &out->slot_count))
        return layout_overflow();
    return SGL_KV_OK;
}

// PagedKvCacheLayout::new (kv_cache.rs:448-478): Uniform geometry.
extern "C" int32_t sgl_kv_paged_layout_new(const sgl_kv_runtime_layout *runtime,
                                           uint64_t page_count, sgl_kv_paged_layout *out) {
    if (!runtime || !out)
        return fail(SGL_KV_INVALID_ARGUMENT, "runtime/out", 0, 0, 0, "null argument");
    sgl_kv_paged_layout l;
    int32_t rc = validate_runtime(runtime, page_count, &l);
    if (rc) return rc;
    if (l.bytes_per_token_per_layer % runtime->kv_tensors_per_token)
        return fail(SGL_KV_LAYOUT_UNEVEN_TENSOR, nullptr, l.bytes_per_token_per_layer,
                    runtime->kv_tensors_per_token, 0,
                    "KV cache per-layer token size %llu bytes is not divisible by %llu KV tensors",
                    (unsigned long long)l.bytes_per_token_per_layer,
                    (unsigned long long)runtime->kv_tensors_per_token);
    const uint64_t token_bytes = l.bytes_per_token_per_layer / runtime->kv_tensors_per_token;
    if (mul_ovf(runtime->page_size, token_bytes, &l.tensor_page_bytes)) return layout_overflow();
    l.tensor_pair = 0;
    l.token_bytes[0] = l.token_bytes[1] = token_bytes;
    *out = l;
    return ok();
}

// PagedKvCacheLayout::new_with_tensor_pair (kv_cache.rs:480-529).
extern "C" int32_t sgl_kv_paged_layout_new_with_tensor_pair(const sgl_kv_runtime_layout *runtime,
                                                            uint64_t page_count,
                                                            uint64_t key_token_bytes,
                                                            uint64_t value_token_bytes,
                                                            sgl_kv_paged_layout *out) {
    if (!runtime || !out)
        return fail(SGL_KV_INVALID_ARGUMENT, "runtime/out", 0, 0, 0, "null argument");
    sgl_kv_paged_layout l;
    int32_t rc = validate_runtime(runtime, page_count, &l);
    if (rc) return rc;
    if (runtime->kv_tensors_per_token != 2)
        return fail(SGL_KV_LAYOUT_TENSOR_PAIR_REQUIRES_TWO_TENSORS, nullptr,
                    runtime->kv_tensors_per_token, 0, 0,
                    "explicit KV tensor-pair layout requires exactly two tensors per token, layout "
                    "has %llu",
                    (unsigned long long)runtime->kv_tensors_per_token);
    if (key_token_bytes == 0)
        return fail(SGL_KV_LAYOUT_ZERO_FIELD, "key_token_bytes", 0, 0, 0,
                    "KV cache layout field key_token_bytes must be non-zero");
    if (value_token_bytes == 0)
        return fail(SGL_KV_LAYOUT_ZERO_FIELD, "value_token_bytes", 0, 0, 0,
                    "KV cache layout field value_token_bytes must be non-zero");
    uint64_t pair;
    if (add_ovf(key_token_bytes, value_token_bytes, &pair)) return layout_overflow();
    if (pair != l.bytes_per_token_per_layer)
        return fail(SGL_KV_LAYOUT_TENSOR_PAIR_SIZE_MISMATCH, nullptr, l.bytes_per_token_per_layer,
                    key_token_bytes, value_token_bytes,
                    "KV tensor-pair widths (%llu key bytes + %llu value bytes) do not match the "
                    "runtime per-layer token size of %llu bytes",
                    (unsigned long long)key_token_bytes, (unsigned long long)value_token_bytes,
                    (unsigned long long)l.bytes_per_token_per_layer);
    if (mul_ovf(runtime->page_size, key_token_bytes, &l.tensor_page_bytes)) return layout_overflow();
    l.tensor_pair = 1;
    l.token_bytes[0] = key_token_bytes;
    l.token_bytes[1] = value_token_bytes;
    *out = l;
    return ok();
}

static int32_t validate_page(const sgl_kv_paged_layout *l, uint64_t page) {
    if (page >= l->page_count)
        return fail(SGL_KV_LAYOUT_PAGE_OUT_OF_RANGE, nullptr, page, l->page_count, 0,
                    "KV cache page index %llu is outside %llu pages", (unsigned long long)page,
                    (unsigned long long)l->page_count);
    return SGL_KV_OK;
}

static int32_t tensor_out_of_range(const sgl_kv_paged_layout *l, uint64_t tensor) {
    return fail(SGL_KV_LAYOUT_TENSOR_OUT_OF_RANGE, nullptr, tensor,
                l->runtime.kv_tensors_per_token, 0,
                "KV cache tensor index %llu is outside %llu tensors per token",
                (unsigned long long)tensor, (unsigned long long)l->runtime.kv_tensors_per_token);
}

// tensor_token_bytes / tensor_page_offset (kv_cache.rs:780-818).
static int32_t tensor_geometry(const sgl_kv_paged_layout *l, uint64_t tensor, uint64_t *token_bytes,
                               uint64_t *page_offset) {
    if (!l->tensor_pair) {
        *token_bytes = l->token_bytes[0];
        if (mul_ovf(tensor, l->tensor_page_bytes, page_offset)) return layout_overflow();
        return SGL_KV_OK;
    }
    if (tensor > 1) return tensor_out_of_range(l, tensor);
    *token_bytes = l->token_bytes[tensor];
    *page_offset = tensor == 0 ? 0 : l->tensor_page_bytes;
    return SGL_KV_OK;
}

// PagedKvCacheLayout::page_byte_range (kv_cache.rs:639-651).
extern "C" int32_t sgl_kv_paged_layout_page_byte_range(const sgl_kv_paged_layout *layout,
                                                       uint64_t page_index, uint64_t *start,
                                                       uint64_t *end) {
    if (!layout || !start || !end)
        return fail(SGL_KV_INVALID_ARGUMENT, "layout/start/end", 0, 0, 0, "null argument");
    int32_t rc = validate_page(layout, page_index);
    if (rc) return rc;
    uint64_t s, e;
    if (mul_ovf(page_index, layout->runtime.page_size_bytes, &s) ||
        add_ovf(s, layout->runtime.page_size_bytes, &e))
        return layout_overflow();
    *start = s;
    *end = e;
    return ok();
}

// PagedKvCacheLayout::tensor_token_byte_range (kv_cache.rs:653-700).
extern "C" int32_t sgl_kv_paged_layout_tensor_token_byte_range(const sgl_kv_paged_layout *layout,
                                                               uint64_t page_index,
                                                               uint64_t layer_index,
                                                               uint64_t tensor_index,
                                                               uint64_t token_index,
                                                               uint64_t *start, uint64_t *end) {
    if (!layout || !start || !end)
        return fail(SGL_KV_INVALID_ARGUMENT, "layout/start/end", 0, 0, 0, "null argument");
    int32_t rc = validate_page(layout, page_index);
    if (rc) return rc;
    const sgl_kv_runtime_layout &rt = layout->runtime;
    if (layer_index >= rt.num_layers)
        return fail(SGL_KV_LAYOUT_LAYER_OUT_OF_RANGE, nullptr, layer_index, rt.num_layers, 0,
                    "KV cache layer index %llu is outside %llu layers",
                    (unsigned long long)layer_index, (unsigned long long)rt.num_layers);
    if (tensor_index >= rt.kv_tensors_per_token) return tensor_out_of_range(layout, tensor_index);
    if (token_index >= rt.page_size)
        return fail(SGL_KV_LAYOUT_TOKEN_OUT_OF_RANGE, nullptr, token_index, rt.page_size, 0,
                    "KV cache token index %llu is outside page size %llu",
                    (unsigned long long)token_index, (unsigned long long)rt.page_size);
    uint64_t page_off, layer_off, tensor_off, token_bytes, token_off, s, e;
    if (mul_ovf(page_index, rt.page_size_bytes, &page_off) ||
        mul_ovf(layer_index, layout->bytes_per_layer_page, &layer_off))
        return layout_overflow();
    rc = tensor_geometry(layout, tensor_index, &token_bytes, &tensor_off);
    if (rc) return rc;
    if (mul_ovf(token_index, token_bytes, &token_off) || add_ovf(page_off, layer_off, &s) ||
        add_ovf(s, tensor_off, &s) || add_ovf(s, token_off, &s) || add_ovf(s, token_bytes, &e))
        return layout_overflow();
    *start = s;
    *end = e;
    return ok();
}

// PagedKvCacheLayout::tensor_slot_byte_range (kv_cache.rs:702-720).
extern "C" int32_t sgl_kv_paged_layout_tensor_slot_byte_range(const sgl_kv_paged_layout *layout,
                                                              uint64_t layer_index,
                                                              uint64_t tensor_index,
                                                              uint64_t slot_index, uint64_t *start,
                                                              uint64_t *end) {
    if (!layout || !start || !end)
        return fail(SGL_KV_INVALID_ARGUMENT, "layout/start/end", 0, 0, 0, "null argument");
    if (slot_index >= layout->slot_count)
        return fail(SGL_KV_LAYOUT_SLOT_OUT_OF_RANGE, nullptr, slot_index, layout->slot_count, 0,
                    "KV cache slot index %llu is outside %llu token slots",
                    (unsigned long long)slot_index, (unsigned long long)layout->slot_count);
    const uint64_t ps = layout->runtime.page_size;
    return sgl_kv_paged_layout_tensor_token_byte_range(layout, slot_index / ps, layer_index,
                                                       tensor_index, slot_index % ps, start, end);
}

// PagedKvCacheLayout::validate_slot_indices (kv_cache.rs:722-736).
extern "C" int32_t sgl_kv_paged_layout_validate_slot_indices(const sgl_kv_paged_layout *layout,
                                                             const uint64_t *slots,
                                                             uint64_t slot_len) {
    if (!layout) return fail(SGL_KV_INVALID_ARGUMENT, "layout", 0, 0, 0, "null argument");
    if (slot_len == 0)
        return fail(SGL_KV_LAYOUT_EMPTY_SLOT_MAP, nullptr, 0, 0, 0,
                    "KV cache slot map must not be empty");
    if (!slots) return fail(SGL_KV_INVALID_ARGUMENT, "slots", 0, 0, 0, "null argument");
    for (uint64_t i = 0; i < slot_len; ++i)
        if (slots[i] >= layout->slot_count)
            return fail(SGL_KV_LAYOUT_BATCH_SLOT_OUT_OF_RANGE, nullptr, i, slots[i],
                        layout->slot_count,
                        "KV cache batch slot %llu references physical slot %llu, outside %llu "
                        "token slots",
                        (unsigned long long)i, (unsigned long long)slots[i],
                        (unsigned long long)layout->slot_count);
    return ok();
}

// PagedKvCacheLayout::kv_pair_copy_geometry (kv_cache.rs:738-777), returned as
// the CudaKvPairCopyLayout it feeds (crates/sglang-srt/src/cuda_kv_cache.rs:510-532).
extern "C" int32_t sgl_kv_paged_layout_kv_pair_copy_geometry(const sgl_kv_paged_layout *layout,
                                                             uint64_t layer_index,
                                                             sgl_kv_pair_copy_layout *out) {
    if (!layout || !out)
        return fail(SGL_KV_INVALID_ARGUMENT, "layout/out", 0, 0, 0, "null argument");
    const sgl_kv_runtime_layout &rt = layout->runtime;
    if (layer_index >= rt.num_layers)
        return fail(SGL_KV_LAYOUT_LAYER_OUT_OF_RANGE, nullptr, layer_index, rt.num_layers, 0,
                    "KV cache layer index %llu is outside %llu layers",
                    (unsigned long long)layer_index, (unsigned long long)rt.num_layers);
    if (rt.kv_tensors_per_token < 2)
        return fail(SGL_KV_LAYOUT_KV_PAIR_REQUIRES_TWO_TENSORS, nullptr, rt.kv_tensors_per_token, 0,
                    0,
                    "KV cache K/V pair layout requires at least two tensors per token, layout has "
                    "%llu",
                    (unsigned long long)rt.kv_tensors_per_token);
    uint64_t layer_off, kb, vb, ko, vo;
    if (mul_ovf(layer_index, layout->bytes_per_layer_page, &layer_off)) return layout_overflow();
    int32_t rc = tensor_geometry(layout, 0, &kb, &ko);
    if (rc) return rc;
    rc = tensor_geometry(layout, 1, &vb, &vo);
    if (rc) return rc;
    if (kb != vb)
        return fail(SGL_KV_LAYOUT_UNEVEN_KV_PAIR_COPY, nullptr, kb, vb, 0,
                    "the selected KV copy/attention kernel requires equal key and value widths, "
                    "but the layout has %llu key bytes and %llu value bytes per token",
                    (unsigned long long)kb, (unsigned long long)vb);
    if (add_ovf(layer_off, ko, &ko) || add_ovf(layer_off, vo, &vo)) return layout_overflow();
    out->page_size = rt.page_size;
    out->page_stride_bytes = rt.page_size_bytes;
    out->key_in_page_offset = ko;
    out->value_in_page_offset = vo;
    out->row_bytes = kb;
    return ok();
}

// CudaKvPairCopyPlan::new (crates/sglang-kernel/src/cuda_kv_kernels.rs:167-264).
extern "C" int32_t sgl_kv_pair_copy_plan_new(uint64_t row_count, uint64_t slot_count,
                                             const sgl_kv_pair_copy_layout *layout,
                                             uint64_t key_row_stride_bytes,
                                             uint64_t value_row_stride_bytes,
                                             sgl_kv_pair_copy_plan *out) {
    if (!layout || !out)
        return fail(SGL_KV_INVALID_ARGUMENT, "layout/out", 0, 0, 0, "null argument");
    const struct {
        const char *dimension;
        uint64_t value;
    } dims[] = {{"row_count", row_count},
                {"slot_count", slot_count},
                {"page_size", layout->page_size},
                {"page_stride_bytes", layout->page_stride_bytes},
                {"row_bytes", layout->row_bytes}};
    for (const auto &d : dims)
        if (d.value == 0)
            return fail(SGL_KV_ZERO_DIMENSION, d.dimension, 0, 0, 0,
                        "KV copy dimension %s must be non-zero", d.dimension);
    const struct {
        const char *tensor;
        uint64_t stride;
    } strides[] = {{"key", key_row_stride_bytes}, {"value", value_row_stride_bytes}};
    for (const auto &s : strides)
        if (s.stride < layout->row_bytes)
            return fail(SGL_KV_ROW_STRIDE_TOO_SMALL, s.tensor, layout->row_bytes, s.stride, 0,
                        "KV copy %s row stride %llu bytes is smaller than row width %llu bytes",
                        s.tensor, (unsigned long long)s.stride,
                        (unsigned long long)layout->row_bytes);
    auto overflow = [] {
        return fail(SGL_KV_SHAPE_OVERFLOW, nullptr, 0, 0, 0, "KV copy tensor shape overflowed");
    };
    uint64_t tensor_page_bytes;
    if (mul_ovf(layout->page_size, layout->row_bytes, &tensor_page_bytes)) return overflow();
    const struct {
        const char *tensor;
        uint64_t offset;
    } regions[] = {{"key", layout->key_in_page_offset}, {"value", layout->value_in_page_offset}};
    uint64_t ends[2];
    for (int i = 0; i < 2; ++i) {
        if (add_ovf(regions[i].offset, tensor_page_bytes, &ends[i])) return overflow();
        if (ends[i] > layout->page_stride_bytes) {
            uint64_t shown;
            if (add_ovf(regions[i].offset, tensor_page_bytes, &shown)) shown = UINT64_MAX;
            return fail(SGL_KV_TENSOR_PAGE_REGION_OUT_OF_BOUNDS, regions[i].tensor,
                        regions[i].offset, tensor_page_bytes, layout->page_stride_bytes,
                        "KV copy %s page region [%llu, %llu) exceeds page stride %llu",
                        regions[i].tensor, (unsigned long long)regions[i].offset,
                        (unsigned long long)shown, (unsigned long long)layout->page_stride_bytes);
        }
    }
    if (layout->key_in_page_offset < ends[1] && layout->value_in_page_offset < ends[0])
        return fail(SGL_KV_TENSOR_PAGE_REGIONS_OVERLAP, nullptr, layout->key_in_page_offset,
                    layout->value_in_page_offset, tensor_page_bytes,
                    "KV copy key/value page regions overlap: key offset %llu, value offset %llu, "
                    "tensor page size %llu bytes",
                    (unsigned long long)layout->key_in_page_offset,
                    (unsigned long long)layout->value_in_page_offset,
                    (unsigned long long)tensor_page_bytes);
    sgl_kv_pair_copy_plan p;
    memset(&p, 0, sizeof p);
    // strided_rows_required_bytes: (rows - 1) * stride + row_bytes.
    if (mul_ovf(row_count - 1, key_row_stride_bytes, &p.key_rows_required_bytes) ||
        add_ovf(p.key_rows_required_bytes, layout->row_bytes, &p.key_rows_required_bytes) ||
        mul_ovf(row_count - 1, value_row_stride_bytes, &p.value_rows_required_bytes) ||
        add_ovf(p.value_rows_required_bytes, layout->row_bytes, &p.value_rows_required_bytes) ||
        mul_ovf(row_count, 8, &p.slot_indices_required_bytes))
        return overflow();
    // The pool must reach the end of the last slot's later tensor row.
    const uint64_t last_slot = slot_count - 1;
    const uint64_t last_page = last_slot / layout->page_size;
    const uint64_t last_token = last_slot % layout->page_size;
    const uint64_t last_tensor_end = ends[0] > ends[1] ? ends[0] : ends[1];
    uint64_t page_off, token_off, tail;
    if (mul_ovf(last_page, layout->page_stride_bytes, &page_off) ||
        last_tensor_end < tensor_page_bytes ||
        mul_ovf(last_token, layout->row_bytes, &token_off) ||
        add_ovf(last_tensor_end - tensor_page_bytes, token_off, &tail) ||
        add_ovf(tail, layout->row_bytes, &tail) || add_ovf(page_off, tail, &p.pool_required_bytes))
        return overflow();
    // The reference sizes a byte-per-thread grid here (2 * rows * row_bytes
    // threads); this library's launch is sized per row, so only the overflow
    // check of that product is kept.
    uint64_t threads;
    if (mul_ovf(row_count, layout->row_bytes, &threads) || mul_ovf(threads, 2, &threads))
        return overflow();
    p.row_count = row_count;
    p.slot_count = slot_count;
    p.layout = *layout;
    p.key_row_stride_bytes = key_row_stride_bytes;
    p.value_row_stride_bytes = value_row_stride_bytes;
    *out = p;
    return ok();
}

// transfer_page_indices (crates/sglang-srt/src/transfer.rs:679-720).
extern "C" int32_t sgl_kv_transfer_page_indices(uint64_t request_index, uint64_t token_offset,
                                                const uint64_t *cache_slots, uint64_t slot_len,
                                                uint64_t page_size, uint64_t *out_pages,
                                                uint64_t *out_len) {
    if (!out_len) return fail(SGL_KV_INVALID_ARGUMENT, "out_len", 0, 0, 0, "null argument");
    *out_len = 0;
    if (slot_len == 0) return ok();
    if (page_size == 0)
        return fail(SGL_KV_PLAN_ZERO_PAGE_SIZE, nullptr, 0, 0, 0,
                    "KV transfer page size must be non-zero");
    if (!cache_slots || !out_pages)
        return fail(SGL_KV_INVALID_ARGUMENT, "cache_slots/out_pages", 0, 0, 0, "null argument");
    if (token_offset % page_size)
        return fail(SGL_KV_PLAN_UNALIGNED_TOKEN_OFFSET, nullptr, request_index, token_offset,
                    page_size, "KV transfer token offset %llu is not aligned to page size %llu",
                    (unsigned long long)token_offset, (unsigned long long)page_size);
    uint64_t n = 0;
    for (uint64_t first = 0; first < slot_len; first += page_size) {
        const uint64_t head = cache_slots[first];
        if (head % page_size)
            return fail(SGL_KV_PLAN_UNALIGNED_CACHE_SLOT, nullptr, request_index, head, page_size,
                        "KV transfer cache slot %llu is not aligned to page size %llu",
                        (unsigned long long)head, (unsigned long long)page_size);
        const uint64_t stop = slot_len - first < page_size ? slot_len : first + page_size;
        for (uint64_t i = first; i < stop; ++i)
            if (cache_slots[i] != head + (i - first))
                return fail(SGL_KV_PLAN_NON_CONTIGUOUS_CACHE_SLOTS, nullptr, request_index,
                            head + (i - first), cache_slots[i],
                            "KV transfer cache slots are not contiguous: expected %llu, got %llu",
                            (unsigned long long)(head + (i - first)),
                            (unsigned long long)cache_slots[i]);
        out_pages[n++] = head / page_size;
    }
    *out_len = n;
    return ok();
}

// paged_kv_cache_layout_for_model (crates/sglang-srt/src/backend_model.rs:348-382).
extern "C" int32_t sgl_kv_paged_layout_for_model(const sgl_kv_model_layout *model, int32_t dtype,
                                                 uint64_t page_size, uint64_t slot_capacity,
                                                 sgl_kv_paged_layout *out) {
    if (!model || !out) return fail(SGL_KV_INVALID_ARGUMENT, "model/out", 0, 0, 0, "null argument");
    // validate_cache_config (backend_model.rs:457-475)
    if (slot_capacity == 0)
        return fail(SGL_KV_MODEL_MISSING_CAPABILITY, "slot_capacity", 0, 0, 0,
                    "missing capabilities: non-zero KV cache slot capacity");
    if (page_size == 0)
        return fail(SGL_KV_MODEL_MISSING_CAPABILITY, "page_size", 0, 0, 0,
                    "missing capabilities: non-zero KV cache page size");
    if (slot_capacity % page_size)
        return fail(SGL_KV_MODEL_MISSING_CAPABILITY, "slot_capacity", slot_capacity, page_size, 0,
                    "missing capabilities: KV cache slot capacity %llu divisible by page size %llu",
                    (unsigned long long)slot_capacity, (unsigned long long)page_size);
    uint64_t bytes_per_token, pair[2];
    uint32_t is_pair;
    int32_t rc = sgl_kv_model_layout_token_size_bytes(model, dtype, &bytes_per_token);
    if (rc) return rc;
    if ((rc = sgl_kv_model_layout_tensor_pair_size_bytes(model, dtype, pair, &is_pair))) return rc;
    sgl_kv_runtime_layout rt;
    memset(&rt, 0, sizeof rt);
    if (mul_ovf(page_size, bytes_per_token, &rt.page_size_bytes))
        return fail(SGL_KV_MODEL_SIZE_OVERFLOW, nullptr, 0, 0, 0, "KV page size overflowed");
    rt.dtype = dtype;
    rt.page_size = page_size;
    rt.num_layers = model->num_layers;
    rt.kv_heads = model->kv_heads;
    rt.head_dim = model->head_dim;
    rt.kv_tensors_per_token = model->kv_tensors_per_token;
    rt.bytes_per_token = bytes_per_token;
    const uint64_t page_count = slot_capacity / page_size;
    if (is_pair) return sgl_kv_paged_layout_new_with_tensor_pair(&rt, page_count, pair[0], pair[1], out);
    return sgl_kv_paged_layout_new(&rt, page_count, out);
}

// View of one layer of a paged pool for the per-layer copies.
extern "C" int32_t sgl_kv_pool_view_for_layer(const sgl_kv_paged_layout *layout, void *base,
                                              uint64_t byte_len, uint32_t head_layout,
                                              uint64_t heads, uint64_t layer_index,
                                              uint64_t first_tensor, uint64_t tensor_count,
                                              sgl_kv_pool_view *out) {
    if (!layout || !out) return fail(SGL_KV_INVALID_ARGUMENT, "layout/out", 0, 0, 0, "null argument");
    const sgl_kv_runtime_layout &rt = layout->runtime;
    if (layer_index >= rt.num_layers)
        return fail(SGL_KV_LAYOUT_LAYER_OUT_OF_RANGE, nullptr, layer_index, rt.num_layers, 0,
                    "KV cache layer index %llu is outside %llu layers",
                    (unsigned long long)layer_index, (unsigned long long)rt.num_layers);
    if (tensor_count == 0 || tensor_count > 2)
        return fail(SGL_KV_INVALID_ARGUMENT, "tensor_count", tensor_count, 2, 0,
                    "a pool view holds one or two tensors, not %llu",
                    (unsigned long long)tensor_count);
    if (first_tensor + tensor_count > rt.kv_tensors_per_token)
        return tensor_out_of_range(layout, first_tensor + tensor_count - 1);
    if (head_layout > SGL_KV_HND)
        return fail(SGL_KV_INVALID_ARGUMENT, "head_layout", head_layout, 0, 0,
                    "unknown head layout %u", head_layout);
    uint64_t tb[2] = {0, 0}, to[2] = {0, 0}, layer_off;
    if (mul_ovf(layer_index, layout->bytes_per_layer_page, &layer_off)) return layout_overflow();
    for (uint64_t t = 0; t < tensor_count; ++t) {
        int32_t rc = tensor_geometry(layout, first_tensor + t, &tb[t], &to[t]);
        if (rc) return rc;
        if (add_ovf(to[t], layer_off, &to[t])) return layout_overflow();
    }
    for (uint64_t t = 0; t < tensor_count; ++t)
        if (heads == 0 || heads > UINT32_MAX || tb[t] % heads)
            return fail(SGL_KV_INVALID_ARGUMENT, "heads", heads, tb[t], 0,
                        "%llu heads do not split a %llu-byte row evenly", (unsigned long long)heads,
                        (unsigned long long)tb[t]);
    sgl_kv_pool_view v;
    memset(&v, 0, sizeof v);
    v.base = base;
    v.byte_len = byte_len;
    v.page_size = rt.page_size;
    v.page_stride_bytes = rt.page_size_bytes;
    v.page_count = layout->page_count;
    v.tensor_offset[0] = to[0];
    v.tensor_offset[1] = to[1];
    v.row_bytes = tb[0];
    v.value_row_bytes = tensor_count == 2 && tb[1] != tb[0] ? tb[1] : 0;
    v.tensor_count = (uint32_t)tensor_count;
    v.heads = (uint32_t)heads;
    v.head_layout = head_layout;
    *out = v;
    return ok();
}

// --- PD page-request descriptors (crates/sglang-srt/src/transfer.rs:1945-2090) ---

static int32_t span_pages_match(uint64_t token_count, uint64_t page_size, uint64_t page_count) {
    // token_count.div_ceil(page_size) == page_indices.len()
    const uint64_t expected = token_count / page_size + (token_count % page_size ? 1 : 0);
    if (expected != page_count)
        return fail(SGL_KV_REQ_SPAN_PAGE_COUNT_MISMATCH, nullptr, expected, page_count, 0,
                    "KV transfer span requires %llu physical pages but has %llu source page "
                    "indices",
                    (unsigned long long)expected, (unsigned long long)page_count);
    return SGL_KV_OK;
}

static int32_t address_overflow() {
    return fail(SGL_KV_REQ_ADDRESS_OVERFLOW, nullptr, 0, 0, 0, "Mooncake source address overflowed");
}

static int32_t offset_overflow() {
    return fail(SGL_KV_REQ_OFFSET_OVERFLOW, nullptr, 0, 0, 0, "Mooncake target offset overflowed");
}

extern "C" int32_t sgl_kv_build_page_requests(uint64_t source_base_addr, uint64_t page_size_bytes,
                                              uint64_t target_base_offset, uint64_t token_offset,
                                              uint64_t token_count, uint64_t page_size,
                                              const uint64_t *page_indices, uint64_t page_count,
                                              sgl_kv_page_request *out, uint64_t out_capacity,
                                              uint64_t *out_len) {
    if (!out_len) return fail(SGL_KV_INVALID_ARGUMENT, "out_len", 0, 0, 0, "null argument");
    *out_len = 0;
    if (page_size_bytes == 0)
        return fail(SGL_KV_REQ_ZERO_PAGE_SIZE, nullptr, 0, 0, 0, "Mooncake KV page size must be non-zero");
    if (page_size == 0)
        return fail(SGL_KV_PLAN_ZERO_PAGE_SIZE, nullptr, 0, 0, 0, "KV transfer page size must be non-zero");
    int32_t rc = span_pages_match(token_count, page_size, page_count);
    if (rc) return rc;
    if (page_count && (!page_indices || !out))
        return fail(SGL_KV_INVALID_ARGUMENT, "page_indices/out", 0, 0, 0, "null argument");
    if (out_capacity < page_count)
        return fail(SGL_KV_INVALID_ARGUMENT, "out_capacity", out_capacity, page_count, 0,
                    "%llu request slots for %llu pages", (unsigned long long)out_capacity,
                    (unsigned long long)page_count);
    const uint64_t page_offset = token_offset / page_size;  // KvCacheTransferSpan::page_offset
    for (uint64_t i = 0; i < page_count; ++i) {
        uint64_t src, tgt_page, tgt;
        if (mul_ovf(page_indices[i], page_size_bytes, &src) || add_ovf(source_base_addr, src, &src))
            return address_overflow();
        if (add_ovf(page_offset, i, &tgt_page) || mul_ovf(tgt_page, page_size_bytes, &tgt) ||
            add_ovf(target_base_offset, tgt, &tgt))
            return offset_overflow();
        out[i].source = src;
        out[i].target_offset = tgt;
        out[i].length = page_size_bytes;
    }
    *out_len = page_count;
    return ok();
}

extern "C" int32_t sgl_kv_build_remote_page_requests(
    uint64_t source_base_addr, uint64_t page_size_bytes, uint64_t token_count, uint64_t page_size,
    const uint64_t *page_indices, uint64_t page_count, const uint64_t *dst_kv_ptrs,
    uint64_t ptr_count, const int32_t *dst_kv_indices, uint64_t index_count,
    uint64_t dst_kv_item_len, sgl_kv_page_request *out, uint64_t out_capacity, uint64_t *out_len) {
    if (!out_len) return fail(SGL_KV_INVALID_ARGUMENT, "out_len", 0, 0, 0, "null argument");
    *out_len = 0;
    if (page_size_bytes == 0)
        return fail(SGL_KV_REQ_ZERO_PAGE_SIZE, nullptr, 0, 0, 0, "Mooncake KV page size must be non-zero");
    if (dst_kv_item_len == 0)
        return fail(SGL_KV_REQ_ZERO_REMOTE_ITEM_SIZE, nullptr, 0, 0, 0,
                    "Mooncake remote KV item size must be non-zero");
    if (ptr_count == 0)
        return fail(SGL_KV_REQ_MISSING_REMOTE_POINTERS, nullptr, 0, 0, 0,
                    "Mooncake remote KV pointers must not be empty");
    if (page_size == 0)
        return fail(SGL_KV_PLAN_ZERO_PAGE_SIZE, nullptr, 0, 0, 0, "KV transfer page size must be non-zero");
    int32_t rc = span_pages_match(token_count, page_size, page_count);
    if (rc) return rc;
    if (page_count != index_count)
        return fail(SGL_KV_REQ_REMOTE_INDEX_COUNT_MISMATCH, nullptr, page_count, index_count, 0,
                    "KV transfer span has %llu source pages but %llu remote KV indices",
                    (unsigned long long)page_count, (unsigned long long)index_count);
    uint64_t split;
    if (mul_ovf(dst_kv_item_len, ptr_count, &split)) return address_overflow();
    if (split != page_size_bytes)
        return fail(SGL_KV_REQ_REMOTE_ITEM_LAYOUT_MISMATCH, nullptr, page_size_bytes, split, 0,
                    "Mooncake remote KV item layout splits a %llu-byte page into %llu bytes",
                    (unsigned long long)page_size_bytes, (unsigned long long)split);
    if (page_count && (!page_indices || !dst_kv_indices || !dst_kv_ptrs || !out))
        return fail(SGL_KV_INVALID_ARGUMENT, "page_indices/dst_kv_indices/dst_kv_ptrs/out", 0, 0, 0,
                    "null argument");
    uint64_t need;
    if (mul_ovf(page_count, ptr_count, &need) || out_capacity < need)
        return fail(SGL_KV_INVALID_ARGUMENT, "out_capacity", out_capacity, need, 0,
                    "%llu request slots for %llu pages x %llu pointers",
                    (unsigned long long)out_capacity, (unsigned long long)page_count,
                    (unsigned long long)ptr_count);
    uint64_t n = 0;
    for (uint64_t i = 0; i < page_count; ++i) {
        const int32_t index = dst_kv_indices[i];
        if (index < 0)
            return fail(SGL_KV_REQ_NEGATIVE_REMOTE_INDEX, nullptr, (uint64_t)(int64_t)index, 0, 0,
                        "Mooncake remote KV index %d is negative", index);
        uint64_t page_addr;
        if (mul_ovf(page_indices[i], page_size_bytes, &page_addr) ||
            add_ovf(source_base_addr, page_addr, &page_addr))
            return address_overflow();
        for (uint64_t j = 0; j < ptr_count; ++j) {
            uint64_t src, tgt;
            if (mul_ovf(j, dst_kv_item_len, &src) || add_ovf(page_addr, src, &src))
                return address_overflow();
            if (mul_ovf((uint64_t)index, dst_kv_item_len, &tgt) || add_ovf(dst_kv_ptrs[j], tgt, &tgt))
                return offset_overflow();
            out[n].source = src;
            out[n].target_offset = tgt;
            out[n].length = dst_kv_item_len;
            ++n;
        }
    }
    *out_len = n;
    return ok();
}
