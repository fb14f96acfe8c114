/*
 * sgl_rocm_kv.h -- C ABI of the MI355X (gfx950) KV-cache transfer path.
 *
 * The library (libsgl_rocm_kv.so) is the ROCm backend of sglang-rs's KV
 * copy path. It has two groups of entry points:
 *
 *  1. Host mirror of the reference's KV layout arithmetic and copy plan
 *     (no GPU needed). The reference keeps these in Rust; they are exported
 *     here so that the C++ launcher, the Python binding and the tests share
 *     one implementation of the validation rules the kernels rely on.
 *  2. Kernel entry points. Kernels are hand-written HIP, compiled ahead of
 *     time into a gfx950 code object (sgl_rocm_kv_gfx950.co) and loaded with
 *     hipModuleLoad. The library links libamdhip64.so.7 but makes no HIP
 *     call before sgl_rocm_kv_init, so it loads (and group 1 works) on a
 *     host without a GPU.
 *
 * Conventions
 *  - Every function returns an sgl_kv_status. On failure, the calling
 *    thread's detail record (sgl_kv_last_error) holds the reference error
 *    variant's fields. No exception, panic or abort crosses the ABI.
 *  - All buffers are borrowed: the caller owns every device allocation and
 *    passes plain device pointers with their byte lengths. The context owns
 *    only the loaded module and a 4-byte device error flag.
 *  - Streams are explicit (hipStream_t passed as void*; NULL is the null
 *    stream). The pair scatter/gather drop-ins synchronise the stream and
 *    read the error flag like the reference; the per-layer transfer calls are
 *    asynchronous and report device-side errors through
 *    sgl_rocm_kv_check_errors.
 *  - One context per device. Calls on one context must not overlap in time
 *    from different host threads (the reference takes &mut self).
 */
#ifndef SGL_ROCM_KV_H
#define SGL_ROCM_KV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SGL_ROCM_KV_ABI_VERSION 1

/* ------------------------------------------------------------------------ */
/* Status codes                                                             */
/* ------------------------------------------------------------------------ */

/*
 * 1..12 mirror CudaKvPairCopyError (crates/sglang-kernel/src/cuda_kv_kernels.rs:304-338)
 * plus the allocation range check of CudaDeviceAllocation::device_ptr_at
 * (crates/sglang-kernel/src/cuda.rs:895-916). 20..36 mirror
 * PagedKvCacheLayoutError (crates/sglang-srt/src/kv_cache.rs:256-318). 40..45
 * mirror KvCacheTransferPlanError (crates/sglang-srt/src/transfer.rs:722-750).
 * 50.. are device-side conditions of the per-layer transfer kernels.
 */
typedef enum sgl_kv_status {
    SGL_KV_OK = 0,
    SGL_KV_ZERO_DIMENSION = 1,                  /* name = dimension */
    SGL_KV_SHAPE_OVERFLOW = 2,
    SGL_KV_DIMENSION_TOO_LARGE = 3,             /* name, a = value, b = maximum */
    SGL_KV_ROW_STRIDE_TOO_SMALL = 4,            /* name = tensor, a = row_bytes, b = row_stride_bytes */
    SGL_KV_TENSOR_PAGE_REGION_OUT_OF_BOUNDS = 5,/* name = tensor, a = offset, b = tensor_page_bytes, c = page_stride_bytes */
    SGL_KV_TENSOR_PAGE_REGIONS_OVERLAP = 6,     /* a = key_offset, b = value_offset, c = tensor_page_bytes */
    SGL_KV_DEVICE_MISMATCH = 7,                 /* name = allocation, a = expected, b = actual ordinal */
    SGL_KV_DEVICE_SLOT_INDEX_OUT_OF_RANGE = 8,  /* a = slot_count */
    SGL_KV_HIP = 9,                             /* a = hipError_t, name = HIP call */
    SGL_KV_MODULE = 10,                         /* code object / libamdhip64 could not be loaded or resolved */
    SGL_KV_ALLOCATION_OUT_OF_BOUNDS = 11,       /* name = buffer, a = offset, b = byte_len, c = allocation_byte_len */
    SGL_KV_INVALID_ARGUMENT = 12,               /* name = argument */

    SGL_KV_LAYOUT_ZERO_PAGE_COUNT = 20,
    SGL_KV_LAYOUT_ZERO_FIELD = 21,              /* name = field */
    SGL_KV_LAYOUT_RUNTIME_PAGE_SIZE_MISMATCH = 22, /* a = expected, b = actual */
    SGL_KV_LAYOUT_UNEVEN_LAYER = 23,            /* a = bytes_per_token, b = num_layers */
    SGL_KV_LAYOUT_UNEVEN_TENSOR = 24,           /* a = bytes_per_token_per_layer, b = kv_tensors_per_token */
    SGL_KV_LAYOUT_SIZE_OVERFLOW = 25,
    SGL_KV_LAYOUT_PAGE_OUT_OF_RANGE = 26,       /* a = page_index, b = page_count */
    SGL_KV_LAYOUT_LAYER_OUT_OF_RANGE = 27,      /* a = layer_index, b = layer_count */
    SGL_KV_LAYOUT_TENSOR_OUT_OF_RANGE = 28,     /* a = tensor_index, b = tensor_count */
    SGL_KV_LAYOUT_TOKEN_OUT_OF_RANGE = 29,      /* a = token_index, b = page_size */
    SGL_KV_LAYOUT_SLOT_OUT_OF_RANGE = 30,       /* a = slot_index, b = slot_count */
    SGL_KV_LAYOUT_EMPTY_SLOT_MAP = 31,
    SGL_KV_LAYOUT_BATCH_SLOT_OUT_OF_RANGE = 32, /* a = batch_index, b = slot_index, c = slot_count */
    SGL_KV_LAYOUT_KV_PAIR_REQUIRES_TWO_TENSORS = 33,     /* a = tensor_count */
    SGL_KV_LAYOUT_TENSOR_PAIR_REQUIRES_TWO_TENSORS = 34, /* a = tensor_count */
    SGL_KV_LAYOUT_TENSOR_PAIR_SIZE_MISMATCH = 35, /* a = bytes_per_token_per_layer, b = key, c = value token bytes */
    SGL_KV_LAYOUT_UNEVEN_KV_PAIR_COPY = 36,     /* a = key_token_bytes, b = value_token_bytes */

    SGL_KV_PLAN_ZERO_PAGE_SIZE = 40,
    SGL_KV_PLAN_CACHE_PAGE_COUNT_MISMATCH = 41, /* a = request index, b = input_token_count, c = cache_page_count */
    SGL_KV_PLAN_TRAILING_CACHE_PAGES = 42,      /* a = consumed, b = cache_page_count */
    SGL_KV_PLAN_UNALIGNED_TOKEN_OFFSET = 43,    /* a = request index, b = token_offset, c = page_size */
    SGL_KV_PLAN_UNALIGNED_CACHE_SLOT = 44,      /* a = request index, b = cache_slot, c = page_size */
    SGL_KV_PLAN_NON_CONTIGUOUS_CACHE_SLOTS = 45,/* a = request index, b = expected, c = actual */
    SGL_KV_PLAN_NON_PREFILL_BATCH = 46,

    SGL_KV_DEVICE_PAGE_INDEX_OUT_OF_RANGE = 50, /* a page-table entry is negative, past the table or past the pool */
    SGL_KV_DEVICE_SPAN_OUT_OF_RANGE = 51,       /* a row is not covered by its span list */
    SGL_KV_DEVICE_REQUEST_OUT_OF_RANGE = 52,    /* a page request outside its source or target region */

    /* 60.. mirror MooncakeRequestBuildError (crates/sglang-srt/src/transfer.rs:2092-2112) */
    SGL_KV_REQ_ZERO_PAGE_SIZE = 60,
    SGL_KV_REQ_ZERO_REMOTE_ITEM_SIZE = 61,
    SGL_KV_REQ_MISSING_REMOTE_POINTERS = 62,
    SGL_KV_REQ_SPAN_PAGE_COUNT_MISMATCH = 63,   /* a = expected_page_count, b = source_page_index_count */
    SGL_KV_REQ_REMOTE_INDEX_COUNT_MISMATCH = 64,/* a = source_page_count, b = dst_kv_index_count */
    SGL_KV_REQ_REMOTE_ITEM_LAYOUT_MISMATCH = 65,/* a = page_size_bytes, b = split_page_size */
    SGL_KV_REQ_NEGATIVE_REMOTE_INDEX = 66,      /* a = the index (as int64) */
    SGL_KV_REQ_ADDRESS_OVERFLOW = 67,
    SGL_KV_REQ_OFFSET_OVERFLOW = 68,

    /* 70.. mirror CacheAllocationError (crates/sglang-srt/src/cache.rs:63-74) */
    SGL_KV_ALLOC_ZERO_PAGE_SIZE = 70,
    SGL_KV_ALLOC_ZERO_SLOT_CAPACITY = 71,
    SGL_KV_ALLOC_SLOT_CAPACITY_NOT_PAGE_ALIGNED = 72, /* a = slot_capacity, b = page_size */
    SGL_KV_ALLOC_OUT_OF_SLOTS = 73,                   /* a = requested, b = available */
    /* RadixCacheError (cache.rs:38-44) */
    SGL_KV_RADIX_TOKEN_PAGE_LENGTH_MISMATCH = 74,     /* a = token_count, b = cache_page_count */

    /* 80.. mirror CudaBf16PagedAttentionError (crates/sglang-kernel/src/cuda_attention.rs:518-564)
     * and CudaPagedAttentionError's plan variants (crates/sglang-srt/src/cuda_attention.rs:15-75);
     * ZeroDimension, ShapeOverflow, DimensionTooLarge, TensorPageRegionOutOfBounds and
     * DeviceMismatch reuse codes 1, 2, 3, 5 and 7. */
    SGL_KV_ATTN_INVALID_SCALE = 80,                   /* a = the scale's f32 bits */
    SGL_KV_ATTN_QUERY_HEADS_NOT_DIVISIBLE = 81,       /* a = query_head_count, b = kv_head_count */
    SGL_KV_ATTN_KEY_ROW_BYTES_MISMATCH = 82,          /* a = expected, b = actual */
    SGL_KV_ATTN_VALUE_ROW_BYTES_MISMATCH = 83,        /* a = expected, b = actual */
    SGL_KV_ATTN_TENSOR_PAGE_REGIONS_OVERLAP = 84,     /* a = key_offset, b = value_offset, c = key_page_bytes, d = value_page_bytes */
    SGL_KV_ATTN_DEVICE_METADATA_INVALID = 85,         /* a = flags: request 0x1, sequence 0x2, slot 0x4 */
    SGL_KV_ATTN_UNSUPPORTED_KV_DTYPE = 86,            /* a = actual dtype, b = required */
    SGL_KV_ATTN_TENSOR_ROW_GEOMETRY_MISMATCH = 87,    /* name = tensor, a = row_bytes, b = kv_head_count, c = element_bytes */

    /* 90.. mirror MooncakeBootstrapFrameError (crates/sglang-srt/src/pd_bootstrap.rs:576-600),
     * MooncakeRemoteKvLayoutError (:504-510) and MooncakeDecodeBootstrapError::MissingAuxIndex
     * (:920); 99 is the decode-layout extension of this build. */
    SGL_KV_BOOT_MISSING_FIELD = 90,             /* name = frame, a = expected, b = actual */
    SGL_KV_BOOT_UTF8_FIELD = 91,                /* name = field */
    SGL_KV_BOOT_INTEGER_FIELD = 92,             /* name = field; the value is quoted in the message */
    SGL_KV_BOOT_BINARY_LENGTH = 93,             /* name = field, a = width, b = actual */
    SGL_KV_BOOT_PACKED_LIST_HEADER = 94,        /* name = field */
    SGL_KV_BOOT_PACKED_LIST_LENGTH = 95,        /* name = field */
    SGL_KV_BOOT_MISSING_TRANSFER_ROOM = 96,     /* a = room */
    SGL_KV_BOOT_MISSING_KV_ARGS = 97,           /* a = room; the session id is quoted in the message */
    SGL_KV_BOOT_MISSING_AUX_INDEX = 98,         /* the session id is quoted in the message */
    SGL_KV_BOOT_DECODE_LAYOUT = 99,             /* name = what is wrong, a, b = values */

    /* 100.. mirror KvCacheLayoutError (crates/sglang-srt/src/kv_cache.rs:227-251) and the
     * MissingCapabilities of validate_cache_config (crates/sglang-srt/src/backend_model.rs:457-475) */
    SGL_KV_MODEL_DTYPE_REQUIRES_MODEL_METADATA = 100, /* a = dtype */
    SGL_KV_MODEL_INVALID_PACKED_MLA_NOPE_HEAD_DIM = 101, /* a = qk_nope_head_dim */
    SGL_KV_MODEL_ZERO_TENSOR_WIDTH = 102,
    SGL_KV_MODEL_SIZE_OVERFLOW = 103,
    SGL_KV_MODEL_MISSING_CAPABILITY = 104,      /* the message names the capability; a, b = values */

    /* 110.. mirror CudaKvStorageError (crates/sglang-srt/src/cuda_kv_cache.rs:20-40),
     * KvCachePoolError (crates/sglang-srt/src/kv_cache.rs:830-833), CudaError::ZeroAllocation
     * (crates/sglang-kernel/src/cuda.rs:121, 477-480) and MooncakeError::UnsupportedMemoryLocation
     * (crates/sglang-srt/src/transfer.rs:1662-1676). Layout errors of the storage calls keep
     * their codes 20..36, device copies 7, 9 and 11. */
    SGL_KV_STORAGE_SIZE_MISMATCH = 110,         /* name = "storage" or "pool", a = expected, b = actual bytes */
    SGL_KV_STORAGE_SLOT_MAP_CAPACITY_MISMATCH = 111, /* a = map_slot_count, b = layout_slot_count */
    SGL_KV_STORAGE_PAGE_BUFFER_SIZE_MISMATCH = 112,  /* a = expected, b = actual bytes */
    SGL_KV_STORAGE_SIZE_OVERFLOW = 113,
    SGL_KV_ZERO_ALLOCATION = 114,
    SGL_KV_UNSUPPORTED_MEMORY_LOCATION = 115,   /* a = sgl_kv_memory_location_kind, b = id */
    SGL_KV_STORAGE_DESCRIPTOR = 116             /* name = what is wrong, a, b = values */
} sgl_kv_status;

/* Detail of the calling thread's most recent failure. */
typedef struct sgl_kv_error_detail {
    int32_t code;          /* sgl_kv_status */
    int32_t reserved;
    uint64_t a, b, c, d;   /* variant fields, in the order listed above */
    char name[64];         /* dimension / tensor / field / allocation / call name */
    char message[320];     /* human-readable text, as the reference's Display impl */
} sgl_kv_error_detail;

void sgl_kv_last_error(sgl_kv_error_detail *out);
const char *sgl_kv_status_name(int32_t code);

/* ------------------------------------------------------------------------ */
/* Group 1: layout and plan (host only)                                      */
/* ------------------------------------------------------------------------ */

/* KvCacheDtype (crates/sglang-srt/src/kv_cache.rs:7-14). */
typedef enum sgl_kv_dtype {
    SGL_KV_DTYPE_AUTO = 0,
    SGL_KV_DTYPE_FLOAT32 = 1,
    SGL_KV_DTYPE_BFLOAT16 = 2,
    SGL_KV_DTYPE_FP8_E4M3 = 3,
    SGL_KV_DTYPE_FP8_E5M2 = 4,
    SGL_KV_DTYPE_FP4_E2M1 = 5
} sgl_kv_dtype;

/* KvCacheDtype::bytes_per_element (kv_cache.rs:39-46): 0 when the width
 * needs model metadata (fp4). */
size_t sgl_kv_dtype_bytes_per_element(int32_t dtype);

/* KvCacheRuntimeLayout (kv_cache.rs:57-66). */
typedef struct sgl_kv_runtime_layout {
    int32_t dtype;
    int32_t reserved;
    uint64_t page_size;
    uint64_t num_layers;
    uint64_t kv_heads;
    uint64_t head_dim;
    uint64_t kv_tensors_per_token;
    uint64_t bytes_per_token;
    uint64_t page_size_bytes;
} sgl_kv_runtime_layout;

/* KvCacheModelLayout (kv_cache.rs:68-225): a model's KV geometry before the
 * dtype and page size are chosen. Built by the constructors below. */
typedef enum sgl_kv_tensor_geometry {
    SGL_KV_GEOMETRY_UNIFORM = 0,      /* multi_tensor: every tensor kv_heads * head_dim elements */
    SGL_KV_GEOMETRY_PAIR = 1,         /* tensor_pair: key and value widths of their own */
    SGL_KV_GEOMETRY_PACKED_BYTES = 2  /* packed_bytes_per_layer / packed_mla: a byte row */
} sgl_kv_tensor_geometry;

typedef struct sgl_kv_model_layout {
    uint64_t num_layers;
    uint64_t kv_heads;
    uint64_t head_dim;
    uint64_t kv_tensors_per_token;
    uint64_t bytes_per_token_per_layer; /* PACKED_BYTES: the packed row (Some); 0 = None */
    uint32_t geometry;                  /* sgl_kv_tensor_geometry */
    uint32_t reserved;
    uint64_t key_elements;              /* PAIR only */
    uint64_t value_elements;            /* PAIR only */
} sgl_kv_model_layout;

/* KvCacheModelLayout::multi_tensor (kv_cache.rs:89-103); infallible. */
int32_t sgl_kv_model_layout_multi_tensor(uint64_t num_layers, uint64_t kv_heads, uint64_t head_dim,
                                         uint64_t kv_tensors_per_token, sgl_kv_model_layout *out);
/* KvCacheModelLayout::tensor_pair (kv_cache.rs:105-132): SizeOverflow,
 * ZeroTensorWidth. DeepSeek-V3 builds tensor_pair(L, 1, kv_lora_rank +
 * qk_rope_head_dim, 1, kv_lora_rank) (models/deepseek.rs:360-369). */
int32_t sgl_kv_model_layout_tensor_pair(uint64_t num_layers, uint64_t key_heads, uint64_t key_head_dim,
                                        uint64_t value_heads, uint64_t value_head_dim,
                                        sgl_kv_model_layout *out);
/* KvCacheModelLayout::packed_bytes_per_layer (kv_cache.rs:134-143); infallible. */
int32_t sgl_kv_model_layout_packed_bytes_per_layer(uint64_t num_layers, uint64_t bytes_per_token_per_layer,
                                                   sgl_kv_model_layout *out);
/* KvCacheModelLayout::packed_mla (kv_cache.rs:201-224): nope + 2 rope +
 * nope / 64 + 1 bytes per token per layer (649 for DeepSeek's 512/64,
 * models/deepseek.rs:1035-1037). InvalidPackedMlaNopeHeadDim unless nope %
 * 64 == 0; SizeOverflow. */
int32_t sgl_kv_model_layout_packed_mla(uint64_t num_layers, uint64_t qk_nope_head_dim,
                                       uint64_t qk_rope_head_dim, sgl_kv_model_layout *out);
/* elements_per_token (kv_cache.rs:146-158): *has = 0 (None) for packed
 * layouts and on overflow. */
int32_t sgl_kv_model_layout_elements_per_token(const sgl_kv_model_layout *layout, uint64_t *out,
                                               uint32_t *has);
/* token_size_bytes (kv_cache.rs:160-176): DtypeRequiresModelMetadata (fp4
 * of a non-packed layout), SizeOverflow. */
int32_t sgl_kv_model_layout_token_size_bytes(const sgl_kv_model_layout *layout, int32_t dtype,
                                             uint64_t *out);
/* tensor_pair_size_bytes (kv_cache.rs:178-199): *is_pair = 0 (None) unless a
 * tensor pair; then out[0], out[1] = key and value bytes per token per layer. */
int32_t sgl_kv_model_layout_tensor_pair_size_bytes(const sgl_kv_model_layout *layout, int32_t dtype,
                                                   uint64_t out[2], uint32_t *is_pair);

/* PagedKvCacheLayout (kv_cache.rs:437-445): page -> layer -> tensor -> token. */
typedef struct sgl_kv_paged_layout {
    sgl_kv_runtime_layout runtime;
    uint64_t page_count;
    uint64_t bytes_per_token_per_layer;
    uint64_t bytes_per_layer_page;
    uint64_t tensor_pair;          /* 0 = Uniform geometry, 1 = explicit Pair */
    uint64_t token_bytes[2];       /* per-tensor token width; Uniform: both = token_bytes */
    uint64_t tensor_page_bytes;    /* Uniform: page_bytes; Pair: key_page_bytes */
    uint64_t total_byte_len;
    uint64_t slot_count;
} sgl_kv_paged_layout;

/* PagedKvCacheLayout::new (kv_cache.rs:448-478). */
int32_t sgl_kv_paged_layout_new(const sgl_kv_runtime_layout *runtime, uint64_t page_count,
                                sgl_kv_paged_layout *out);
/* PagedKvCacheLayout::new_with_tensor_pair (kv_cache.rs:480-529). */
int32_t sgl_kv_paged_layout_new_with_tensor_pair(const sgl_kv_runtime_layout *runtime,
                                                 uint64_t page_count, uint64_t key_token_bytes,
                                                 uint64_t value_token_bytes,
                                                 sgl_kv_paged_layout *out);
/* paged_kv_cache_layout_for_model (crates/sglang-srt/src/backend_model.rs:348-382):
 * the runtime layout and pool a model gets for `dtype` at `page_size` with
 * `slot_capacity` slots (slot_capacity / page_size pages): validate_cache_config
 * (MissingCapability: zero capacity, zero page size, capacity not a multiple
 * of the page size), token_size_bytes, then new_with_tensor_pair for a pair
 * geometry and new otherwise. */
int32_t sgl_kv_paged_layout_for_model(const sgl_kv_model_layout *model, int32_t dtype, uint64_t page_size,
                                      uint64_t slot_capacity, sgl_kv_paged_layout *out);
/* PagedKvCacheLayout::page_byte_range (kv_cache.rs:639-651); [start, end). */
int32_t sgl_kv_paged_layout_page_byte_range(const sgl_kv_paged_layout *layout, uint64_t page_index,
                                            uint64_t *start, uint64_t *end);
/* PagedKvCacheLayout::tensor_token_byte_range (kv_cache.rs:653-700). */
int32_t sgl_kv_paged_layout_tensor_token_byte_range(const sgl_kv_paged_layout *layout,
                                                    uint64_t page_index, uint64_t layer_index,
                                                    uint64_t tensor_index, uint64_t token_index,
                                                    uint64_t *start, uint64_t *end);
/* PagedKvCacheLayout::tensor_slot_byte_range (kv_cache.rs:702-720). */
int32_t sgl_kv_paged_layout_tensor_slot_byte_range(const sgl_kv_paged_layout *layout,
                                                   uint64_t layer_index, uint64_t tensor_index,
                                                   uint64_t slot_index, uint64_t *start,
                                                   uint64_t *end);
/* PagedKvCacheLayout::validate_slot_indices (kv_cache.rs:722-736); host slots. */
int32_t sgl_kv_paged_layout_validate_slot_indices(const sgl_kv_paged_layout *layout,
                                                  const uint64_t *slots, uint64_t slot_len);

/* CudaKvPairCopyLayout (crates/sglang-kernel/src/cuda_kv_kernels.rs:106-128). */
typedef struct sgl_kv_pair_copy_layout {
    uint64_t page_size;
    uint64_t page_stride_bytes;
    uint64_t key_in_page_offset;
    uint64_t value_in_page_offset;
    uint64_t row_bytes;
} sgl_kv_pair_copy_layout;

/* PagedKvCacheLayout::kv_pair_copy_geometry (kv_cache.rs:738-777), returned
 * directly as the copy layout it feeds (cuda_kv_cache.rs:510-532). */
int32_t sgl_kv_paged_layout_kv_pair_copy_geometry(const sgl_kv_paged_layout *layout,
                                                  uint64_t layer_index,
                                                  sgl_kv_pair_copy_layout *out);

/* CudaKvPairCopyPlan (cuda_kv_kernels.rs:153-164). grid_x / rows_per_tile
 * describe this library's launch, not the reference's byte-per-thread grid. */
typedef struct sgl_kv_pair_copy_plan {
    uint64_t row_count;
    uint64_t slot_count;
    sgl_kv_pair_copy_layout layout;
    uint64_t key_row_stride_bytes;
    uint64_t value_row_stride_bytes;
    uint64_t key_rows_required_bytes;
    uint64_t value_rows_required_bytes;
    uint64_t slot_indices_required_bytes;
    uint64_t pool_required_bytes;
} sgl_kv_pair_copy_plan;

/* CudaKvPairCopyPlan::new (cuda_kv_kernels.rs:167-264): same validation
 * order, same errors, same required-byte arithmetic. */
int32_t sgl_kv_pair_copy_plan_new(uint64_t row_count, uint64_t slot_count,
                                  const sgl_kv_pair_copy_layout *layout,
                                  uint64_t key_row_stride_bytes, uint64_t value_row_stride_bytes,
                                  sgl_kv_pair_copy_plan *out);

/* transfer_page_indices (crates/sglang-srt/src/transfer.rs:679-720): splits
 * one request's cache slots into pages. `out_pages` needs
 * ceil(slot_len / page_size) entries; *out_len receives the count.
 * `request_index` is echoed in error details (the reference carries the
 * request id). */
int32_t sgl_kv_transfer_page_indices(uint64_t request_index, uint64_t token_offset,
                                     const uint64_t *cache_slots, uint64_t slot_len,
                                     uint64_t page_size, uint64_t *out_pages, uint64_t *out_len);

/* One page write of a PD transfer (MooncakeTransferRequest without the
 * transport fields, transfer.rs:1945-2090): `length` bytes from host-visible
 * address `source` to `target_offset` in the target's registered memory. */
typedef struct sgl_kv_page_request {
    uint64_t source;
    uint64_t target_offset;
    uint64_t length;
} sgl_kv_page_request;

/* build_mooncake_kv_transfer_requests (transfer.rs:1945-1997): one request per
 * source page of a span; target page = span page offset (token_offset /
 * page_size) + i. `out` needs page_count entries. */
int32_t sgl_kv_build_page_requests(uint64_t source_base_addr, uint64_t page_size_bytes,
                                   uint64_t target_base_offset, uint64_t token_offset,
                                   uint64_t token_count, uint64_t page_size,
                                   const uint64_t *page_indices, uint64_t page_count,
                                   sgl_kv_page_request *out, uint64_t out_capacity,
                                   uint64_t *out_len);
/* build_mooncake_remote_kv_transfer_requests (transfer.rs:1999-2090): the
 * decode side advertises dst_kv_ptrs (one per split of a page) and one
 * dst_kv_indices entry per page; each source page becomes ptr_count
 * requests of dst_kv_item_len bytes. `out` needs page_count * ptr_count
 * entries. */
int32_t sgl_kv_build_remote_page_requests(uint64_t source_base_addr, uint64_t page_size_bytes,
                                          uint64_t token_count, uint64_t page_size,
                                          const uint64_t *page_indices, uint64_t page_count,
                                          const uint64_t *dst_kv_ptrs, uint64_t ptr_count,
                                          const int32_t *dst_kv_indices, uint64_t index_count,
                                          uint64_t dst_kv_item_len, sgl_kv_page_request *out,
                                          uint64_t out_capacity, uint64_t *out_len);

/* KV page allocator (CachePageAllocator, crates/sglang-srt/src/cache.rs:
 * 340-473): the producer of the slot indices every copy call takes. Pages
 * are handed out from the front of a free list; released pages return to
 * its front in release order. Not thread-safe (the reference takes &mut). */
typedef struct sgl_kv_page_allocator sgl_kv_page_allocator;
/* CachePageAllocator::with_page_size (cache.rs:353-376). */
int32_t sgl_kv_page_allocator_new(uint64_t slot_capacity, uint64_t page_size,
                                  sgl_kv_page_allocator **out);
int32_t sgl_kv_page_allocator_destroy(sgl_kv_page_allocator *allocator);
uint64_t sgl_kv_page_allocator_available_pages(const sgl_kv_page_allocator *allocator);
uint64_t sgl_kv_page_allocator_available_slots(const sgl_kv_page_allocator *allocator);
/* CachePageAllocator::allocate_for_sequence (cache.rs:397-447): writes
 * slot_count slots to out_slots, first the free tail of the sequence's last
 * page, then whole new pages. OutOfSlots leaves the allocator unchanged.
 * sequence_len 0 is CachePageAllocator::allocate. */
int32_t sgl_kv_page_allocator_allocate_for_sequence(sgl_kv_page_allocator *allocator,
                                                    const uint64_t *sequence_slots,
                                                    uint64_t sequence_len, uint64_t slot_count,
                                                    uint64_t *out_slots);
/* CachePageAllocator::release (cache.rs:449-466). */
int32_t sgl_kv_page_allocator_release(sgl_kv_page_allocator *allocator, const uint64_t *cache_pages,
                                      uint64_t count);
/* CachePageAllocator::reset (cache.rs:468-471). */
int32_t sgl_kv_page_allocator_reset(sgl_kv_page_allocator *allocator);

/* Token-prefix cache (RadixCache, crates/sglang-srt/src/cache.rs:475-547):
 * a trie over token ids whose nodes remember the KV slot ("cache page") of
 * their token. The scheduler matches a prompt against it before it
 * allocates, and the matched token count becomes the transfer span's
 * token_offset (only the uncached suffix moves). Not thread-safe (the
 * reference takes &mut). */
typedef struct sgl_kv_radix_cache sgl_kv_radix_cache;
int32_t sgl_kv_radix_cache_new(sgl_kv_radix_cache **out);
int32_t sgl_kv_radix_cache_destroy(sgl_kv_radix_cache *cache);
/* RadixCache::clear (cache.rs:481-483). */
int32_t sgl_kv_radix_cache_clear(sgl_kv_radix_cache *cache);
/* RadixCache::insert (cache.rs:485-504): every node on the path of
 * input_ids takes the matching cache page (an existing node's page is
 * replaced). TokenPageLengthMismatch when the lengths differ. */
int32_t sgl_kv_radix_cache_insert(sgl_kv_radix_cache *cache, const uint32_t *input_ids, uint64_t token_count,
                                  const uint64_t *cache_pages, uint64_t cache_page_count);
/* RadixCache::match_prefix (cache.rs:506-530), and with page_size > 0 its
 * page-aligned form match_prefix_page_aligned (:532-540): the match rounded
 * down to whole pages (page_size 0 is InvalidArgument; the reference
 * asserts). *matched_token_count receives the matched length m; the first m
 * entries of out_cache_pages (capacity token_count) its cache pages. The
 * remaining input ids are input_ids[m..]. page_size 1 is the plain match. */
int32_t sgl_kv_radix_cache_match_prefix(const sgl_kv_radix_cache *cache, const uint32_t *input_ids,
                                        uint64_t token_count, uint64_t page_size, uint64_t *matched_token_count,
                                        uint64_t *out_cache_pages);

/* The transfer-plan fields of a prefill ModelWorkerBatch
 * (crates/sglang-srt/src/model_executor.rs:15-198): per request, in batch
 * order, the tokens this forward computes (input_token_counts, the
 * uncached suffix), the tokens already cached (cached_token_counts, the
 * forward prefix) and whether it carries disaggregated params (a PD
 * request; the others have no span); out_cache_pages are the forward's
 * cache slots, the requests' runs concatenated. */
typedef enum sgl_kv_forward_mode { SGL_KV_FORWARD_PREFILL = 0, SGL_KV_FORWARD_DECODE = 1 } sgl_kv_forward_mode;
typedef struct sgl_kv_prefill_batch {
    int32_t forward_mode;                     /* sgl_kv_forward_mode */
    uint64_t request_count;
    const uint64_t *input_token_counts;       /* request_count entries */
    const uint64_t *cached_token_counts;      /* request_count entries */
    const uint8_t *has_disaggregated_params;  /* request_count entries, 0 or 1 */
    const uint64_t *out_cache_pages;
    uint64_t out_cache_page_count;
} sgl_kv_prefill_batch;

/* One KvCacheTransferSpan (transfer.rs:495-505) as offsets into the batch
 * and the plan's page-index array. */
typedef struct sgl_kv_plan_span {
    uint64_t request_index;      /* the request's position in the batch */
    uint64_t token_offset;       /* cached_token_counts[request_index] */
    uint64_t token_count;        /* input_token_counts[request_index] */
    uint64_t cache_page_offset;  /* its slots: out_cache_pages[cache_page_offset .. + token_count) */
    uint64_t page_index_offset;  /* its pages: page_indices[page_index_offset .. + page_index_count) */
    uint64_t page_index_count;
} sgl_kv_plan_span;

/* KvCacheTransferPlan::from_prefill_worker_batch_with_page_size
 * (transfer.rs:604-668): one span per request with disaggregated params,
 * errors in the reference's order (NonPrefillBatch, ZeroPageSize, then per
 * request CachePageCountMismatch and the transfer_page_indices errors, then
 * TrailingCachePages). `spans` needs one entry per PD request (request_count
 * is always enough); `page_indices` one per page of their slots
 * (out_cache_page_count / page_size + request_count is always enough);
 * too little room is InvalidArgument, checked after the plan's own errors.
 * On success *span_count and *page_index_count receive the counts. */
int32_t sgl_kv_transfer_plan_from_prefill_batch(const sgl_kv_prefill_batch *batch, uint64_t page_size,
                                                sgl_kv_plan_span *spans, uint64_t span_capacity,
                                                uint64_t *page_indices, uint64_t page_index_capacity,
                                                uint64_t *span_count, uint64_t *page_index_count);

/* KvCacheTransferSpan::descriptor_checksum (transfer.rs:548-570): lowercase
 * hex SHA-256 of the span's identifying fields, as /poll_transfers reports
 * it. Strings are (pointer, length) byte strings. */
int32_t sgl_kv_transfer_span_checksum(const char *request_id, uint64_t request_id_len,
                                      const char *bootstrap_host, uint64_t bootstrap_host_len,
                                      uint16_t bootstrap_port, uint64_t bootstrap_room,
                                      int32_t data_parallel_rank, uint64_t token_offset,
                                      uint64_t token_count, uint64_t page_size,
                                      const uint64_t *cache_pages, uint64_t cache_page_count,
                                      const uint64_t *page_indices, uint64_t page_index_count,
                                      char out_hex[65]);
/* SHA-256 (FIPS 180-4) of `len` bytes as lowercase hex; the checksum's hash. */
int32_t sgl_kv_sha256_hex(const void *data, uint64_t len, char out_hex[65]);

/* ------------------------------------------------------------------------ */
/* Group 2: kernels                                                         */
/* ------------------------------------------------------------------------ */

typedef struct sgl_rocm_kv_ctx sgl_rocm_kv_ctx;

/* Replaces CudaKvPairCopyKernels::compile (cuda_kv_kernels.rs:447-469):
 * no runtime compilation; loads the prebuilt gfx950 code object from
 * `code_object_path` (NULL: sgl_rocm_kv_gfx950.co beside the library) on
 * `device`, resolves every kernel and allocates + zeroes the error flag.
 * The library holds no per-process HIP state outside its contexts. Every
 * call on a context makes its device current for the call's duration and
 * restores the caller's device afterwards. */
int32_t sgl_rocm_kv_init(int32_t device, const char *code_object_path, sgl_rocm_kv_ctx **out);
/* Replaces the Drop of CudaKvPairCopyKernels / CudaModule (cuda.rs:693-708,
 * 933-939): unloads the module and frees the flag. NULL is accepted. */
int32_t sgl_rocm_kv_destroy(sgl_rocm_kv_ctx *ctx);
/* CudaContext::device_ordinal for the context. */
int32_t sgl_rocm_kv_device(const sgl_rocm_kv_ctx *ctx);
/* Number of compute units of the context's device (launch sizing, tests). */
int32_t sgl_rocm_kv_cu_count(const sgl_rocm_kv_ctx *ctx);

/* CudaDeviceAllocation's (device_ptr, byte_len) pair (cuda.rs:611-620). */
typedef struct sgl_kv_device_buffer {
    void *ptr;
    uint64_t byte_len;
} sgl_kv_device_buffer;

/* CudaKvPairScatter / CudaKvPairGather (cuda_kv_kernels.rs:424-444). */
typedef struct sgl_kv_pair_copy_buffers {
    sgl_kv_device_buffer keys;
    uint64_t keys_offset;
    sgl_kv_device_buffer values;
    uint64_t values_offset;
    sgl_kv_device_buffer slot_indices; /* u64 physical slots, one per row */
    uint64_t slot_indices_offset;
    sgl_kv_device_buffer pool;
    uint64_t pool_offset;
} sgl_kv_pair_copy_buffers;

/* CudaKvPairCopyKernels::scatter (cuda_kv_kernels.rs:471-504, launch
 * :541-623): strided K/V rows -> pool slots. Checks each buffer's device and
 * range, clears the flag, launches on `stream`, synchronises `stream` and
 * returns SGL_KV_DEVICE_SLOT_INDEX_OUT_OF_RANGE when any slot was >=
 * slot_count (those rows are skipped, as in the reference). */
int32_t sgl_rocm_kv_pair_scatter(sgl_rocm_kv_ctx *ctx, const sgl_kv_pair_copy_plan *plan,
                                 const sgl_kv_pair_copy_buffers *buffers, void *stream);
/* CudaKvPairCopyKernels::gather (cuda_kv_kernels.rs:506-539): pool slots ->
 * strided K/V rows. Same contract as sgl_rocm_kv_pair_scatter. */
int32_t sgl_rocm_kv_pair_gather(sgl_rocm_kv_ctx *ctx, const sgl_kv_pair_copy_plan *plan,
                                const sgl_kv_pair_copy_buffers *buffers, void *stream);

/* --- per-layer PD transfer (pack / unpack) ------------------------------ */

typedef enum sgl_kv_head_layout {
    SGL_KV_NHD = 0, /* token-major: a (page, layer, tensor) region is [page_size][heads][dim] */
    SGL_KV_HND = 1  /* head-major:  a (page, layer, tensor) region is [heads][page_size][dim] */
} sgl_kv_head_layout;

/* One layer of a page-major pool. The page -> layer -> tensor nesting and
 * the byte offsets follow PagedKvCacheLayout::tensor_token_byte_range
 * (kv_cache.rs:653-700); head_layout = HND only reorders bytes inside each
 * (page, layer, tensor) region. Build it with sgl_kv_pool_view_for_layer,
 * or fill it directly for pools this library did not describe. */
typedef struct sgl_kv_pool_view {
    void *base;                 /* device pointer to byte 0 of the pool */
    uint64_t byte_len;          /* pool allocation length */
    uint64_t page_size;         /* tokens per page */
    uint64_t page_stride_bytes; /* page_size_bytes */
    uint64_t page_count;
    uint64_t tensor_offset[2];  /* in-page offset of this layer's tensor regions */
    uint64_t row_bytes;         /* bytes per (token, tensor 0): heads * head_dim * element bytes */
    uint32_t tensor_count;      /* 2 = K/V pair, 1 = single tensor (MLA latent row) */
    uint32_t heads;             /* KV heads; HND splits a row into `heads` chunks */
    uint32_t head_layout;       /* sgl_kv_head_layout */
    uint32_t reserved;
    float *scale;               /* optional device pointer to this layer's tensor_count
                                   quantisation scales (fp8), or NULL */
    uint64_t value_row_bytes;   /* bytes per (token, tensor 1) when they differ from
                                   row_bytes (the tensor-pair layout of MLA: keys 576 and
                                   values 512 wide, kv_cache.rs:480-529); 0 = row_bytes */
} sgl_kv_pool_view;

/* Builds the view of `layer` for tensors [first_tensor, first_tensor +
 * tensor_count). Errors: layer/tensor out of range (LayerOutOfRange,
 * TensorOutOfRange, kv_cache.rs:672-685). A two-tensor view of a tensor-pair
 * layout carries each tensor's width (value_row_bytes), so one launch moves
 * a layer of keys and values of unequal widths; the reference's pair copy
 * rejects such layouts (UnevenKvPairCopy, kv_cache.rs:758-763), and so does
 * sgl_kv_paged_layout_kv_pair_copy_geometry, its drop-in. */
int32_t sgl_kv_pool_view_for_layer(const sgl_kv_paged_layout *layout, void *base,
                                   uint64_t byte_len, uint32_t head_layout, uint64_t heads,
                                   uint64_t layer_index, uint64_t first_tensor,
                                   uint64_t tensor_count, sgl_kv_pool_view *out);

/* Contiguous transfer rows: row r of tensor t at planes[t] + r * row_stride[t],
 * token-major ([token][heads][dim]). */
typedef struct sgl_kv_rows_view {
    void *planes[2];
    uint64_t plane_bytes[2];    /* allocation bytes available from planes[t] */
    uint64_t row_stride[2];
    float *scale;               /* optional device pointer receiving / supplying the
                                   layer's tensor_count scales, or NULL */
} sgl_kv_rows_view;

/* Pack (generalises sglang_gather_kv_pair_bytes, cuda_kv_kernels.rs:54-99):
 * row r of the transfer <- the pool row at physical slot slots[r], for
 * r in [0, row_count). `slots` is the per-row u64 slot map the reference
 * uploads with CudaKvStorage::upload_slot_map (cuda_kv_cache.rs:199-222);
 * it must hold row_count entries. Asynchronous on `stream` (NULL: null
 * stream); a slot outside the pool skips that row and raises the context's
 * error word (read it with sgl_rocm_kv_check_errors). row_count 0 is a
 * no-op. Scales are copied when both views carry a pointer. */
int32_t sgl_rocm_kv_pack_layer(sgl_rocm_kv_ctx *ctx, const sgl_kv_pool_view *src,
                               const sgl_kv_device_buffer *slots, uint64_t row_count,
                               const sgl_kv_rows_view *dst, void *stream);
/* Unpack (generalises sglang_scatter_kv_pair_bytes, cuda_kv_kernels.rs:
 * 11-52): the pool row at slots[r] <- transfer row r, into the decode pool
 * with its own page size and head layout. Asynchronous. */
int32_t sgl_rocm_kv_unpack_layer(sgl_rocm_kv_ctx *ctx, const sgl_kv_rows_view *src,
                                 uint64_t row_count, const sgl_kv_pool_view *dst,
                                 const sgl_kv_device_buffer *slots, void *stream);
/* Multi-layer forms: one launch covers `layer_count` consecutive layers
 * (no counterpart in the reference, which launches per layer). Layer i's
 * pool view is `src`/`dst` with every tensor_offset advanced by
 * i * pool_layer_stride (PagedKvCacheLayout::bytes_per_layer_page for a
 * paged pool); layer i's rows sit i * rows_layer_stride bytes after the
 * given planes. Scales, when given, are layer_count consecutive groups of
 * tensor_count floats. The first and last layers are validated like a
 * single-layer call, and the destination's layers must not overlap. */
int32_t sgl_rocm_kv_pack_layers(sgl_rocm_kv_ctx *ctx, const sgl_kv_pool_view *src,
                                uint64_t pool_layer_stride, uint32_t layer_count,
                                const sgl_kv_device_buffer *slots, uint64_t row_count,
                                const sgl_kv_rows_view *dst, uint64_t rows_layer_stride,
                                void *stream);
int32_t sgl_rocm_kv_unpack_layers(sgl_rocm_kv_ctx *ctx, const sgl_kv_rows_view *src,
                                  uint64_t rows_layer_stride, uint32_t layer_count,
                                  uint64_t row_count, const sgl_kv_pool_view *dst,
                                  uint64_t pool_layer_stride, const sgl_kv_device_buffer *slots,
                                  void *stream);
/* One tensor of one layer for `count` slots (u64, on the device), between a
 * pool laid out by `layout` (NHD) and rows source_offset + i *
 * source_row_stride: the batched form of
 * CudaKvStorage::write_tensor_slot_from_device / read_tensor_slot_to_device
 * (crates/sglang-srt/src/cuda_kv_cache.rs:258-294), which the MLA forward
 * pass calls once per token and tensor (cuda_mla.rs:256-271). Works for
 * tensor-pair layouts with unequal key/value widths (MLA 576/512), one
 * call per tensor. Layer and tensor are checked on the host
 * (LayerOutOfRange / TensorOutOfRange); a slot past the pool raises the
 * error word (SLOT) and its row is skipped. Asynchronous. */
int32_t sgl_rocm_kv_write_tensor_slots(sgl_rocm_kv_ctx *ctx, const sgl_kv_paged_layout *layout,
                                       const sgl_kv_device_buffer *pool, uint64_t layer,
                                       uint64_t tensor, const sgl_kv_device_buffer *slots,
                                       uint64_t count, const sgl_kv_device_buffer *source,
                                       uint64_t source_offset, uint64_t source_row_stride,
                                       void *stream);
/* Both tensors of one layer (key rows keys_offset + i * keys_row_stride,
 * value rows values_offset + i * values_row_stride; widths from the
 * layout, unequal for MLA's 576/512 pair) to `count` slots in one launch:
 * the forward-pass write the reference's MLA decode makes per token with
 * two write_tensor_slot_from_device calls (cuda_mla.rs:256-271 through
 * cuda_kv_cache.rs:258-294). Layer checked on the host (LayerOutOfRange;
 * TensorOutOfRange for a one-tensor layout); a slot past the pool raises
 * the error word (SLOT) and its row is skipped. Asynchronous. */
int32_t sgl_rocm_kv_write_tensor_pair_slots(sgl_rocm_kv_ctx *ctx, const sgl_kv_paged_layout *layout,
                                            const sgl_kv_device_buffer *pool, uint64_t layer,
                                            const sgl_kv_device_buffer *slots, uint64_t count,
                                            const sgl_kv_device_buffer *keys, uint64_t keys_offset,
                                            uint64_t keys_row_stride, const sgl_kv_device_buffer *values,
                                            uint64_t values_offset, uint64_t values_row_stride,
                                            void *stream);
int32_t sgl_rocm_kv_read_tensor_slots(sgl_rocm_kv_ctx *ctx, const sgl_kv_paged_layout *layout,
                                      const sgl_kv_device_buffer *pool, uint64_t layer,
                                      uint64_t tensor, const sgl_kv_device_buffer *slots,
                                      uint64_t count, const sgl_kv_device_buffer *destination,
                                      uint64_t destination_offset,
                                      uint64_t destination_row_stride, void *stream);
/* Pool -> pool in one pass for co-resident prefill and decode pools:
 * the composition unpack(pack(.)) without the transfer rows. */
int32_t sgl_rocm_kv_transfer_layer(sgl_rocm_kv_ctx *ctx, const sgl_kv_pool_view *src,
                                   const sgl_kv_device_buffer *src_slots, uint64_t row_count,
                                   const sgl_kv_pool_view *dst,
                                   const sgl_kv_device_buffer *dst_slots, void *stream);

/* Multi-layer pool -> pool: layer i of each side is its view with every
 * tensor_offset advanced by i * that side's layer stride. */
int32_t sgl_rocm_kv_transfer_layers(sgl_rocm_kv_ctx *ctx, const sgl_kv_pool_view *src,
                                    uint64_t src_layer_stride, uint32_t layer_count,
                                    const sgl_kv_device_buffer *src_slots, uint64_t row_count,
                                    const sgl_kv_pool_view *dst, uint64_t dst_layer_stride,
                                    const sgl_kv_device_buffer *dst_slots, void *stream);

/* A request's run of transfer rows (KvCacheTransferSpan, transfer.rs:495-505):
 * rows [row_start, row_start + token_count) hold request tokens
 * [token_offset, token_offset + token_count); token k lives in page
 * page_table[page_table_start + k / page_size] at position k % page_size.
 * token_offset > 0 is a prefix already cached on the decode side. */
typedef struct sgl_kv_span {
    uint32_t row_start;
    uint32_t token_offset;
    uint32_t token_count;
    uint32_t page_table_start;
} sgl_kv_span;

/* Expands spans + a page table (the decode side's dst_kv_indices,
 * pd_bootstrap.rs:416-494) into the per-row slot map taken by the calls
 * above, on the device. `spans` (device) must be sorted by row_start with
 * row_start[i] + token_count[i] <= row_start[i + 1]. Rows no span covers and
 * rows whose page entry is negative, past the table or >= page_count get
 * slot UINT64_MAX and raise the error word (SPAN / PAGE); the copy calls
 * then skip them. Asynchronous. */
int32_t sgl_rocm_kv_resolve_spans(sgl_rocm_kv_ctx *ctx, uint64_t page_size, uint64_t page_count,
                                  const sgl_kv_device_buffer *spans, uint64_t span_count,
                                  const sgl_kv_device_buffer *page_table, uint64_t page_table_len,
                                  uint64_t row_count, const sgl_kv_device_buffer *out_slots,
                                  void *stream);

/* --- layer pipeline (pack -> hop -> unpack, overlapped across layers) ---- */

/* A whole-request transfer, layer by layer: the device-side half of a PD
 * transfer backend (KvTransferBackend::submit, transfer.rs:1145-1151, driven
 * by execute_kv_cache_transfer_plan, transfer.rs:1205-1231). For each layer l:
 *   pack(src_layers[l]) -> send[l % 2]
 *   [staged]  D2H send -> host[l % 2] (pinned), then H2D host -> recv[l % 2]
 *   unpack(recv[l % 2], or send[l % 2] when not staged) -> dst_layers[l]
 * on four streams (pack, D2H, H2D, unpack) so that layer l + 1 packs while
 * layer l crosses the hop and layer l - 1 unpacks. The staged hop stands in
 * for the inter-node link on one GPU. Buffers are double-buffered; events
 * order every reuse. Each send/recv/host buffer holds one layer's rows as
 * [tensor][row][row bytes of the tensor] (row_count * (row_bytes +
 * value_row_bytes) bytes for a pair, row_count * row_bytes for one tensor).
 * All buffers are the caller's; host buffers must be pinned (hipHostMalloc)
 * for the copies to be asynchronous. */
typedef struct sgl_kv_pipeline_desc {
    uint32_t layers;
    uint32_t staged;                       /* 1: host hop; 0: unpack reads send[] directly */
    const sgl_kv_pool_view *src_layers;    /* host array of `layers` views (copied) */
    const sgl_kv_pool_view *dst_layers;    /* host array of `layers` views (copied) */
    sgl_kv_device_buffer src_slots;        /* u64 slot per row, source pool */
    sgl_kv_device_buffer dst_slots;        /* u64 slot per row, destination pool */
    uint64_t row_count;
    sgl_kv_device_buffer send[2];          /* device */
    sgl_kv_device_buffer recv[2];          /* device; unused when not staged */
    void *host[2];                         /* pinned host; unused when not staged */
    uint64_t host_bytes;                   /* bytes available at each host[i] */
} sgl_kv_pipeline_desc;

typedef struct sgl_rocm_kv_pipeline sgl_rocm_kv_pipeline;

/* Validates the description (every layer view against row_count and the
 * staging sizes), creates the four streams (default priority) and the
 * per-layer events. */
int32_t sgl_rocm_kv_pipeline_create(sgl_rocm_kv_ctx *ctx, const sgl_kv_pipeline_desc *desc,
                                    sgl_rocm_kv_pipeline **out);
/* Enqueues every layer and returns; `after` (a hipEvent_t or NULL) gates the
 * first pack. */
int32_t sgl_rocm_kv_pipeline_run(sgl_rocm_kv_pipeline *pipe, void *after);
/* Waits for the last unpack and reports device errors (check_errors). */
int32_t sgl_rocm_kv_pipeline_wait(sgl_rocm_kv_pipeline *pipe);
/* Durations in ms of layer `layer`'s last run: ms[0] pack, ms[1] D2H,
 * ms[2] H2D, ms[3] unpack (hop entries 0 when not staged), and ms[4] the
 * layer's latency from pack start to unpack end. */
int32_t sgl_rocm_kv_pipeline_layer_times(const sgl_rocm_kv_pipeline *pipe, uint32_t layer,
                                         float *ms);
/* Elapsed ms from the first pack start to the last unpack end of the last run. */
int32_t sgl_rocm_kv_pipeline_elapsed(const sgl_rocm_kv_pipeline *pipe, float *ms);
int32_t sgl_rocm_kv_pipeline_destroy(sgl_rocm_kv_pipeline *pipe);

/* Synthetic-input generator for benchmarks and tests; it has no counterpart
 * in the reference. Fills `buffer` (byte_len a multiple of 8) word by word:
 * word i (8 bytes) derives from z = splitmix64(seed + (i + 1) *
 * 0x9E3779B97F4A7C15). kind 0: the word is z (reproducible on the host);
 * kind 1: four bf16 N(0,1) values (Box-Muller); kind 2: four bf16 U(-1,1)
 * values. Asynchronous. */
typedef enum sgl_kv_fill_kind {
    SGL_KV_FILL_BITS = 0,
    SGL_KV_FILL_BF16_NORMAL = 1,
    SGL_KV_FILL_BF16_UNIFORM = 2
} sgl_kv_fill_kind;
int32_t sgl_rocm_kv_fill_synthetic(sgl_rocm_kv_ctx *ctx, const sgl_kv_device_buffer *buffer,
                                   uint64_t seed, uint32_t kind, void *stream);

/* Streaming ceilings of the device, for the benchmark's roofline context;
 * no counterpart in the reference. kind COPY moves `bytes` from src to
 * dst, READ reads `bytes` of src (dst receives at most 16 bytes), WRITE
 * writes `bytes` of dst; contiguous, 16-byte non-temporal vectors.
 * `bytes` is a multiple of 16. Asynchronous. */
typedef enum sgl_kv_stream_kind {
    SGL_KV_STREAM_COPY = 0,
    SGL_KV_STREAM_READ = 1,
    SGL_KV_STREAM_WRITE = 2
} sgl_kv_stream_kind;
int32_t sgl_rocm_kv_stream(sgl_rocm_kv_ctx *ctx, uint32_t kind, const sgl_kv_device_buffer *src,
                           const sgl_kv_device_buffer *dst, uint64_t bytes, void *stream);

/* Executes page requests (sgl_kv_build_page_requests /
 * sgl_kv_build_remote_page_requests output, uploaded to the device) as
 * device copies: the page-for-page PD transfer between co-resident pools of
 * equal page size and layout, one launch for the whole list instead of one
 * transport write per page (transfer.rs:3071-3137). Request i copies
 * length_i bytes from `source` to target_base + target_offset_i, where
 * target_base is target_region.ptr, or 0 when `offsets_are_addresses` (the
 * remote form, whose offsets are dst_kv_ptrs-based addresses). Every request
 * must lie inside source_region and target_region and be at most
 * `max_length` bytes; others are skipped and raise the error word (REQUEST).
 * Asynchronous. */
int32_t sgl_rocm_kv_execute_page_requests(sgl_rocm_kv_ctx *ctx,
                                          const sgl_kv_device_buffer *requests, uint64_t count,
                                          uint64_t max_length,
                                          const sgl_kv_device_buffer *source_region,
                                          const sgl_kv_device_buffer *target_region,
                                          uint32_t offsets_are_addresses, void *stream);

/* ---- Paged attention over bf16 K/V pages ----
 * The reader of the pools the copies write: CudaBf16PagedAttentionKernels
 * (crates/sglang-kernel/src/cuda_attention.rs:10-850) with the same plan,
 * metadata and results, plus head-major (HND) pages, which the reference's
 * kernel cannot read. Query q of request r attends the first
 * query_sequence_lengths[q] slots of
 * sequence_slots[request_slot_offsets[r] .. request_slot_offsets[r+1]);
 * query head h reads KV head h / (query_head_count / kv_head_count). */
typedef struct sgl_kv_attention_layout {   /* CudaBf16PagedAttentionLayout (:157-236) */
    uint64_t page_size;
    uint64_t page_stride_bytes;
    uint64_t key_in_page_offset;
    uint64_t value_in_page_offset;
    uint64_t key_row_bytes;    /* kv_head_count * query_key_head_dim * 2 */
    uint64_t value_row_bytes;  /* kv_head_count * value_head_dim * 2 */
    uint32_t head_layout;      /* SGL_KV_NHD (the reference's) or SGL_KV_HND */
    uint32_t reserved;
} sgl_kv_attention_layout;

typedef struct sgl_kv_attention_plan_config {  /* CudaBf16PagedAttentionPlanConfig (:263-275) */
    uint64_t query_count;
    uint64_t request_count;
    uint64_t sequence_slot_count;
    uint64_t slot_count;
    uint64_t query_head_count;
    uint64_t kv_head_count;
    uint64_t query_key_head_dim;
    uint64_t value_head_dim;
    float scale;
    uint32_t flags;            /* 0, SGL_KV_ATTN_EXACT_WEIGHTS or SGL_KV_ATTN_FAST_WEIGHTS */
    sgl_kv_attention_layout layout;
} sgl_kv_attention_plan_config;

/* Plan flags, with no counterpart in the reference (its config has no such
 * field); 0 is the reference's behaviour. Every body feeds its softmax
 * weights to the P.V matrix products as a hi + lo pair of bf16 values
 * (relative error about 2^-16 per weight), so outputs stay within the
 * reference's fp32-weight precision (cuda_attention.rs:138-149) up to the
 * bf16 output rounding. SGL_KV_ATTN_FAST_WEIGHTS lets the latent body (the
 * MLA shape: 576-wide keys whose first 512 dims are the values, one KV head)
 * round each weight to one bf16 value instead (at most 2^-8 relative), which
 * saves one matrix product per tile: 4 % (one query of 8,192 tokens, 128
 * heads) to 20 % (64 such queries) of that launch on MI355X. Other bodies
 * ignore it. SGL_KV_ATTN_EXACT_WEIGHTS names the default and is accepted
 * for callers that set it; setting both, or any other bit, is rejected
 * (InvalidArgument "flags") by sgl_kv_attention_plan_new and at enqueue. */
#define SGL_KV_ATTN_EXACT_WEIGHTS 1u
#define SGL_KV_ATTN_FAST_WEIGHTS 2u

typedef struct sgl_kv_attention_plan {  /* CudaBf16PagedAttentionPlan (:239-261) */
    sgl_kv_attention_plan_config config;
    uint64_t query_required_bytes;
    uint64_t query_request_indices_required_bytes;
    uint64_t query_sequence_lengths_required_bytes;
    uint64_t request_slot_offsets_required_bytes;
    uint64_t sequence_slots_required_bytes;
    uint64_t pool_required_bytes;
    uint64_t output_required_bytes;
} sgl_kv_attention_plan;

/* CudaBf16PagedAttentionLaunch (:659-674): queries bf16 [query][head][dk];
 * query_request_indices u32; query_sequence_lengths u64;
 * request_slot_offsets u64 (request_count + 1); sequence_slots u64; output
 * bf16 [query][head][dv]. */
typedef struct sgl_kv_attention_buffers {
    sgl_kv_device_buffer queries;                uint64_t queries_offset;
    sgl_kv_device_buffer query_request_indices;  uint64_t query_request_indices_offset;
    sgl_kv_device_buffer query_sequence_lengths; uint64_t query_sequence_lengths_offset;
    sgl_kv_device_buffer request_slot_offsets;   uint64_t request_slot_offsets_offset;
    sgl_kv_device_buffer sequence_slots;         uint64_t sequence_slots_offset;
    sgl_kv_device_buffer pool;                   uint64_t pool_offset;
    sgl_kv_device_buffer output;                 uint64_t output_offset;
} sgl_kv_attention_buffers;

/* CudaBf16PagedAttentionPlan::new (cuda_attention.rs:277-430): same checks,
 * same order, same variants. HND pools must hold the last page's whole key
 * and value regions. */
int32_t sgl_kv_attention_plan_new(const sgl_kv_attention_plan_config *config,
                                  sgl_kv_attention_plan *out);
/* build_plan (crates/sglang-srt/src/cuda_attention.rs:505-572): the plan for
 * layer `layer` of a bf16 pool (UnsupportedKvDtype otherwise). */
int32_t sgl_kv_attention_plan_for_layer(const sgl_kv_paged_layout *layout, uint64_t layer,
                                        uint64_t query_count, uint64_t request_count,
                                        uint64_t sequence_slot_count, uint64_t query_head_count,
                                        float scale, uint32_t head_layout,
                                        sgl_kv_attention_plan *out);
/* CudaBf16PagedAttentionKernels::forward (cuda_attention.rs:681-850):
 * checks devices and ranges, runs, synchronises `stream` and reports bad
 * metadata as SGL_KV_ATTN_DEVICE_METADATA_INVALID (the outputs of the
 * affected queries are then unspecified). It raises an error word of its
 * own, which every call leaves clear, so asynchronous launches still
 * running on other streams neither lose their errors to it nor report
 * theirs through it.
 * max_sequence_length (0 = unknown, then sequence_slot_count) bounds the
 * query lengths and steers how sequences are split across workgroups; a
 * query longer than it is reported as a sequence error (flag 0x2), not
 * truncated. Long sequences use a
 * context-owned workspace, grown on demand. */
int32_t sgl_rocm_kv_paged_attention(sgl_rocm_kv_ctx *ctx, const sgl_kv_attention_plan *plan,
                                    const sgl_kv_attention_buffers *buffers,
                                    uint64_t max_sequence_length, void *stream);
/* The same launch without the wait: nothing synchronises, and bad metadata
 * surfaces at the next sgl_rocm_kv_check_errors on `stream` (as
 * SGL_KV_ATTN_DEVICE_METADATA_INVALID). The error word is not cleared
 * first, so an earlier unchecked error stays visible. The split workspace
 * is shared by all calls on the context: issue calls that split on one
 * stream (growing it waits for the whole device). No counterpart in the
 * reference, whose forward always synchronises (cuda_attention.rs:821-829);
 * it is for decode loops that check errors once per step. */
int32_t sgl_rocm_kv_paged_attention_async(sgl_rocm_kv_ctx *ctx, const sgl_kv_attention_plan *plan,
                                          const sgl_kv_attention_buffers *buffers,
                                          uint64_t max_sequence_length, void *stream);

/* No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). sgl_rocm_kv_paged_attention_async with
 * the split records in the library's static device workspace of
 * SGL_KV_NOALLOC_WORKSPACE_BYTES bytes, instead of the context's buffer that
 * grows on demand: it calls no hipMalloc, hipFree or other allocating
 * routine. Each device the library runs on holds the workspace until the
 * process ends (its address is resolved at sgl_rocm_kv_init). A launch whose
 * records need more is rejected with SGL_KV_DIMENSION_TOO_LARGE (name
 * "workspace", a = bytes needed, b = the maximum) before anything is
 * enqueued. Every call on a device shares that device's workspace, and the
 * records a call leaves stay until the next one. Calls are therefore ordered
 * on the device: each call's launches wait for the previous call's combine
 * (an event the library keeps per device, recorded after every call), on
 * whatever stream and from whatever context of the process either was made,
 * so concurrent calls run one after another instead of overwriting each
 * other's records. A stream under graph capture skips that wait and record
 * (an event recorded outside the capture cannot be waited on inside it):
 * there the graph's own dependencies order the calls it holds, and the
 * caller must not replay such a graph while another call that uses the
 * workspace runs. Results equal those of sgl_rocm_kv_paged_attention_async
 * on the same arguments. */
#define SGL_KV_NOALLOC_WORKSPACE_BYTES (128ull << 20)
int32_t sgl_rocm_kv_paged_attention_async_noalloc(sgl_rocm_kv_ctx *ctx, const sgl_kv_attention_plan *plan,
                                                  const sgl_kv_attention_buffers *buffers,
                                                  uint64_t max_sequence_length, void *stream);

/* ---- Bootstrap wire format: the decode side's page table and layout ----
 * The multipart frames a decode worker sends a prefill worker's bootstrap
 * listener (Mooncake protocol, crates/sglang-srt/src/pd_bootstrap.rs):
 *  - KVArgs registration, part 0 "None": endpoint, port, session id, then
 *    dst_kv_ptrs (u64 LE), dst_aux_ptrs, dst_state_data_ptrs (packed u64
 *    lists), tp rank, attn tp size, dst_kv_item_len, optional packed u32
 *    lists (:416-449, encoder :685-706);
 *  - transfer metadata, part 0 the room: endpoint, port, session id,
 *    dst_kv_indices (i32 LE), aux index, dst_state_indices (packed i32
 *    lists), required_dst_info_num, optional decode_prefix_len (:451-494,
 *    encoder :720-749).
 * Integers in text parts are ASCII decimal; a packed list is a u32 LE
 * count, the u32 LE byte length of each buffer, then the buffers
 * (:1255-1270, decoder :1605-1636).
 *
 * Decode-layout extension (no counterpart in the reference): a KVArgs frame
 * may carry one more part, after the 14 the reference's encoder writes, that
 * describes the decode pool's page geometry, so a prefill side can relayout
 * (page size, NHD/HND) instead of copying page for page. A reference prefill
 * reads only parts 0..11 and ignores it. Layout of the part, little endian:
 *   u32 magic 0x4C564B53 ("SKVL"), u32 version 1,
 *   i32 dtype, u32 head_layout,
 *   u64 page_size, num_layers, kv_heads, head_dim, kv_tensors_per_token,
 *       bytes_per_token, page_size_bytes, page_count,
 *   u64 tensor_pair (0/1), key_token_bytes, value_token_bytes, heads
 * (112 bytes). */
#define SGL_KV_DECODE_LAYOUT_MAGIC 0x4C564B53u
#define SGL_KV_DECODE_LAYOUT_BYTES 112u
#define SGL_KV_BOOTSTRAP_MAX_PARTS 16u

typedef struct sgl_kv_frame_part {
    const uint8_t *data;
    uint64_t len;
} sgl_kv_frame_part;

/* The decode pool as the extension advertises it: the geometry, its head
 * layout and head chunks per row (what sgl_kv_backend_memory needs besides
 * the base pointer, which travels as dst_kv_ptrs[0]). */
typedef struct sgl_kv_decode_layout {
    sgl_kv_paged_layout layout;
    uint32_t head_layout;  /* sgl_kv_head_layout */
    uint32_t reserved;
    uint64_t heads;        /* 0 = layout.runtime.kv_heads */
} sgl_kv_decode_layout;

/* A flattened list of lists: list i is values[offsets[i] .. offsets[i+1]),
 * offsets has count + 1 entries. */
typedef struct sgl_kv_u64_lists { const uint64_t *values; const uint64_t *offsets; uint64_t count; } sgl_kv_u64_lists;
typedef struct sgl_kv_u32_lists { const uint32_t *values; const uint64_t *offsets; uint64_t count; } sgl_kv_u32_lists;
typedef struct sgl_kv_i32_lists { const int32_t *values; const uint64_t *offsets; uint64_t count; } sgl_kv_i32_lists;

/* MooncakeKvArgsRegisterInfo (pd_bootstrap.rs:416-429) / the encoder's
 * MooncakeDecodeKvArgsRegistration (:671-683). Strings are NUL-terminated.
 * As a view returned by sgl_kv_bootstrap_get_kv_args, every pointer stays valid
 * until the next ingest into, or the destruction of, the state. */
typedef struct sgl_kv_bootstrap_kv_args {
    const char *endpoint;
    const char *mooncake_session_id;
    uint32_t dst_port;
    int32_t dst_tp_rank;
    uint64_t dst_attn_tp_size;
    uint64_t dst_kv_item_len;
    const uint64_t *dst_kv_ptrs;  uint64_t dst_kv_ptr_count;
    const uint64_t *dst_aux_ptrs; uint64_t dst_aux_ptr_count;
    sgl_kv_u64_lists dst_state_data_ptrs;
    sgl_kv_u32_lists dst_state_item_lens;
    sgl_kv_u32_lists dst_state_dim_per_tensor;
    const sgl_kv_decode_layout *decode_layout;  /* NULL: none advertised */
} sgl_kv_bootstrap_kv_args;

/* MooncakeTransferInfo (pd_bootstrap.rs:451-462) / the encoder's
 * MooncakeDecodeTransferMetadata (:708-718). */
typedef struct sgl_kv_bootstrap_transfer {
    uint64_t room;
    const char *endpoint;
    const char *mooncake_session_id;
    uint32_t dst_port;
    uint32_t is_dummy;
    const int32_t *dst_kv_indices; uint64_t dst_kv_index_count;
    uint32_t has_dst_aux_index;
    int32_t dst_aux_index;
    sgl_kv_i32_lists dst_state_indices;
    uint64_t required_dst_info_num;
    uint32_t has_decode_prefix_len;
    uint32_t reserved;
    uint64_t decode_prefix_len;
} sgl_kv_bootstrap_transfer;

/* MooncakeRemoteKvLayout (crates/sglang-srt/src/transfer.rs:1651-1656) of
 * one decode session, plus the advertised decode layout if any. */
typedef struct sgl_kv_remote_kv_layout {
    const char *mooncake_session_id;
    const uint64_t *dst_kv_ptrs;    uint64_t dst_kv_ptr_count;
    const int32_t *dst_kv_indices;  uint64_t dst_kv_index_count;
    uint64_t dst_kv_item_len;
    const sgl_kv_decode_layout *decode_layout;  /* NULL: none advertised */
} sgl_kv_remote_kv_layout;

/* The Mooncake tables of PrefillBootstrapState (pd_bootstrap.rs:150-235). */
typedef struct sgl_kv_bootstrap sgl_kv_bootstrap;
int32_t sgl_kv_bootstrap_create(sgl_kv_bootstrap **out);
int32_t sgl_kv_bootstrap_destroy(sgl_kv_bootstrap *state);
/* ingest_mooncake_bootstrap_frame (:180-217): "WATERMARK" and
 * "STAGING_RSP" frames are accepted and ignored, "None" registers KVArgs
 * (replacing the session's previous registration), anything else is
 * transfer metadata for a room, which turns WaitingForInput once
 * required_dst_info_num sessions have reported. Errors leave the state
 * unchanged. */
int32_t sgl_kv_bootstrap_ingest(sgl_kv_bootstrap *state, const sgl_kv_frame_part *parts, uint32_t part_count);
/* KVArgs registrations ingested so far (decode_kv_args_registration_count). */
int32_t sgl_kv_bootstrap_registration_count(const sgl_kv_bootstrap *state, uint64_t *count);
/* decode_kv_args (:221-223); SGL_KV_BOOT_MISSING_KV_ARGS (room 0) when the
 * session has not registered. */
int32_t sgl_kv_bootstrap_get_kv_args(const sgl_kv_bootstrap *state, const char *mooncake_session_id,
                                 sgl_kv_bootstrap_kv_args *out);
/* transfer_status (:233-235): *status = KvPoll (Failed 0, Bootstrapping 1,
 * WaitingForInput 2, Transferring 3, Success 4; transfer.rs:355-361), or -1
 * for an unknown room. */
int32_t sgl_kv_bootstrap_transfer_status(const sgl_kv_bootstrap *state, uint64_t room, int32_t *status);
/* MooncakeTransferRoom (:497-502): the room's required_dst_info_num,
 * decode_prefix_len (has = 0: none) and the sessions reported so far. */
int32_t sgl_kv_bootstrap_room(const sgl_kv_bootstrap *state, uint64_t room, uint64_t *required_dst_info_num,
                              uint32_t *has_decode_prefix_len, uint64_t *decode_prefix_len,
                              uint64_t *session_count);
/* One session's transfer metadata in a room. */
int32_t sgl_kv_bootstrap_get_transfer(const sgl_kv_bootstrap *state, uint64_t room, const char *mooncake_session_id,
                                  sgl_kv_bootstrap_transfer *out);
/* remote_kv_layouts_for_room (:237-270): one entry per non-dummy session,
 * in session-id order; writes up to `capacity`, *count = the total. */
int32_t sgl_kv_bootstrap_remote_layouts(const sgl_kv_bootstrap *state, uint64_t room,
                                        sgl_kv_remote_kv_layout *out, uint64_t capacity, uint64_t *count);
/* The encoders (:685-706 and :720-749): write the frame's parts into `buf`
 * and describe them in parts[SGL_KV_BOOTSTRAP_MAX_PARTS]. With buf NULL,
 * only *bytes_needed is computed; a non-NULL buf shorter than that is
 * AllocationOutOfBounds. The KVArgs frame has 14 parts as the reference
 * writes it, 15 with a decode layout. A non-dummy transfer without an aux
 * index is SGL_KV_BOOT_MISSING_AUX_INDEX. */
int32_t sgl_kv_bootstrap_encode_kv_args(const sgl_kv_bootstrap_kv_args *args, uint8_t *buf, uint64_t capacity,
                                        sgl_kv_frame_part *parts, uint32_t *part_count,
                                        uint64_t *bytes_needed);
int32_t sgl_kv_bootstrap_encode_transfer(const sgl_kv_bootstrap_transfer *transfer, uint8_t *buf,
                                         uint64_t capacity, sgl_kv_frame_part *parts, uint32_t *part_count,
                                         uint64_t *bytes_needed);

/* ---- Transfer backend: KvTransferBackend (transfer.rs:1145-1151) ----
 * register / submit / poll / cancel / shutdown for a prefill pool and a
 * decode pool on this context's device. A span's rows are validated on the
 * host at submit, then moved asynchronously:
 *   DIRECT  one pool-to-pool launch over all layers (transfer_layers);
 *   STAGED  the layer pipeline with the pinned-host hop (pack -> D2H ->
 *           H2D -> unpack), spans in submission order over shared staging.
 * poll reports each finished span once (poll_submitted_transfers,
 * transfer.rs:2633-2674); cancel drops a room's spans without an event
 * (cancel_submitted_transfers_for_room, transfer.rs:2605-2631). Calls on one
 * backend must not overlap. */
typedef struct sgl_rocm_kv_backend sgl_rocm_kv_backend;

typedef enum sgl_kv_backend_mode {
    SGL_KV_BACKEND_DIRECT = 0,
    SGL_KV_BACKEND_STAGED = 1
} sgl_kv_backend_mode;

typedef struct sgl_kv_backend_config {
    uint32_t mode;       /* sgl_kv_backend_mode */
    uint32_t reserved;
    uint64_t max_rows;   /* largest token_count a span may carry; sizes the staging */
} sgl_kv_backend_config;

/* One side's TransferableKvCacheMemory (defined in the un-vendored
 * nexus-transfer crate, pinned at crates/sglang-srt/Cargo.toml:35; provided
 * by kv_cache.rs's KvCacheMemoryProvider): the pool's layout and its device
 * allocation. Layouts of one or two tensors per token are moved whole (a
 * tensor pair of unequal widths in one launch per layer); register rejects
 * layouts of more tensors. */
typedef struct sgl_kv_backend_memory {
    sgl_kv_paged_layout layout;
    void *base;
    uint64_t byte_len;
    uint32_t head_layout;  /* sgl_kv_head_layout */
    uint32_t reserved;
    uint64_t heads;        /* head chunks per row; 0 = layout.runtime.kv_heads */
} sgl_kv_backend_memory;

/* One KvCacheTransferSpan (transfer.rs:495-505) as the decode side sees it:
 * rows token_offset .. token_offset+token_count of the request move from
 * prefill slots cache_slots[i] to decode slot
 * dst_page_table[(token_offset+i) / decode_page_size] * decode_page_size +
 * (token_offset+i) % decode_page_size. Host arrays, read during submit. */
typedef struct sgl_kv_transfer_span_desc {
    uint64_t bootstrap_room;
    char descriptor_checksum[65];  /* NUL-terminated hex (sgl_kv_transfer_span_checksum) */
    char reserved[7];
    uint64_t token_offset;
    uint64_t token_count;
    const uint64_t *cache_slots;     /* token_count prefill slots */
    const int32_t *dst_page_table;   /* decode pages of the request */
    uint64_t dst_page_table_len;
} sgl_kv_transfer_span_desc;

/* KvTransferEventStatus (transfer.rs:1066-1071). */
typedef enum sgl_kv_transfer_status {
    SGL_KV_TRANSFER_COMPLETED = 0,
    SGL_KV_TRANSFER_FAILED = 1,
    SGL_KV_TRANSFER_CANCELED = 2
} sgl_kv_transfer_status;

/* KvTransferCompletionEvent (transfer.rs:1073-1078); a failed event carries
 * the status code of the device error in error_code. */
typedef struct sgl_kv_transfer_event {
    uint64_t bootstrap_room;
    char descriptor_checksum[65];
    char reserved[3];
    int32_t status;       /* sgl_kv_transfer_status */
    int32_t error_code;   /* SGL_KV_OK unless FAILED */
} sgl_kv_transfer_event;

int32_t sgl_rocm_kv_backend_create(sgl_rocm_kv_ctx *ctx, const sgl_kv_backend_config *config,
                                   sgl_rocm_kv_backend **out);
/* Registers both pools; their layer count, tensors per token and token
 * widths must agree. STAGED allocates its staging here (4 device and 2
 * pinned host buffers of one layer's rows at max_rows). */
int32_t sgl_rocm_kv_backend_register(sgl_rocm_kv_backend *backend,
                                     const sgl_kv_backend_memory *prefill,
                                     const sgl_kv_backend_memory *decode);
/* Validates the span (prefill slots, decode page table entries) and
 * enqueues its transfer; a span with token_count 0 completes at once. At
 * most 1,024 spans may be in flight (DimensionTooLarge beyond): each owns
 * one of the backend's error words until poll reports it. */
int32_t sgl_rocm_kv_backend_submit(sgl_rocm_kv_backend *backend,
                                   const sgl_kv_transfer_span_desc *span);
/* The same with dst_page_table a device pointer (dst_page_table_len int32
 * entries on the backend's device, valid until the span is reported), as a
 * decode page table received into device memory: the prefill slots are
 * validated on the host, the decode slots are resolved on the device
 * (sgl_rocm_kv_resolve_spans). A row whose page entry is negative, past the
 * table or past the decode pool is skipped and fails the span: poll reports
 * it FAILED with SGL_KV_DEVICE_PAGE_INDEX_OUT_OF_RANGE, and the span's other
 * rows and every other span are moved normally. No counterpart in the
 * reference, whose Mooncake executor reads the indices on the host
 * (transfer.rs:2298-2329 reports the failure). */
int32_t sgl_rocm_kv_backend_submit_device_table(sgl_rocm_kv_backend *backend,
                                                const sgl_kv_transfer_span_desc *span);
/* Writes up to `capacity` events for finished spans; *pending = spans
 * submitted, not canceled and not yet reported. Never blocks on transfers. */
int32_t sgl_rocm_kv_backend_poll(sgl_rocm_kv_backend *backend, sgl_kv_transfer_event *events,
                                 uint64_t capacity, uint64_t *event_count, uint64_t *pending);
int32_t sgl_rocm_kv_backend_cancel(sgl_rocm_kv_backend *backend, uint64_t bootstrap_room);
/* Blocks until every submitted span has finished on the device (no events
 * are consumed). */
int32_t sgl_rocm_kv_backend_wait(sgl_rocm_kv_backend *backend);
/* Drains, releases every transfer and the staging, and forgets the pools. */
int32_t sgl_rocm_kv_backend_shutdown(sgl_rocm_kv_backend *backend);
int32_t sgl_rocm_kv_backend_destroy(sgl_rocm_kv_backend *backend);

/* ---- KV storage: the pool's device memory (CudaKvStorage, crates/sglang-srt/src/cuda_kv_cache.rs:170-509) ----
 * One library-owned device allocation holding a paged pool (page -> layer ->
 * tensor -> token, PagedKvCacheLayout), zero-filled at allocation like
 * CudaKvStorage::allocate (:177-189) and freed by sgl_rocm_kv_storage_destroy
 * (the reference frees on Drop, crates/sglang-kernel/src/cuda.rs:693-708). A
 * storage records the device of the context that allocated it and does not
 * keep the context. Every call that takes a layout first checks it against
 * the storage (validate_layout, :391-405): StorageSizeMismatch unless
 * byte_len == layout.total_byte_len, then PageBufferSizeMismatch unless the
 * storage's page_size_bytes == layout.runtime.page_size_bytes. Writes to one
 * storage must not overlap other calls on it (the reference takes &mut self). */
typedef struct sgl_rocm_kv_storage sgl_rocm_kv_storage;
/* CudaKvCacheSlotMap (:109-140): a validated slot list uploaded as u64. */
typedef struct sgl_rocm_kv_slot_map sgl_rocm_kv_slot_map;

/* CudaContext::memory_info (crates/sglang-kernel/src/cuda.rs:496-511):
 * hipMemGetInfo on the context's device. */
int32_t sgl_rocm_kv_memory_info(const sgl_rocm_kv_ctx *ctx, uint64_t *free_bytes, uint64_t *total_bytes);
/* CudaKvStorage::allocate (cuda_kv_cache.rs:177-189): byte_len bytes on the
 * context's device, every byte zero when the call returns. byte_len 0 is
 * ZeroAllocation (CudaContext::allocate, cuda.rs:477-480). page_size_bytes
 * is recorded for validate_layout and the memory descriptor. */
int32_t sgl_rocm_kv_storage_allocate(sgl_rocm_kv_ctx *ctx, uint64_t byte_len, uint64_t page_size_bytes,
                                     sgl_rocm_kv_storage **out);
/* allocate_cuda_kv_cache (cuda_kv_cache.rs:478-490): PagedKvCacheLayout::new
 * (runtime, page_count), then a zero-filled storage of its total_byte_len and
 * page_size_bytes; *layout receives the pool's layout (KvCachePool::layout). */
int32_t sgl_rocm_kv_cache_allocate(sgl_rocm_kv_ctx *ctx, const sgl_kv_runtime_layout *runtime,
                                   uint64_t page_count, sgl_kv_paged_layout *layout,
                                   sgl_rocm_kv_storage **out);
/* The same for a layout built elsewhere (a tensor pair from
 * sgl_kv_paged_layout_new_with_tensor_pair or sgl_kv_paged_layout_for_model):
 * CudaKvStorage::allocate of layout->total_byte_len, then KvCachePool::new's
 * size check (kv_cache.rs:849-856). */
int32_t sgl_rocm_kv_pool_allocate(sgl_rocm_kv_ctx *ctx, const sgl_kv_paged_layout *layout,
                                  sgl_rocm_kv_storage **out);

/* What sgl_rocm_kv_storage_allocate_placed measured. */
#define SGL_KV_PLACEMENT_MAX_CANDIDATES 8u
typedef struct sgl_kv_placement_report {
    uint32_t candidates;  /* allocations probed (fewer than asked when the device ran out) */
    uint32_t chosen;      /* index of the one kept */
    uint64_t probe_rows;  /* rows each probe scattered */
    float probe_us[SGL_KV_PLACEMENT_MAX_CANDIDATES]; /* median probe launch per candidate, µs */
} sgl_kv_placement_report;

/* No counterpart in the reference, which allocates one pool
 * (CudaKvStorage::allocate, cuda_kv_cache.rs:177-189). On MI355X the same
 * scatter into a pool runs at one of two speeds depending on where the
 * allocation lands in physical memory (Llama-3-8B-shape unpack: 177-183 or
 * 205-211 µs per layer), fixed for the allocation's lifetime, and no HIP
 * allocation call selects it. This call allocates `candidates` (1..8) buffers
 * of byte_len bytes at once and probes each: up to 131,072 rows of the layer
 * `probe_view` describes (its base and byte_len replaced by the candidate's;
 * the rows' pages a fixed permutation of the pool's pages) are packed into
 * `probe_rows` and unpacked back, one warm-up and five timed rounds on
 * `stream`, and the median unpack is kept. It keeps the fastest candidate,
 * frees the others, and zero-fills the one it returns, as
 * sgl_rocm_kv_storage_allocate does. `probe_rows` is scratch for the probe
 * (its contents are overwritten): pass the buffer the caller will unpack
 * from, at least one row of the view's tensors. A caller that will fill the
 * pool from another pool on the device (sgl_rocm_kv_transfer_layer) passes
 * that pool's layer as `probe_source` instead: each round is then one timed
 * pool-to-pool transfer of up to 131,072 rows (a fixed permutation of the
 * source's pages) into the candidate, the source only read, and probe_rows
 * may be NULL. Past the first candidate, an allocation the device cannot
 * satisfy ends the probing instead of failing the call. Peak device memory
 * during the call is candidates x byte_len. `report` may be NULL. */
int32_t sgl_rocm_kv_storage_allocate_placed(sgl_rocm_kv_ctx *ctx, uint64_t byte_len,
                                            uint64_t page_size_bytes, const sgl_kv_pool_view *probe_view,
                                            const sgl_kv_device_buffer *probe_rows,
                                            const sgl_kv_pool_view *probe_source, uint32_t candidates,
                                            void *stream, sgl_rocm_kv_storage **out,
                                            sgl_kv_placement_report *report);
/* Frees the allocation; NULL is accepted. Slot maps uploaded through the
 * storage stay valid (they own their memory). */
int32_t sgl_rocm_kv_storage_destroy(sgl_rocm_kv_storage *storage);
/* CudaKvStorage::allocation (:191-197): device pointer and byte length, the
 * `pool` buffer of every copy entry point. */
int32_t sgl_rocm_kv_storage_allocation(const sgl_rocm_kv_storage *storage, sgl_kv_device_buffer *out);
/* KvCacheStorage::byte_len (kv_cache.rs:825-828; impl :444-447); 0 for NULL. */
uint64_t sgl_rocm_kv_storage_byte_len(const sgl_rocm_kv_storage *storage);
/* The page size the storage was allocated for; 0 for NULL. */
uint64_t sgl_rocm_kv_storage_page_size_bytes(const sgl_rocm_kv_storage *storage);
/* The storage's device ordinal (CudaDeviceAllocation::device_ordinal); -1 for NULL. */
int32_t sgl_rocm_kv_storage_device(const sgl_rocm_kv_storage *storage);
/* KvCacheStorage::clear (impl :449-452, allocation.fill(0)): every byte zero
 * when the call returns. */
int32_t sgl_rocm_kv_storage_clear(sgl_rocm_kv_storage *storage);
/* CudaKvStorage::validate_layout (:391-405). */
int32_t sgl_rocm_kv_storage_validate_layout(const sgl_rocm_kv_storage *storage,
                                            const sgl_kv_paged_layout *layout);
/* CudaKvStorage::write_page / read_page (:224-256): one whole page between
 * host memory and the pool. `len` must equal layout.runtime.page_size_bytes
 * (PageBufferSizeMismatch), the page must exist (PageOutOfRange). Both return
 * when the copy is complete. */
int32_t sgl_rocm_kv_storage_write_page(sgl_rocm_kv_storage *storage, const sgl_kv_paged_layout *layout,
                                       uint64_t page_index, const void *bytes, uint64_t len);
int32_t sgl_rocm_kv_storage_read_page(const sgl_rocm_kv_storage *storage, const sgl_kv_paged_layout *layout,
                                      uint64_t page_index, void *bytes, uint64_t len);
/* CudaKvStorage::write_tensor_slot_from_device / read_tensor_slot_to_device
 * (:258-294): one (layer, tensor, slot)'s bytes (tensor_slot_byte_range)
 * device to device. The other buffer must be on the storage's device
 * (DeviceMismatch, CudaDeviceAllocation::copy_from_device, cuda.rs:827-857)
 * and hold the range (AllocationOutOfBounds). Asynchronous on `stream`;
 * sgl_rocm_kv_write_tensor_slots is the batched form. */
int32_t sgl_rocm_kv_storage_write_tensor_slot(sgl_rocm_kv_storage *storage, const sgl_kv_paged_layout *layout,
                                              uint64_t layer, uint64_t tensor, uint64_t slot,
                                              const sgl_kv_device_buffer *source, uint64_t source_offset,
                                              void *stream);
int32_t sgl_rocm_kv_storage_read_tensor_slot(const sgl_rocm_kv_storage *storage, const sgl_kv_paged_layout *layout,
                                             uint64_t layer, uint64_t tensor, uint64_t slot,
                                             const sgl_kv_device_buffer *destination,
                                             uint64_t destination_offset, void *stream);

/* CudaKvCacheTensorLocation (:103-107). */
typedef struct sgl_kv_tensor_location {
    uint64_t device_ptr;
    uint64_t byte_offset;
    uint64_t byte_len;
} sgl_kv_tensor_location;
/* CudaKvStorage::tensor_location / slot_location (:376-403): the byte range
 * of tensor_token_byte_range / tensor_slot_byte_range and its device address. */
int32_t sgl_rocm_kv_storage_tensor_location(const sgl_rocm_kv_storage *storage,
                                            const sgl_kv_paged_layout *layout, uint64_t page_index,
                                            uint64_t layer, uint64_t tensor, uint64_t token,
                                            sgl_kv_tensor_location *out);
int32_t sgl_rocm_kv_storage_slot_location(const sgl_rocm_kv_storage *storage,
                                          const sgl_kv_paged_layout *layout, uint64_t layer,
                                          uint64_t tensor, uint64_t slot, sgl_kv_tensor_location *out);

/* CudaKvStorage::upload_slot_map (:199-222): validate_layout, then the
 * slots against the layout (validate_slot_indices: EmptySlotMap,
 * BatchSlotOutOfRange), then a new device array of slot_len u64 slots. The
 * map remembers the host slots and the layout's slot_count. */
int32_t sgl_rocm_kv_storage_upload_slot_map(const sgl_rocm_kv_storage *storage,
                                            const sgl_kv_paged_layout *layout, const uint64_t *slots,
                                            uint64_t slot_len, sgl_rocm_kv_slot_map **out);
int32_t sgl_rocm_kv_slot_map_destroy(sgl_rocm_kv_slot_map *map);
/* CudaKvCacheSlotMap::allocation / len / slots (:126-140). */
int32_t sgl_rocm_kv_slot_map_allocation(const sgl_rocm_kv_slot_map *map, sgl_kv_device_buffer *out);
uint64_t sgl_rocm_kv_slot_map_len(const sgl_rocm_kv_slot_map *map);
const uint64_t *sgl_rocm_kv_slot_map_slots(const sgl_rocm_kv_slot_map *map);

/* The key and value rows of CudaKvSlotScatterLaunch / CudaKvSlotGatherLaunch
 * (:142-166). */
typedef struct sgl_kv_slot_rows {
    sgl_kv_device_buffer keys;
    uint64_t keys_offset;
    uint64_t key_row_stride_bytes;
    sgl_kv_device_buffer values;
    uint64_t values_offset;
    uint64_t value_row_stride_bytes;
} sgl_kv_slot_rows;
/* CudaKvStorage::write_kv_slots_from_device / read_kv_slots_to_device
 * (:296-374): validate_slot_map (:407-421: validate_layout,
 * SlotMapCapacityMismatch, the map's slots against the layout), the layer's
 * pair-copy plan (kv_pair_copy_plan, :510-532: kv_pair_copy_geometry, then
 * CudaKvPairCopyPlan::new with the map's length as row_count), then
 * sgl_rocm_kv_pair_scatter / sgl_rocm_kv_pair_gather on `stream` with the
 * storage as the pool (synchronous, as those are). */
int32_t sgl_rocm_kv_storage_write_kv_slots(sgl_rocm_kv_ctx *ctx, sgl_rocm_kv_storage *storage,
                                           const sgl_kv_paged_layout *layout, uint64_t layer,
                                           const sgl_rocm_kv_slot_map *map, const sgl_kv_slot_rows *rows,
                                           void *stream);
int32_t sgl_rocm_kv_storage_read_kv_slots(sgl_rocm_kv_ctx *ctx, const sgl_rocm_kv_storage *storage,
                                          const sgl_kv_paged_layout *layout, uint64_t layer,
                                          const sgl_rocm_kv_slot_map *map, const sgl_kv_slot_rows *rows,
                                          void *stream);

/* KvCacheMemoryLocation (nexus-transfer; the variants named at
 * crates/sglang-srt/src/transfer.rs:1662-1676). */
typedef enum sgl_kv_memory_location_kind {
    SGL_KV_LOCATION_CPU = 0,   /* id = numa_node */
    SGL_KV_LOCATION_CUDA = 1,
    SGL_KV_LOCATION_ROCM = 2,
    SGL_KV_LOCATION_MUSA = 3,
    SGL_KV_LOCATION_NPU = 4,
    SGL_KV_LOCATION_METAL = 5,
    SGL_KV_LOCATION_XPU = 6,
    SGL_KV_LOCATION_HPU = 7
} sgl_kv_memory_location_kind;

/* TransferableKvCacheRegion (used at cuda_kv_cache.rs:464-468). */
typedef struct sgl_kv_memory_region {
    uint64_t base_addr;
    uint64_t byte_len;
    uint64_t page_size_bytes;
} sgl_kv_memory_region;

#define SGL_KV_MAX_MEMORY_REGIONS 8u
/* TransferableKvCacheMemory (nexus-transfer, un-vendored: pinned at
 * crates/sglang-srt/Cargo.toml:35): regions, the logical page size and the
 * memory location. */
typedef struct sgl_kv_transferable_memory {
    sgl_kv_memory_region regions[SGL_KV_MAX_MEMORY_REGIONS];
    uint64_t region_count;
    uint64_t page_size_bytes;
    int32_t location_kind;  /* sgl_kv_memory_location_kind */
    int32_t location_id;    /* device id, or numa node for CPU */
} sgl_kv_transferable_memory;

/* KvCacheMemoryProvider::transferable_kv_cache_memory for the storage
 * (impl :455-476), with location KvCacheMemoryLocation::Rocm { device_id }:
 * one region {base, byte_len, page_size_bytes}. The descriptor's own checks
 * live in nexus-transfer, which the reference tree does not hold; this
 * library rejects (StorageDescriptor) a zero page size and a region that is
 * not a whole number of pages, the conditions its consumers reject
 * (model_executor.rs:687-692). */
int32_t sgl_rocm_kv_storage_transferable_memory(const sgl_rocm_kv_storage *storage,
                                                sgl_kv_transferable_memory *out);
/* The storage as the transfer backend registers it (sgl_kv_backend_memory),
 * after validate_layout. heads 0 = layout.runtime.kv_heads. */
int32_t sgl_rocm_kv_storage_backend_memory(const sgl_rocm_kv_storage *storage,
                                           const sgl_kv_paged_layout *layout, uint32_t head_layout,
                                           uint64_t heads, sgl_kv_backend_memory *out);
/* MooncakeMemoryLocationExt::mooncake_memory_location_label
 * (transfer.rs:1662-1676): "cpu:{numa}", "cuda:{id}", "hip:{id}",
 * "musa:{id}", "npu:{id}"; Metal, Xpu and Hpu are UnsupportedMemoryLocation. */
int32_t sgl_kv_memory_location_label(int32_t location_kind, int32_t location_id, char out[32]);
/* MooncakeKvCacheMemoryExt::mooncake_decode_remote_layout (transfer.rs:
 * 1693-1703): dst_kv_ptrs = each region's base address (capacity entries
 * available at dst_kv_ptrs; *ptr_count = region_count) and dst_kv_item_len =
 * page_size_bytes / region_count. The indices are the caller's. A
 * descriptor without regions is StorageDescriptor. */
int32_t sgl_kv_transferable_memory_decode_remote_layout(const sgl_kv_transferable_memory *memory,
                                                        uint64_t *dst_kv_ptrs, uint64_t capacity,
                                                        uint64_t *ptr_count, uint64_t *dst_kv_item_len);

/* After the work queued on `stream`, reads and clears (atomically, on the
 * device) the error words of the asynchronous calls: the copies' word and
 * the asynchronous attention's. Maps them to
 * SGL_KV_DEVICE_PAGE_INDEX_OUT_OF_RANGE, _SPAN_, _SLOT_INDEX_ or _REQUEST_
 * (the first raised, in that order: a row span resolution could not place
 * also reaches the copies as a bad slot), then
 * SGL_KV_ATTN_DEVICE_METADATA_INVALID. The synchronous pair scatter/gather
 * and paged attention keep words of their own. Replaces the flag readback of
 * cuda_kv_kernels.rs:613-621 for the asynchronous calls. The values are read
 * back through one context-owned slot, so, like every call on a context,
 * calls from different host threads must not overlap. */
int32_t sgl_rocm_kv_check_errors(sgl_rocm_kv_ctx *ctx, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* SGL_ROCM_KV_H */
