// kv_storage.cpp -- the pool's device memory: the ROCm counterpart of
// CudaKvStorage (crates/sglang-srt/src/cuda_kv_cache.rs:170-509), of its
// KvCacheStorage / KvCacheMemoryProvider impls (:444-476) and of
// allocate_cuda_kv_cache (:478-490), plus the Mooncake descriptor helpers the
// transfer side derives from the pool (crates/sglang-srt/src/transfer.rs:
// 1662-1703).
//
// A storage is one hipMalloc'd allocation, zero-filled before it is handed
// out. Addressing is PagedKvCacheLayout's (kv_layout.cpp); the slot copies
// reuse the pair scatter/gather drop-ins (kv_runtime.cpp) with the storage
// as their pool.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <vector>

#include "kv_internal.h"

using namespace sglkv;

struct sgl_rocm_kv_storage {
    int device;
    void *base;
    uint64_t byte_len;
    uint64_t page_size_bytes;
};

struct sgl_rocm_kv_slot_map {
    int device;
    void *base;                  // slot_len u64 slots on the device
    std::vector<uint64_t> slots; // the host copy the map was validated with
    uint64_t slot_count;         // the layout's slot count at upload
};

namespace {

int32_t null_arg(const char *name) {
    return fail(SGL_KV_INVALID_ARGUMENT, name, 0, 0, 0, "null argument");
}

int32_t size_mismatch(const char *what, uint64_t expected, uint64_t actual) {
    const bool pool = strcmp(what, "pool") == 0;
    return fail(SGL_KV_STORAGE_SIZE_MISMATCH, what, expected, actual, 0,
                pool ? "KV cache storage has %llu bytes but layout requires exactly %llu bytes"
                     : "ROCm KV storage has %llu bytes but layout requires exactly %llu bytes",
                (unsigned long long)actual, (unsigned long long)expected);
}

int32_t page_buffer_mismatch(uint64_t expected, uint64_t actual, bool buffer) {
    return fail(SGL_KV_STORAGE_PAGE_BUFFER_SIZE_MISMATCH, buffer ? "page_buffer" : "page_size_bytes",
                expected, actual, 0,
                "ROCm KV page buffer has %llu bytes but requires exactly %llu bytes",
                (unsigned long long)actual, (unsigned long long)expected);
}

// CudaKvStorage::validate_layout (cuda_kv_cache.rs:391-405).
int32_t validate_layout(const sgl_rocm_kv_storage *s, const sgl_kv_paged_layout *layout) {
    if (!s) return null_arg("storage");
    if (!layout) return null_arg("layout");
    if (s->byte_len != layout->total_byte_len) return size_mismatch("storage", layout->total_byte_len, s->byte_len);
    if (s->page_size_bytes != layout->runtime.page_size_bytes)
        return page_buffer_mismatch(layout->runtime.page_size_bytes, s->page_size_bytes, false);
    return SGL_KV_OK;
}

// CudaContext::allocate (crates/sglang-kernel/src/cuda.rs:477-494) + fill(0)
// (:859-873), as CudaKvStorage::allocate (cuda_kv_cache.rs:177-189) does.
int32_t allocate(sgl_rocm_kv_ctx *ctx, uint64_t byte_len, uint64_t page_size_bytes,
                 sgl_rocm_kv_storage **out) {
    if (!out) return null_arg("out");
    *out = nullptr;
    if (!ctx) return null_arg("ctx");
    if (byte_len == 0)
        return fail(SGL_KV_ZERO_ALLOCATION, nullptr, 0, 0, 0, "ROCm allocation of zero bytes");
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    void *base = nullptr;
    hipError_t err = hipMalloc(&base, byte_len);
    if (err != hipSuccess) return hip_fail(err, "hipMalloc");
    err = hipMemsetAsync(base, 0, byte_len, nullptr);
    if (err == hipSuccess) err = hipStreamSynchronize(nullptr);
    if (err != hipSuccess) {
        (void)hipFree(base);
        return hip_fail(err, "hipMemsetAsync");
    }
    *out = new sgl_rocm_kv_storage{ctx->device, base, byte_len, page_size_bytes};
    return ok();
}

// CudaDeviceAllocation::device_ptr_at (cuda.rs:895-916) for a caller buffer.
int32_t buffer_range(const char *name, const sgl_kv_device_buffer &b, uint64_t offset, uint64_t len,
                     uint64_t *addr) {
    uint64_t end;
    if (add_ovf(offset, len, &end) || end > b.byte_len)
        return fail(SGL_KV_ALLOCATION_OUT_OF_BOUNDS, name, offset, len, b.byte_len,
                    "allocation %s range [%llu, +%llu) exceeds its %llu bytes", name,
                    (unsigned long long)offset, (unsigned long long)len, (unsigned long long)b.byte_len);
    *addr = (uint64_t)(uintptr_t)b.ptr + offset;
    return SGL_KV_OK;
}

// CudaDeviceAllocation::copy_from_device's DeviceMismatch (cuda.rs:834-839):
// the other buffer must live on the storage's device.
int32_t same_device(const sgl_rocm_kv_storage *s, const char *name, const sgl_kv_device_buffer &b) {
    hipPointerAttribute_t attr;
    memset(&attr, 0, sizeof attr);
    int dev = -1;
    if (hipPointerGetAttributes(&attr, b.ptr) == hipSuccess)
        dev = attr.type == hipMemoryTypeHost ? -1 : attr.device;
    else
        (void)hipGetLastError();
    if (dev != s->device)
        return fail(SGL_KV_DEVICE_MISMATCH, name, (uint64_t)s->device, (uint64_t)(int64_t)dev, 0,
                    "ROCm copy between device %d and device %d", dev, s->device);
    return SGL_KV_OK;
}

// One (layer, tensor, slot) range between the pool and a caller buffer,
// device to device (write_tensor_slot_from_device / read_tensor_slot_to_device,
// cuda_kv_cache.rs:258-294).
int32_t tensor_slot_copy(const sgl_rocm_kv_storage *s, const sgl_kv_paged_layout *layout, uint64_t layer,
                         uint64_t tensor, uint64_t slot, const sgl_kv_device_buffer *other,
                         uint64_t other_offset, hipStream_t stream, bool to_pool) {
    int32_t rc = validate_layout(s, layout);
    if (rc) return rc;
    if (!other) return null_arg(to_pool ? "source" : "destination");
    uint64_t start, end;
    if ((rc = sgl_kv_paged_layout_tensor_slot_byte_range(layout, layer, tensor, slot, &start, &end))) return rc;
    const uint64_t len = end - start;
    const char *name = to_pool ? "source" : "destination";
    if ((rc = same_device(s, name, *other))) return rc;
    uint64_t addr = 0;
    if ((rc = buffer_range(name, *other, other_offset, len, &addr))) return rc;
    if (len == 0) return ok();
    DeviceScope scope(s->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    uint8_t *pool = static_cast<uint8_t *>(s->base) + start;
    void *buf = reinterpret_cast<void *>(addr);
    SGLKV_CHECK_HIP(hipMemcpyAsync(to_pool ? (void *)pool : buf, to_pool ? buf : (void *)pool, len,
                                   hipMemcpyDeviceToDevice, stream));
    return ok();
}

int32_t location(const sgl_rocm_kv_storage *s, uint64_t start, uint64_t end, sgl_kv_tensor_location *out) {
    out->byte_offset = start;
    out->byte_len = end - start;
    out->device_ptr = (uint64_t)(uintptr_t)s->base + start;
    return ok();
}

// CudaKvStorage::validate_slot_map (cuda_kv_cache.rs:407-421).
int32_t validate_slot_map(const sgl_rocm_kv_storage *s, const sgl_kv_paged_layout *layout,
                          const sgl_rocm_kv_slot_map *map) {
    int32_t rc = validate_layout(s, layout);
    if (rc) return rc;
    if (!map) return null_arg("slot_map");
    if (map->slot_count != layout->slot_count)
        return fail(SGL_KV_STORAGE_SLOT_MAP_CAPACITY_MISMATCH, nullptr, map->slot_count, layout->slot_count, 0,
                    "ROCm KV slot map was validated for %llu slots but layout contains %llu slots",
                    (unsigned long long)map->slot_count, (unsigned long long)layout->slot_count);
    return sgl_kv_paged_layout_validate_slot_indices(layout, map->slots.data(), map->slots.size());
}

// write_kv_slots_from_device / read_kv_slots_to_device (cuda_kv_cache.rs:296-374)
// with kv_pair_copy_plan (:510-532).
int32_t kv_slots(sgl_rocm_kv_ctx *ctx, const sgl_rocm_kv_storage *s, const sgl_kv_paged_layout *layout,
                 uint64_t layer, const sgl_rocm_kv_slot_map *map, const sgl_kv_slot_rows *rows,
                 hipStream_t stream, bool scatter) {
    if (!ctx) return null_arg("ctx");
    if (!rows) return null_arg("rows");
    int32_t rc = validate_slot_map(s, layout, map);
    if (rc) return rc;
    sgl_kv_pair_copy_layout geometry;
    if ((rc = sgl_kv_paged_layout_kv_pair_copy_geometry(layout, layer, &geometry))) return rc;
    sgl_kv_pair_copy_plan plan;
    if ((rc = sgl_kv_pair_copy_plan_new(map->slots.size(), layout->slot_count, &geometry,
                                        rows->key_row_stride_bytes, rows->value_row_stride_bytes, &plan)))
        return rc;
    sgl_kv_pair_copy_buffers b;
    memset(&b, 0, sizeof b);
    b.keys = rows->keys;
    b.keys_offset = rows->keys_offset;
    b.values = rows->values;
    b.values_offset = rows->values_offset;
    b.slot_indices = sgl_kv_device_buffer{map->base, map->slots.size() * sizeof(uint64_t)};
    b.pool = sgl_kv_device_buffer{s->base, s->byte_len};
    return scatter ? sgl_rocm_kv_pair_scatter(ctx, &plan, &b, stream)
                   : sgl_rocm_kv_pair_gather(ctx, &plan, &b, stream);
}

int32_t descriptor_error(const char *what, uint64_t a, uint64_t b, const char *message) {
    return fail(SGL_KV_STORAGE_DESCRIPTOR, what, a, b, 0, "invalid KV memory descriptor: %s", message);
}

}  // namespace

extern "C" int32_t sgl_rocm_kv_memory_info(const sgl_rocm_kv_ctx *ctx, uint64_t *free_bytes,
                                           uint64_t *total_bytes) {
    if (!ctx) return null_arg("ctx");
    if (!free_bytes || !total_bytes) return null_arg("free_bytes/total_bytes");
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    size_t f = 0, t = 0;
    SGLKV_CHECK_HIP(hipMemGetInfo(&f, &t));
    *free_bytes = f;
    *total_bytes = t;
    return ok();
}

extern "C" int32_t sgl_rocm_kv_storage_allocate(sgl_rocm_kv_ctx *ctx, uint64_t byte_len,
                                                uint64_t page_size_bytes, sgl_rocm_kv_storage **out) {
    return allocate(ctx, byte_len, page_size_bytes, out);
}

extern "C" int32_t sgl_rocm_kv_cache_allocate(sgl_rocm_kv_ctx *ctx, const sgl_kv_runtime_layout *runtime,
                                              uint64_t page_count, sgl_kv_paged_layout *layout,
                                              sgl_rocm_kv_storage **out) {
    if (!out) return null_arg("out");
    *out = nullptr;
    if (!ctx) return null_arg("ctx");
    if (!runtime || !layout) return null_arg("runtime/layout");
    sgl_kv_paged_layout l;
    int32_t rc = sgl_kv_paged_layout_new(runtime, page_count, &l);
    if (rc) return rc;
    if ((rc = allocate(ctx, l.total_byte_len, l.runtime.page_size_bytes, out))) return rc;
    *layout = l;
    return ok();
}

extern "C" int32_t sgl_rocm_kv_pool_allocate(sgl_rocm_kv_ctx *ctx, const sgl_kv_paged_layout *layout,
                                             sgl_rocm_kv_storage **out) {
    if (!out) return null_arg("out");
    *out = nullptr;
    if (!ctx) return null_arg("ctx");
    if (!layout) return null_arg("layout");
    sgl_rocm_kv_storage *s = nullptr;
    int32_t rc = allocate(ctx, layout->total_byte_len, layout->runtime.page_size_bytes, &s);
    if (rc) return rc;
    // KvCachePool::new (kv_cache.rs:849-856).
    if (s->byte_len != layout->total_byte_len) {
        rc = size_mismatch("pool", layout->total_byte_len, s->byte_len);
        (void)sgl_rocm_kv_storage_destroy(s);
        return rc;
    }
    *out = s;
    return ok();
}

namespace {

constexpr uint64_t kProbeMaxRows = 131072;
constexpr int kProbeTimed = 5;

uint64_t gcd64(uint64_t a, uint64_t b) {
    while (b) {
        const uint64_t t = a % b;
        a = b;
        b = t;
    }
    return a;
}

// The probe's slot map: rows r of a fixed permutation of the pool's pages,
// r % page_size within its page, the way a decode page table spreads a
// request over the pool. The permutation is affine (i -> (a i + c) mod
// pages with a coprime to pages), so nothing proportional to the page count
// is built.
std::vector<uint64_t> probe_slots(uint64_t rows, uint64_t page_size, uint64_t pages) {
    uint64_t a = 0x9E3779B97F4A7C15ull % pages;
    if (a == 0) a = 1;
    while (gcd64(a, pages) != 1) a = a + 1 < pages ? a + 1 : 1;
    const uint64_t c = pages / 3;
    std::vector<uint64_t> slots(rows);
    for (uint64_t r = 0; r < rows; ++r) {
        const uint64_t i = r / page_size;
        const uint64_t page = (uint64_t)(((unsigned __int128)a * i + c) % pages);
        slots[r] = page * page_size + r % page_size;
    }
    return slots;
}

// Frees every candidate but `keep` (-1: all of them).
void free_candidates(std::vector<void *> &bases, int keep) {
    for (size_t i = 0; i < bases.size(); ++i)
        if ((int)i != keep && bases[i]) (void)hipFree(bases[i]);
}

}  // namespace

extern "C" int32_t sgl_rocm_kv_storage_allocate_placed(sgl_rocm_kv_ctx *ctx, uint64_t byte_len,
                                                       uint64_t page_size_bytes, const sgl_kv_pool_view *probe_view,
                                                       const sgl_kv_device_buffer *probe_rows,
                                                       const sgl_kv_pool_view *probe_source, uint32_t candidates,
                                                       void *stream, sgl_rocm_kv_storage **out,
                                                       sgl_kv_placement_report *report) {
    if (!out) return null_arg("out");
    *out = nullptr;
    if (!ctx) return null_arg("ctx");
    if (!probe_view) return null_arg("probe_view");
    if (!probe_source && (!probe_rows || !probe_rows->ptr)) return null_arg("probe_rows");
    if (candidates < 1 || candidates > SGL_KV_PLACEMENT_MAX_CANDIDATES)
        return fail(SGL_KV_INVALID_ARGUMENT, "candidates", candidates, SGL_KV_PLACEMENT_MAX_CANDIDATES, 0,
                    "placement candidates must be 1..%u, got %u", SGL_KV_PLACEMENT_MAX_CANDIDATES, candidates);
    if (byte_len == 0)
        return fail(SGL_KV_ZERO_ALLOCATION, nullptr, 0, 0, 0, "ROCm allocation of zero bytes");
    const sgl_kv_pool_view &v = *probe_view;
    for (const sgl_kv_pool_view *w : {probe_view, probe_source}) {
        if (!w) continue;
        if (w->tensor_count < 1 || w->tensor_count > 2)
            return fail(SGL_KV_INVALID_ARGUMENT, "tensor_count", w->tensor_count, 2, 0,
                        "probe view tensor_count must be 1 or 2, got %u", w->tensor_count);
        if (w->page_size == 0 || w->page_count == 0)
            return fail(SGL_KV_INVALID_ARGUMENT, "page_size/page_count", w->page_size, w->page_count, 0,
                        "probe view has no slots");
    }
    auto slot_count = [](const sgl_kv_pool_view &w) {
        uint64_t n;
        return __builtin_mul_overflow(w.page_size, w.page_count, &n) ? UINT64_MAX : n;
    };
    const uint64_t rb0 = v.row_bytes;
    const uint64_t rb1 = v.tensor_count == 2 ? (v.value_row_bytes ? v.value_row_bytes : v.row_bytes) : 0;
    const uint64_t token_bytes = rb0 + rb1;
    uint64_t rows = slot_count(v);
    if (probe_source) {
        rows = std::min(rows, slot_count(*probe_source));
    } else {
        rows = std::min(rows, token_bytes ? probe_rows->byte_len / token_bytes : 0);
        if (rows == 0)
            return fail(SGL_KV_INVALID_ARGUMENT, "probe_rows", probe_rows->byte_len, token_bytes, 0,
                        "probe rows of %llu bytes hold no row of %llu bytes",
                        (unsigned long long)probe_rows->byte_len, (unsigned long long)token_bytes);
    }
    rows = std::min(rows, kProbeMaxRows);

    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    if (!probe_source) {
        // The probe's kernels read and write probe_rows: it must be memory
        // of the context's device.
        const sgl_rocm_kv_storage probe_owner{ctx->device, nullptr, 0, 0};
        const int32_t rc = same_device(&probe_owner, "probe_rows", *probe_rows);
        if (rc) return rc;
    }
    hipStream_t s = static_cast<hipStream_t>(stream);

    // All candidates are held at once: a freed allocation would come back at
    // the same physical memory.
    std::vector<void *> bases;
    for (uint32_t i = 0; i < candidates; ++i) {
        void *base = nullptr;
        const hipError_t err = hipMalloc(&base, byte_len);
        if (err != hipSuccess) {
            (void)hipGetLastError();
            if (i == 0) return hip_fail(err, "hipMalloc");
            break;  // probe what fits
        }
        bases.push_back(base);
    }

    // Slot maps: the candidate's rows at [0, rows), the source's (pool to
    // pool) at [rows, 2 rows).
    std::vector<uint64_t> host_slots = probe_slots(rows, v.page_size, v.page_count);
    if (probe_source) {
        const std::vector<uint64_t> src = probe_slots(rows, probe_source->page_size, probe_source->page_count);
        host_slots.insert(host_slots.end(), src.begin(), src.end());
    }
    void *slot_dev = nullptr;
    hipEvent_t ev[kProbeTimed + 1] = {};
    int32_t rc = SGL_KV_OK;
    std::vector<float> probe_us(bases.size(), 0.0f);
    auto cleanup = [&](int keep) {
        // Nothing may still be writing a candidate when it is freed.
        (void)hipStreamSynchronize(s);
        for (hipEvent_t &e : ev)
            if (e) (void)hipEventDestroy(e);
        if (slot_dev) (void)hipFree(slot_dev);
        free_candidates(bases, keep);
    };
    hipError_t err = hipMalloc(&slot_dev, host_slots.size() * sizeof(uint64_t));
    if (err == hipSuccess)
        err = hipMemcpy(slot_dev, host_slots.data(), host_slots.size() * sizeof(uint64_t), hipMemcpyHostToDevice);
    for (int i = 0; err == hipSuccess && i <= kProbeTimed; ++i) err = hipEventCreate(&ev[i]);
    if (err != hipSuccess) {
        cleanup(-1);
        return hip_fail(err, "probe set-up");
    }
    const sgl_kv_device_buffer slots{slot_dev, rows * sizeof(uint64_t)};
    const sgl_kv_device_buffer src_slots{static_cast<uint64_t *>(slot_dev) + rows, rows * sizeof(uint64_t)};
    sgl_kv_rows_view rv;
    memset(&rv, 0, sizeof rv);
    if (!probe_source) {
        uint8_t *p = static_cast<uint8_t *>(probe_rows->ptr);
        rv.planes[0] = p;
        rv.plane_bytes[0] = rows * rb0;
        rv.row_stride[0] = rb0;
        if (v.tensor_count == 2) {
            rv.planes[1] = p + rows * rb0;
            rv.plane_bytes[1] = rows * rb1;
            rv.row_stride[1] = rb1;
        }
    }
    sgl_kv_pool_view sv;
    if (probe_source) {
        sv = *probe_source;
        sv.scale = nullptr;
    }
    for (size_t c = 0; c < bases.size() && rc == SGL_KV_OK; ++c) {
        sgl_kv_pool_view pv = v;
        pv.base = bases[c];
        pv.byte_len = byte_len;
        pv.scale = nullptr;  // the probe moves bytes only
        // Rows mode: each round packs the candidate's rows into probe_rows
        // and unpacks them back, so that the timed unpack reads rows just
        // written, as one that follows a transfer's pack or receive does;
        // only the unpack is timed. Pool-to-pool mode: each round is one
        // timed transfer from the source pool into the candidate.
        auto prepare = [&]() {
            return probe_source ? SGL_KV_OK : sgl_rocm_kv_pack_layer(ctx, &pv, &slots, rows, &rv, s);
        };
        auto timed = [&]() {
            return probe_source ? sgl_rocm_kv_transfer_layer(ctx, &sv, &src_slots, rows, &pv, &slots, s)
                                : sgl_rocm_kv_unpack_layer(ctx, &rv, rows, &pv, &slots, s);
        };
        rc = prepare();  // warm-up round
        if (rc == SGL_KV_OK) rc = timed();
        float t[kProbeTimed];
        for (int i = 0; i < kProbeTimed && rc == SGL_KV_OK; ++i) {
            if ((rc = prepare()) != SGL_KV_OK) break;
            if ((err = hipEventRecord(ev[i], s)) != hipSuccess) break;
            rc = timed();
            if (rc == SGL_KV_OK && (err = hipEventRecord(ev[i + 1], s)) != hipSuccess) break;
            if (rc == SGL_KV_OK && (err = hipEventSynchronize(ev[i + 1])) != hipSuccess) break;
            if (rc == SGL_KV_OK && (err = hipEventElapsedTime(&t[i], ev[i], ev[i + 1])) != hipSuccess) break;
        }
        if (rc == SGL_KV_OK && err != hipSuccess) rc = hip_fail(err, "probe timing");
        if (rc != SGL_KV_OK) break;
        std::sort(t, t + kProbeTimed);
        probe_us[c] = t[kProbeTimed / 2] * 1000.0f;
    }
    if (rc == SGL_KV_OK && (err = hipStreamSynchronize(s)) != hipSuccess) rc = hip_fail(err, "hipStreamSynchronize");
    if (rc != SGL_KV_OK) {
        cleanup(-1);
        return rc;
    }
    size_t best = 0;
    for (size_t c = 1; c < bases.size(); ++c)
        if (probe_us[c] < probe_us[best]) best = c;
    void *base = bases[best];
    cleanup((int)best);
    err = hipMemsetAsync(base, 0, byte_len, nullptr);
    if (err == hipSuccess) err = hipStreamSynchronize(nullptr);
    if (err != hipSuccess) {
        (void)hipFree(base);
        return hip_fail(err, "hipMemsetAsync");
    }
    if (report) {
        memset(report, 0, sizeof *report);
        report->candidates = (uint32_t)bases.size();
        report->chosen = (uint32_t)best;
        report->probe_rows = rows;
        for (size_t c = 0; c < bases.size(); ++c) report->probe_us[c] = probe_us[c];
    }
    *out = new sgl_rocm_kv_storage{ctx->device, base, byte_len, page_size_bytes};
    return ok();
}

extern "C" int32_t sgl_rocm_kv_storage_destroy(sgl_rocm_kv_storage *storage) {
    if (!storage) return ok();
    DeviceScope scope(storage->device);
    const hipError_t err = hipFree(storage->base);
    delete storage;
    if (err != hipSuccess) return hip_fail(err, "hipFree");
    return ok();
}

extern "C" int32_t sgl_rocm_kv_storage_allocation(const sgl_rocm_kv_storage *storage, sgl_kv_device_buffer *out) {
    if (!storage) return null_arg("storage");
    if (!out) return null_arg("out");
    out->ptr = storage->base;
    out->byte_len = storage->byte_len;
    return ok();
}

extern "C" uint64_t sgl_rocm_kv_storage_byte_len(const sgl_rocm_kv_storage *storage) {
    return storage ? storage->byte_len : 0;
}

extern "C" uint64_t sgl_rocm_kv_storage_page_size_bytes(const sgl_rocm_kv_storage *storage) {
    return storage ? storage->page_size_bytes : 0;
}

extern "C" int32_t sgl_rocm_kv_storage_device(const sgl_rocm_kv_storage *storage) {
    return storage ? storage->device : -1;
}

extern "C" int32_t sgl_rocm_kv_storage_clear(sgl_rocm_kv_storage *storage) {
    if (!storage) return null_arg("storage");
    DeviceScope scope(storage->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    SGLKV_CHECK_HIP(hipMemsetAsync(storage->base, 0, storage->byte_len, nullptr));
    SGLKV_CHECK_HIP(hipStreamSynchronize(nullptr));
    return ok();
}

extern "C" int32_t sgl_rocm_kv_storage_validate_layout(const sgl_rocm_kv_storage *storage,
                                                       const sgl_kv_paged_layout *layout) {
    const int32_t rc = validate_layout(storage, layout);
    return rc ? rc : ok();
}

// CudaKvStorage::write_page / read_page (cuda_kv_cache.rs:224-256).
extern "C" int32_t sgl_rocm_kv_storage_write_page(sgl_rocm_kv_storage *storage, const sgl_kv_paged_layout *layout,
                                                  uint64_t page_index, const void *bytes, uint64_t len) {
    int32_t rc = validate_layout(storage, layout);
    if (rc) return rc;
    if (len != layout->runtime.page_size_bytes) return page_buffer_mismatch(layout->runtime.page_size_bytes, len, true);
    uint64_t start, end;
    if ((rc = sgl_kv_paged_layout_page_byte_range(layout, page_index, &start, &end))) return rc;
    if (len && !bytes) return null_arg("bytes");
    if (len == 0) return ok();
    DeviceScope scope(storage->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    SGLKV_CHECK_HIP(hipMemcpy(static_cast<uint8_t *>(storage->base) + start, bytes, len, hipMemcpyHostToDevice));
    return ok();
}

extern "C" int32_t sgl_rocm_kv_storage_read_page(const sgl_rocm_kv_storage *storage, const sgl_kv_paged_layout *layout,
                                                 uint64_t page_index, void *bytes, uint64_t len) {
    int32_t rc = validate_layout(storage, layout);
    if (rc) return rc;
    if (len != layout->runtime.page_size_bytes) return page_buffer_mismatch(layout->runtime.page_size_bytes, len, true);
    uint64_t start, end;
    if ((rc = sgl_kv_paged_layout_page_byte_range(layout, page_index, &start, &end))) return rc;
    if (len && !bytes) return null_arg("bytes");
    if (len == 0) return ok();
    DeviceScope scope(storage->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    SGLKV_CHECK_HIP(hipMemcpy(bytes, static_cast<const uint8_t *>(storage->base) + start, len, hipMemcpyDeviceToHost));
    return ok();
}

extern "C" int32_t sgl_rocm_kv_storage_write_tensor_slot(sgl_rocm_kv_storage *storage,
                                                         const sgl_kv_paged_layout *layout, uint64_t layer,
                                                         uint64_t tensor, uint64_t slot,
                                                         const sgl_kv_device_buffer *source,
                                                         uint64_t source_offset, void *stream) {
    return tensor_slot_copy(storage, layout, layer, tensor, slot, source, source_offset,
                            static_cast<hipStream_t>(stream), true);
}

extern "C" int32_t sgl_rocm_kv_storage_read_tensor_slot(const sgl_rocm_kv_storage *storage,
                                                        const sgl_kv_paged_layout *layout, uint64_t layer,
                                                        uint64_t tensor, uint64_t slot,
                                                        const sgl_kv_device_buffer *destination,
                                                        uint64_t destination_offset, void *stream) {
    return tensor_slot_copy(storage, layout, layer, tensor, slot, destination, destination_offset,
                            static_cast<hipStream_t>(stream), false);
}

// CudaKvStorage::tensor_location / slot_location (cuda_kv_cache.rs:376-403).
extern "C" int32_t sgl_rocm_kv_storage_tensor_location(const sgl_rocm_kv_storage *storage,
                                                       const sgl_kv_paged_layout *layout, uint64_t page_index,
                                                       uint64_t layer, uint64_t tensor, uint64_t token,
                                                       sgl_kv_tensor_location *out) {
    int32_t rc = validate_layout(storage, layout);
    if (rc) return rc;
    if (!out) return null_arg("out");
    uint64_t start, end;
    if ((rc = sgl_kv_paged_layout_tensor_token_byte_range(layout, page_index, layer, tensor, token, &start, &end)))
        return rc;
    return location(storage, start, end, out);
}

extern "C" int32_t sgl_rocm_kv_storage_slot_location(const sgl_rocm_kv_storage *storage,
                                                     const sgl_kv_paged_layout *layout, uint64_t layer,
                                                     uint64_t tensor, uint64_t slot, sgl_kv_tensor_location *out) {
    int32_t rc = validate_layout(storage, layout);
    if (rc) return rc;
    if (!out) return null_arg("out");
    uint64_t start, end;
    if ((rc = sgl_kv_paged_layout_tensor_slot_byte_range(layout, layer, tensor, slot, &start, &end))) return rc;
    return location(storage, start, end, out);
}

// CudaKvStorage::upload_slot_map (cuda_kv_cache.rs:199-222).
extern "C" int32_t sgl_rocm_kv_storage_upload_slot_map(const sgl_rocm_kv_storage *storage,
                                                       const sgl_kv_paged_layout *layout, const uint64_t *slots,
                                                       uint64_t slot_len, sgl_rocm_kv_slot_map **out) {
    if (!out) return null_arg("out");
    *out = nullptr;
    int32_t rc = validate_layout(storage, layout);
    if (rc) return rc;
    if ((rc = sgl_kv_paged_layout_validate_slot_indices(layout, slots, slot_len))) return rc;
    uint64_t bytes;
    if (mul_ovf(slot_len, sizeof(uint64_t), &bytes))
        return fail(SGL_KV_STORAGE_SIZE_OVERFLOW, nullptr, 0, 0, 0, "ROCm KV storage size overflowed");
    DeviceScope scope(storage->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    void *base = nullptr;
    SGLKV_CHECK_HIP(hipMalloc(&base, bytes));
    const hipError_t err = hipMemcpy(base, slots, bytes, hipMemcpyHostToDevice);
    if (err != hipSuccess) {
        (void)hipFree(base);
        return hip_fail(err, "hipMemcpy");
    }
    *out = new sgl_rocm_kv_slot_map{storage->device, base, std::vector<uint64_t>(slots, slots + slot_len),
                                    layout->slot_count};
    return ok();
}

extern "C" int32_t sgl_rocm_kv_slot_map_destroy(sgl_rocm_kv_slot_map *map) {
    if (!map) return ok();
    DeviceScope scope(map->device);
    const hipError_t err = hipFree(map->base);
    delete map;
    if (err != hipSuccess) return hip_fail(err, "hipFree");
    return ok();
}

extern "C" int32_t sgl_rocm_kv_slot_map_allocation(const sgl_rocm_kv_slot_map *map, sgl_kv_device_buffer *out) {
    if (!map) return null_arg("slot_map");
    if (!out) return null_arg("out");
    out->ptr = map->base;
    out->byte_len = map->slots.size() * sizeof(uint64_t);
    return ok();
}

extern "C" uint64_t sgl_rocm_kv_slot_map_len(const sgl_rocm_kv_slot_map *map) {
    return map ? map->slots.size() : 0;
}

extern "C" const uint64_t *sgl_rocm_kv_slot_map_slots(const sgl_rocm_kv_slot_map *map) {
    return map ? map->slots.data() : nullptr;
}

extern "C" int32_t sgl_rocm_kv_storage_write_kv_slots(sgl_rocm_kv_ctx *ctx, sgl_rocm_kv_storage *storage,
                                                      const sgl_kv_paged_layout *layout, uint64_t layer,
                                                      const sgl_rocm_kv_slot_map *map, const sgl_kv_slot_rows *rows,
                                                      void *stream) {
    return kv_slots(ctx, storage, layout, layer, map, rows, static_cast<hipStream_t>(stream), true);
}

extern "C" int32_t sgl_rocm_kv_storage_read_kv_slots(sgl_rocm_kv_ctx *ctx, const sgl_rocm_kv_storage *storage,
                                                     const sgl_kv_paged_layout *layout, uint64_t layer,
                                                     const sgl_rocm_kv_slot_map *map, const sgl_kv_slot_rows *rows,
                                                     void *stream) {
    return kv_slots(ctx, storage, layout, layer, map, rows, static_cast<hipStream_t>(stream), false);
}

// impl KvCacheMemoryProvider for CudaKvStorage (cuda_kv_cache.rs:455-476),
// located on ROCm device `device`.
extern "C" int32_t sgl_rocm_kv_storage_transferable_memory(const sgl_rocm_kv_storage *storage,
                                                           sgl_kv_transferable_memory *out) {
    if (!storage) return null_arg("storage");
    if (!out) return null_arg("out");
    if (storage->page_size_bytes == 0) return descriptor_error("page_size_bytes", 0, 0, "zero page size");
    if (storage->byte_len % storage->page_size_bytes)
        return descriptor_error("region", storage->byte_len, storage->page_size_bytes,
                                "region length is not a whole number of pages");
    memset(out, 0, sizeof *out);
    out->regions[0].base_addr = (uint64_t)(uintptr_t)storage->base;
    out->regions[0].byte_len = storage->byte_len;
    out->regions[0].page_size_bytes = storage->page_size_bytes;
    out->region_count = 1;
    out->page_size_bytes = storage->page_size_bytes;
    out->location_kind = SGL_KV_LOCATION_ROCM;
    out->location_id = storage->device;
    return ok();
}

extern "C" int32_t sgl_rocm_kv_storage_backend_memory(const sgl_rocm_kv_storage *storage,
                                                      const sgl_kv_paged_layout *layout, uint32_t head_layout,
                                                      uint64_t heads, sgl_kv_backend_memory *out) {
    int32_t rc = validate_layout(storage, layout);
    if (rc) return rc;
    if (!out) return null_arg("out");
    if (head_layout != SGL_KV_NHD && head_layout != SGL_KV_HND)
        return fail(SGL_KV_INVALID_ARGUMENT, "head_layout", head_layout, 0, 0, "unknown head layout %u", head_layout);
    memset(out, 0, sizeof *out);
    out->layout = *layout;
    out->base = storage->base;
    out->byte_len = storage->byte_len;
    out->head_layout = head_layout;
    out->heads = heads;
    return ok();
}

// MooncakeMemoryLocationExt::mooncake_memory_location_label (transfer.rs:1662-1676).
extern "C" int32_t sgl_kv_memory_location_label(int32_t location_kind, int32_t location_id, char out[32]) {
    if (!out) return null_arg("out");
    out[0] = '\0';
    const char *prefix = nullptr;
    switch (location_kind) {
    case SGL_KV_LOCATION_CPU: prefix = "cpu"; break;
    case SGL_KV_LOCATION_CUDA: prefix = "cuda"; break;
    case SGL_KV_LOCATION_ROCM: prefix = "hip"; break;
    case SGL_KV_LOCATION_MUSA: prefix = "musa"; break;
    case SGL_KV_LOCATION_NPU: prefix = "npu"; break;
    case SGL_KV_LOCATION_METAL:
    case SGL_KV_LOCATION_XPU:
    case SGL_KV_LOCATION_HPU:
        return fail(SGL_KV_UNSUPPORTED_MEMORY_LOCATION, nullptr, (uint64_t)location_kind,
                    (uint64_t)(int64_t)location_id, 0, "mooncake transfer engine does not support KV memory location kind %d",
                    location_kind);
    default:
        return fail(SGL_KV_INVALID_ARGUMENT, "location_kind", (uint64_t)(int64_t)location_kind, 0, 0,
                    "unknown memory location kind %d", location_kind);
    }
    snprintf(out, 32, "%s:%d", prefix, location_id);
    return ok();
}

// MooncakeKvCacheMemoryExt::mooncake_decode_remote_layout (transfer.rs:1693-1703).
extern "C" int32_t sgl_kv_transferable_memory_decode_remote_layout(const sgl_kv_transferable_memory *memory,
                                                                   uint64_t *dst_kv_ptrs, uint64_t capacity,
                                                                   uint64_t *ptr_count, uint64_t *dst_kv_item_len) {
    if (!memory) return null_arg("memory");
    if (!ptr_count || !dst_kv_item_len) return null_arg("ptr_count/dst_kv_item_len");
    if (memory->region_count == 0 || memory->region_count > SGL_KV_MAX_MEMORY_REGIONS)
        return descriptor_error("region_count", memory->region_count, SGL_KV_MAX_MEMORY_REGIONS,
                                "the descriptor needs 1 to 8 regions");
    if (capacity < memory->region_count)
        return fail(SGL_KV_INVALID_ARGUMENT, "capacity", capacity, memory->region_count, 0,
                    "dst_kv_ptrs has room for %llu of %llu pointers", (unsigned long long)capacity,
                    (unsigned long long)memory->region_count);
    if (!dst_kv_ptrs) return null_arg("dst_kv_ptrs");
    for (uint64_t i = 0; i < memory->region_count; ++i) dst_kv_ptrs[i] = memory->regions[i].base_addr;
    *ptr_count = memory->region_count;
    *dst_kv_item_len = memory->page_size_bytes / memory->region_count;
    return ok();
}
