// kv_backend.cpp -- a KV transfer backend for prefill and decode pools on
// one MI355X: the ROCm counterpart of the reference's KvTransferBackend
// (crates/sglang-srt/src/transfer.rs:1145-1151) with register / submit /
// poll / cancel / shutdown. A submitted span (KvCacheTransferSpan,
// transfer.rs:495-505, plus the decode side's page table) is validated on
// the host, then moved asynchronously:
//   direct  one pool-to-pool launch over all layers (co-resident pools);
//   staged  the layer pipeline: pack -> pinned host -> unpack, the
//           single-GPU stand-in for the inter-node hop.
// poll reports each finished span once as a completion event carrying its
// bootstrap room and descriptor checksum, like the Mooncake executor's poll
// (transfer.rs:2633-2674). cancel drops a
// room's spans from the pending set without an event (transfer.rs:
// 2606-2631); their device work drains before its buffers are released.
#include <hip/hip_runtime.h>
#include <string.h>

#include <vector>

#include "kv_internal.h"

using namespace sglkv;

namespace {

// Device memory for one span's slot lists (source slots, then
// destination slots). Buffers are recycled, never freed before shutdown:
// hipFree waits for the device, and poll must not.
struct SlotBuffer {
    void *ptr;
    uint64_t bytes;
};

struct Transfer {
    uint64_t room;
    char checksum[65];
    bool canceled;
    hipEvent_t done;
    SlotBuffer slots;
    sgl_rocm_kv_pipeline *pipeline;    // staged mode
    int32_t word;                      // index of the span's error word (-1: none)
};

// Error words, one per span in flight: a span's kernels raise only its own
// word, so poll charges a device error to the span that hit it.
constexpr uint32_t kSpanWords = 1024;

}  // namespace

struct sgl_rocm_kv_backend {
    sgl_rocm_kv_ctx *ctx = nullptr;
    sgl_kv_backend_config config{};
    bool registered = false;
    sgl_kv_backend_memory memory[2];   // prefill, decode
    std::vector<sgl_kv_pool_view> views[2];
    uint64_t layer_stride[2] = {0, 0};
    hipStream_t stream = nullptr;      // direct launches
    hipStream_t side = nullptr;        // non-blocking: slot uploads, error-word reads
    uint32_t *flag_host = nullptr;     // pinned copy of an error word
    uint32_t *span_words = nullptr;    // device: kSpanWords error words
    std::vector<int32_t> free_words;
    void *staging_device = nullptr;    // staged: send[2] + recv[2]
    void *staging_host = nullptr;      // staged: host[2] (pinned)
    uint64_t layer_bytes = 0;
    hipEvent_t last_done = nullptr;    // staged: the previous span's completion
    std::vector<Transfer> inflight;
    std::vector<SlotBuffer> free_slots;
};

namespace {

// Releases a finished span's resources; its slot buffer goes back to the
// free list.
void release_transfer(sgl_rocm_kv_backend *b, Transfer &t) {
    if (t.pipeline) sgl_rocm_kv_pipeline_destroy(t.pipeline);
    if (t.slots.ptr) b->free_slots.push_back(t.slots);
    if (t.done) (void)hipEventDestroy(t.done);
    if (b->last_done == t.done) b->last_done = nullptr;
    if (t.word >= 0) b->free_words.push_back(t.word);
    t.pipeline = nullptr;
    t.slots = SlotBuffer{nullptr, 0};
    t.done = nullptr;
    t.word = -1;
}

// A free slot buffer of at least `bytes` (the smallest that fits), or a new one.
int32_t take_slot_buffer(sgl_rocm_kv_backend *b, uint64_t bytes, SlotBuffer *out) {
    size_t best = b->free_slots.size();
    for (size_t i = 0; i < b->free_slots.size(); ++i)
        if (b->free_slots[i].bytes >= bytes &&
            (best == b->free_slots.size() || b->free_slots[i].bytes < b->free_slots[best].bytes))
            best = i;
    if (best < b->free_slots.size()) {
        *out = b->free_slots[best];
        b->free_slots.erase(b->free_slots.begin() + best);
        return SGL_KV_OK;
    }
    void *ptr = nullptr;
    SGLKV_CHECK_HIP(hipMalloc(&ptr, bytes));
    *out = SlotBuffer{ptr, bytes};
    return SGL_KV_OK;
}

void release_staging(sgl_rocm_kv_backend *b) {
    if (b->staging_device) (void)hipFree(b->staging_device);
    if (b->staging_host) (void)hipHostFree(b->staging_host);
    b->staging_device = b->staging_host = nullptr;
}

// Reads a finished span's error word without waiting for work queued on
// other streams. Only that span's kernels raise the word and they have all
// finished (its completion event fired), so the read is final; the word is
// cleared again when a later span takes it.
int32_t read_span_errors(sgl_rocm_kv_backend *b, const Transfer &t, uint32_t *flag) {
    *flag = 0;
    if (t.word < 0) return SGL_KV_OK;
    SGLKV_CHECK_HIP(hipMemcpyAsync(b->flag_host, b->span_words + t.word, sizeof(uint32_t),
                                   hipMemcpyDeviceToHost, b->side));
    SGLKV_CHECK_HIP(hipStreamSynchronize(b->side));
    *flag = *b->flag_host;
    return SGL_KV_OK;
}

int32_t check_backend(const sgl_rocm_kv_backend *b) {
    if (!b) return fail(SGL_KV_INVALID_ARGUMENT, "backend", 0, 0, 0, "null backend");
    return SGL_KV_OK;
}

}  // namespace

extern "C" int32_t sgl_rocm_kv_backend_create(sgl_rocm_kv_ctx *ctx, const sgl_kv_backend_config *config,
                                              sgl_rocm_kv_backend **out) {
    if (!ctx || !config || !out)
        return fail(SGL_KV_INVALID_ARGUMENT, "ctx/config/out", 0, 0, 0, "null argument");
    *out = nullptr;
    if (config->mode > SGL_KV_BACKEND_STAGED)
        return fail(SGL_KV_INVALID_ARGUMENT, "mode", config->mode, 0, 0, "unknown backend mode %u",
                    config->mode);
    if (config->max_rows == 0 || config->max_rows > UINT32_MAX)
        return fail(SGL_KV_INVALID_ARGUMENT, "max_rows", config->max_rows, UINT32_MAX, 0,
                    "max_rows must be in [1, 2^32)");
    sgl_rocm_kv_backend *b = new sgl_rocm_kv_backend();
    b->ctx = ctx;
    b->config = *config;
    DeviceScope scope(ctx->device);
    hipError_t err = scope.status();
    if (err == hipSuccess) err = hipStreamCreate(&b->stream);
    if (err == hipSuccess) err = hipStreamCreateWithFlags(&b->side, hipStreamNonBlocking);
    if (err == hipSuccess) err = hipHostMalloc((void **)&b->flag_host, sizeof(uint32_t), 0);
    if (err == hipSuccess) err = hipMalloc((void **)&b->span_words, kSpanWords * sizeof(uint32_t));
    if (err == hipSuccess) err = hipMemset(b->span_words, 0, kSpanWords * sizeof(uint32_t));
    if (err != hipSuccess) {
        if (b->stream) (void)hipStreamDestroy(b->stream);
        if (b->side) (void)hipStreamDestroy(b->side);
        if (b->flag_host) (void)hipHostFree(b->flag_host);
        if (b->span_words) (void)hipFree(b->span_words);
        delete b;
        return hip_fail(err, "sgl_rocm_kv_backend_create");
    }
    for (uint32_t w = kSpanWords; w-- > 0;) b->free_words.push_back((int32_t)w);
    *out = b;
    return ok();
}

// KvTransferBackend::register: the prefill and decode pools (both on this
// backend's device). Their rows must agree: layers, tensors per token and
// bytes per (token, layer, tensor).
extern "C" int32_t sgl_rocm_kv_backend_register(sgl_rocm_kv_backend *b,
                                                const sgl_kv_backend_memory *prefill,
                                                const sgl_kv_backend_memory *decode) {
    int32_t rc = check_backend(b);
    if (rc) return rc;
    if (!prefill || !decode) return fail(SGL_KV_INVALID_ARGUMENT, "memory", 0, 0, 0, "null memory");
    if (b->registered) return fail(SGL_KV_INVALID_ARGUMENT, "register", 0, 0, 0, "memory is already registered");
    const sgl_kv_backend_memory *m[2] = {prefill, decode};
    const sgl_kv_runtime_layout &r0 = prefill->layout.runtime, &r1 = decode->layout.runtime;
    if (r0.num_layers != r1.num_layers || r0.kv_tensors_per_token != r1.kv_tensors_per_token ||
        prefill->layout.token_bytes[0] != decode->layout.token_bytes[0] ||
        prefill->layout.token_bytes[1] != decode->layout.token_bytes[1])
        return fail(SGL_KV_INVALID_ARGUMENT, "decode", r1.num_layers, r0.num_layers, 0,
                    "prefill and decode pools hold different rows (layers %llu vs %llu)",
                    (unsigned long long)r0.num_layers, (unsigned long long)r1.num_layers);
    static const char *const side_names[2] = {"prefill", "decode"};
    for (int side = 0; side < 2; ++side) {
        if (!m[side]->base)
            return fail(SGL_KV_INVALID_ARGUMENT, side_names[side], 0, 0, 0, "null %s pool",
                        side_names[side]);
        if (m[side]->byte_len < m[side]->layout.total_byte_len)
            return fail(SGL_KV_ALLOCATION_OUT_OF_BOUNDS, side_names[side], 0,
                        m[side]->layout.total_byte_len, m[side]->byte_len,
                        "the %s pool's %llu bytes hold less than its layout's %llu",
                        side_names[side], (unsigned long long)m[side]->byte_len,
                        (unsigned long long)m[side]->layout.total_byte_len);
    }
    // One view per layer carries both tensors (of unequal widths for the
    // MLA tensor pair); layouts of more tensors are not moved partially.
    if (r0.kv_tensors_per_token > 2)
        return fail(SGL_KV_INVALID_ARGUMENT, "kv_tensors_per_token", r0.kv_tensors_per_token, 2, 0,
                    "the transfer backend moves layouts of one or two tensors per token, not %llu",
                    (unsigned long long)r0.kv_tensors_per_token);
    const uint64_t tensors = r0.kv_tensors_per_token;
    std::vector<sgl_kv_pool_view> views[2];
    for (int side = 0; side < 2; ++side) {
        const uint64_t heads = m[side]->heads ? m[side]->heads : m[side]->layout.runtime.kv_heads;
        views[side].resize(r0.num_layers);
        for (uint64_t l = 0; l < r0.num_layers; ++l)
            if ((rc = sgl_kv_pool_view_for_layer(&m[side]->layout, m[side]->base, m[side]->byte_len,
                                                 m[side]->head_layout, heads, l, 0, tensors,
                                                 &views[side][l])))
                return rc;
    }
    uint64_t row_bytes = views[0][0].row_bytes + (tensors == 2 ? view_row_bytes(views[0][0], 1) : 0);
    if (mul_ovf(b->config.max_rows, row_bytes, &b->layer_bytes))
        return fail(SGL_KV_SHAPE_OVERFLOW, nullptr, 0, 0, 0, "KV copy tensor shape overflowed");
    if (b->config.mode == SGL_KV_BACKEND_STAGED) {
        DeviceScope scope(b->ctx->device);
        hipError_t err = scope.status();
        if (err == hipSuccess) err = hipMalloc(&b->staging_device, 4 * b->layer_bytes);
        if (err == hipSuccess) err = hipHostMalloc(&b->staging_host, 2 * b->layer_bytes, 0);
        if (err != hipSuccess) {
            release_staging(b);
            return hip_fail(err, "sgl_rocm_kv_backend_register");
        }
    }
    for (int side = 0; side < 2; ++side) {
        b->memory[side] = *m[side];
        b->views[side] = views[side];
        b->layer_stride[side] = m[side]->layout.bytes_per_layer_page;
    }
    b->registered = true;
    return ok();
}

namespace {

// KvTransferBackend::submit. With `device_table`, span->dst_page_table is a
// device pointer and the decode slots are resolved on the device into the
// span's slot buffer; otherwise the table is a host array, checked entry by
// entry here.
int32_t submit_span(sgl_rocm_kv_backend *b, const sgl_kv_transfer_span_desc *span, bool device_table) {
    int32_t rc = check_backend(b);
    if (rc) return rc;
    if (!span) return fail(SGL_KV_INVALID_ARGUMENT, "span", 0, 0, 0, "null span");
    if (!b->registered) return fail(SGL_KV_INVALID_ARGUMENT, "register", 0, 0, 0, "no memory is registered");
    const uint64_t n = span->token_count;
    if (n > b->config.max_rows) return too_large_rows(n, b->config.max_rows);
    if (b->free_words.empty())
        return fail(SGL_KV_DIMENSION_TOO_LARGE, "spans in flight", kSpanWords + 1, kSpanWords, 0,
                    "more than %u spans in flight: poll before submitting more", kSpanWords);
    Transfer t;
    memset(&t, 0, sizeof t);
    t.word = -1;
    t.room = span->bootstrap_room;
    memcpy(t.checksum, span->descriptor_checksum, 64);
    t.checksum[64] = '\0';
    DeviceScope scope(b->ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    if (n == 0) {  // a no-op span completes at once
        SGLKV_CHECK_HIP(hipEventCreateWithFlags(&t.done, hipEventDisableTiming));
        SGLKV_CHECK_HIP(hipEventRecord(t.done, b->stream));
        b->inflight.push_back(t);
        return ok();
    }
    if (!span->cache_slots || !span->dst_page_table)
        return fail(SGL_KV_INVALID_ARGUMENT, "cache_slots/dst_page_table", 0, 0, 0, "null argument");
    if (device_table) {
        uint64_t table_bytes;
        if (mul_ovf(span->dst_page_table_len, sizeof(int32_t), &table_bytes))
            return fail(SGL_KV_SHAPE_OVERFLOW, nullptr, 0, 0, 0, "KV copy tensor shape overflowed");
        const sgl_kv_device_buffer table{const_cast<int32_t *>(span->dst_page_table), table_bytes};
        if ((rc = check_device(b->ctx, "dst_page_table", table))) return rc;
    }
    // Prefill slots: PagedKvCacheLayout::validate_slot_indices (kv_cache.rs:722-736).
    if ((rc = sgl_kv_paged_layout_validate_slot_indices(&b->memory[0].layout, span->cache_slots, n)))
        return rc;
    // Decode slots from the decode page table: token k of the request is in
    // page dst_page_table[k / page_size] at position k % page_size.
    const sgl_kv_paged_layout &dl = b->memory[1].layout;
    const uint64_t P = dl.runtime.page_size;
    if (device_table && (P > UINT32_MAX || span->token_offset + n > UINT32_MAX))
        return too_large_dim("token_offset + token_count", span->token_offset + n, UINT32_MAX);
    // The upload holds the prefill slots, then (host table) the decode
    // slots, or (device table) the one span the resolve kernel reads.
    std::vector<uint64_t> upload(2 * n + (device_table ? 2 : 0));
    memcpy(upload.data(), span->cache_slots, n * sizeof(uint64_t));
    if (device_table) {
        const sgl_kv_span one{0, (uint32_t)span->token_offset, (uint32_t)n, 0};
        memcpy(&upload[2 * n], &one, sizeof one);
    } else {
        for (uint64_t i = 0; i < n; ++i) {
            const uint64_t token = span->token_offset + i;
            const uint64_t index = token / P;
            if (index >= span->dst_page_table_len)
                return fail(SGL_KV_INVALID_ARGUMENT, "dst_page_table", index, span->dst_page_table_len, 0,
                            "token %llu needs page-table entry %llu of %llu", (unsigned long long)token,
                            (unsigned long long)index, (unsigned long long)span->dst_page_table_len);
            const int32_t page = span->dst_page_table[index];
            if (page < 0 || (uint64_t)page >= dl.page_count)
                return fail(SGL_KV_LAYOUT_PAGE_OUT_OF_RANGE, nullptr, (uint64_t)(int64_t)page, dl.page_count, 0,
                            "KV cache page index %d is outside %llu pages", page,
                            (unsigned long long)dl.page_count);
            upload[n + i] = (uint64_t)page * P + token % P;
        }
    }
    // The upload and the clear of the span's error word go through the side
    // stream, so that they do not wait for earlier spans still running on
    // the transfer streams; the buffer and the word are free, so no running
    // span reads them.
    const uint64_t bytes = upload.size() * sizeof(uint64_t);
    if ((rc = take_slot_buffer(b, bytes, &t.slots))) return rc;
    t.word = b->free_words.back();
    b->free_words.pop_back();
    uint32_t *word = b->span_words + t.word;
    hipError_t err = hipMemcpyAsync(t.slots.ptr, upload.data(), bytes, hipMemcpyHostToDevice, b->side);
    if (err == hipSuccess) err = hipMemsetAsync(word, 0, sizeof(uint32_t), b->side);
    if (err == hipSuccess) err = hipStreamSynchronize(b->side);
    if (err == hipSuccess) err = hipEventCreateWithFlags(&t.done, hipEventDisableTiming);
    if (err != hipSuccess) {
        release_transfer(b, t);
        return hip_fail(err, "sgl_rocm_kv_backend_submit");
    }
    uint64_t *slot_words = static_cast<uint64_t *>(t.slots.ptr);
    sgl_kv_device_buffer src_slots{slot_words, n * sizeof(uint64_t)};
    sgl_kv_device_buffer dst_slots{slot_words + n, n * sizeof(uint64_t)};
    const uint32_t layers = (uint32_t)b->views[0].size();
    hipEvent_t resolved = nullptr;  // staged: the device-side resolve precedes the pipeline
    if (device_table) {
        // Staged spans share the staging set, so even the resolve waits for
        // the previous span; direct spans are ordered by b->stream itself.
        if (b->config.mode == SGL_KV_BACKEND_STAGED && b->last_done)
            err = hipStreamWaitEvent(b->stream, b->last_done, 0);
        sglkv_resolve_params rp;
        memset(&rp, 0, sizeof rp);
        rp.spans = reinterpret_cast<const sglkv_span *>(slot_words + 2 * n);
        rp.page_table = span->dst_page_table;
        rp.out_slots = slot_words + n;
        rp.flag = word;
        rp.page_table_len = span->dst_page_table_len;
        rp.page_count = dl.page_count;
        rp.span_count = 1;
        rp.page_size = (uint32_t)P;
        rp.rows = (uint32_t)n;
        void *args[] = {&rp};
        if (err == hipSuccess)
            err = hipModuleLaunchKernel(b->ctx->resolve, (unsigned)((n + SGLKV_BLOCK_THREADS - 1) / SGLKV_BLOCK_THREADS),
                                        1, 1, SGLKV_BLOCK_THREADS, 1, 1, 0, b->stream, args, nullptr);
        if (err == hipSuccess && b->config.mode == SGL_KV_BACKEND_STAGED) {
            err = hipEventCreateWithFlags(&resolved, hipEventDisableTiming);
            if (err == hipSuccess) err = hipEventRecord(resolved, b->stream);
        }
        if (err != hipSuccess) {
            if (resolved) (void)hipEventDestroy(resolved);
            (void)hipStreamSynchronize(b->stream);
            release_transfer(b, t);
            return hip_fail(err, "sgl_rocm_kv_backend_submit_device_table");
        }
    }
    if (b->config.mode == SGL_KV_BACKEND_DIRECT) {
        Launch l;
        rc = prepare_transfer(b->ctx, &b->views[0][0], &src_slots, n, &b->views[1][0], &dst_slots, &l,
                              layers, b->layer_stride[0], b->layer_stride[1]);
        if (!rc) {
            set_launch_flag(l, word);
            rc = submit_launch(b->ctx, l, b->stream);
        }
        if (!rc && (err = hipEventRecord(t.done, b->stream)) != hipSuccess) rc = hip_fail(err, "hipEventRecord");
    } else {
        sgl_kv_pipeline_desc d;
        memset(&d, 0, sizeof d);
        d.layers = layers;
        d.staged = 1;
        d.src_layers = b->views[0].data();
        d.dst_layers = b->views[1].data();
        d.src_slots = src_slots;
        d.dst_slots = dst_slots;
        d.row_count = n;
        char *dev = static_cast<char *>(b->staging_device);
        char *host = static_cast<char *>(b->staging_host);
        for (int i = 0; i < 2; ++i) {
            d.send[i] = sgl_kv_device_buffer{dev + i * b->layer_bytes, b->layer_bytes};
            d.recv[i] = sgl_kv_device_buffer{dev + (2 + i) * b->layer_bytes, b->layer_bytes};
            d.host[i] = host + i * b->layer_bytes;
        }
        d.host_bytes = b->layer_bytes;
        rc = sgl_rocm_kv_pipeline_create(b->ctx, &d, &t.pipeline);
        if (!rc) pipeline_set_error_word(t.pipeline, word);
        // Spans share the staging buffers: each starts after the previous
        // one (or after its own resolve, which waited for it).
        if (!rc) rc = sgl_rocm_kv_pipeline_run(t.pipeline, resolved ? resolved : b->last_done);
        if (!rc && (err = hipEventRecord(t.done, pipeline_final_stream(t.pipeline))) != hipSuccess)
            rc = hip_fail(err, "hipEventRecord");
        if (!rc) b->last_done = t.done;
    }
    if (resolved) (void)hipEventDestroy(resolved);
    if (rc) {
        // Nothing was enqueued after a failed preparation; a failed enqueue
        // leaves work that must drain before the buffers are reused.
        if (t.pipeline) (void)sgl_rocm_kv_pipeline_wait(t.pipeline);
        (void)hipStreamSynchronize(b->stream);
        release_transfer(b, t);
        return rc;
    }
    b->inflight.push_back(t);
    return ok();
}

}  // namespace

extern "C" int32_t sgl_rocm_kv_backend_submit(sgl_rocm_kv_backend *b, const sgl_kv_transfer_span_desc *span) {
    return submit_span(b, span, false);
}

extern "C" int32_t sgl_rocm_kv_backend_submit_device_table(sgl_rocm_kv_backend *b,
                                                           const sgl_kv_transfer_span_desc *span) {
    return submit_span(b, span, true);
}

// KvTransferBackend::poll: each finished span once, in submission order
// (poll_submitted_transfers, transfer.rs:2633-2674); at most `capacity`
// events per call, the rest stay for the next poll.
extern "C" int32_t sgl_rocm_kv_backend_poll(sgl_rocm_kv_backend *b, sgl_kv_transfer_event *events,
                                            uint64_t capacity, uint64_t *event_count,
                                            uint64_t *pending) {
    int32_t rc = check_backend(b);
    if (rc) return rc;
    if (!event_count || !pending || (capacity && !events))
        return fail(SGL_KV_INVALID_ARGUMENT, "events/event_count/pending", 0, 0, 0, "null argument");
    *event_count = 0;
    DeviceScope scope(b->ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    std::vector<Transfer> still;
    still.reserve(b->inflight.size());
    for (size_t i = 0; i < b->inflight.size(); ++i) {
        Transfer &t = b->inflight[i];
        const hipError_t q = (*event_count == capacity && !t.canceled) ? hipErrorNotReady
                                                                       : hipEventQuery(t.done);
        if (q == hipErrorNotReady) {
            still.push_back(t);
            continue;
        }
        if (q != hipSuccess) {
            // Keep the unvisited spans so that a later poll or shutdown
            // still owns them.
            still.insert(still.end(), b->inflight.begin() + i, b->inflight.end());
            b->inflight.swap(still);
            return hip_fail(q, "hipEventQuery");
        }
        if (!t.canceled) {
            // A device-side error fails the span that raised it (a decode
            // page-table entry the device-side resolve found out of range;
            // host-validated spans raise none).
            uint32_t flag = 0;
            if ((rc = read_span_errors(b, t, &flag))) {
                still.insert(still.end(), b->inflight.begin() + i, b->inflight.end());
                b->inflight.swap(still);
                return rc;
            }
            const int32_t code = flag ? flag_status(flag) : SGL_KV_OK;
            sgl_kv_transfer_event &e = events[(*event_count)++];
            memset(&e, 0, sizeof e);
            e.bootstrap_room = t.room;
            memcpy(e.descriptor_checksum, t.checksum, 65);
            e.status = code ? SGL_KV_TRANSFER_FAILED : SGL_KV_TRANSFER_COMPLETED;
            e.error_code = code;
        }
        release_transfer(b, t);
    }
    b->inflight.swap(still);
    uint64_t live = 0;
    for (const Transfer &t : b->inflight) live += t.canceled ? 0 : 1;
    *pending = live;
    return ok();
}

// KvTransferBackend::cancel: the room's spans leave the pending set and
// will produce no event; their device work drains before release.
extern "C" int32_t sgl_rocm_kv_backend_cancel(sgl_rocm_kv_backend *b, uint64_t bootstrap_room) {
    int32_t rc = check_backend(b);
    if (rc) return rc;
    for (Transfer &t : b->inflight)
        if (t.room == bootstrap_room) t.canceled = true;
    return ok();
}

// Blocks until every submitted span has finished on the device.
extern "C" int32_t sgl_rocm_kv_backend_wait(sgl_rocm_kv_backend *b) {
    int32_t rc = check_backend(b);
    if (rc) return rc;
    DeviceScope scope(b->ctx->device);
    for (Transfer &t : b->inflight) SGLKV_CHECK_HIP(hipEventSynchronize(t.done));
    return ok();
}

// KvTransferBackend::shutdown: drains, releases every buffer and forgets
// the registered memory; the backend can be registered again.
extern "C" int32_t sgl_rocm_kv_backend_shutdown(sgl_rocm_kv_backend *b) {
    int32_t rc = check_backend(b);
    if (rc) return rc;
    DeviceScope scope(b->ctx->device);
    for (Transfer &t : b->inflight) {
        if (t.done) (void)hipEventSynchronize(t.done);
        release_transfer(b, t);
    }
    b->inflight.clear();
    b->last_done = nullptr;
    for (SlotBuffer &s : b->free_slots) (void)hipFree(s.ptr);
    b->free_slots.clear();
    release_staging(b);
    b->views[0].clear();
    b->views[1].clear();
    b->registered = false;
    return ok();
}

extern "C" int32_t sgl_rocm_kv_backend_destroy(sgl_rocm_kv_backend *b) {
    if (!b) return ok();
    sgl_rocm_kv_backend_shutdown(b);
    {
        DeviceScope scope(b->ctx->device);
        if (b->stream) (void)hipStreamDestroy(b->stream);
        if (b->side) (void)hipStreamDestroy(b->side);
        if (b->flag_host) (void)hipHostFree(b->flag_host);
        if (b->span_words) (void)hipFree(b->span_words);
    }
    delete b;
    return ok();
}
