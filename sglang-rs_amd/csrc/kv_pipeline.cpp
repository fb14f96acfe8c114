// kv_pipeline.cpp -- layer pipeline of a whole-request KV transfer:
// pack -> (D2H -> pinned host -> H2D) -> unpack, overlapped across layers on
// four HIP streams. This is the device half of a PD transfer backend
// (KvTransferBackend, crates/sglang-srt/src/transfer.rs:1145-1151, which
// execute_kv_cache_transfer_plan drives per span, transfer.rs:1205-1231);
// the pinned-host hop stands in for the inter-node link on one GPU.
//
// Every launch is validated when the pipeline is created, so a run only
// enqueues work. Two send, recv and host buffers alternate between layers;
// events order each reuse:
//   pack(l)   writes send[l%2]  after D2H(l-2) (staged) / unpack(l-2) read it
//   D2H(l)    writes host[l%2]  after H2D(l-2) read it
//   H2D(l)    writes recv[l%2]  after unpack(l-2) read it
#include <hip/hip_runtime.h>
#include <string.h>

#include <vector>

#include "kv_internal.h"

using namespace sglkv;

namespace {

enum Stage { kPack = 0, kD2H = 1, kH2D = 2, kUnpack = 3, kStages = 4 };

}  // namespace

struct sgl_rocm_kv_pipeline {
    sgl_rocm_kv_ctx *ctx = nullptr;
    uint32_t layers = 0;
    bool staged = false;
    uint64_t layer_bytes = 0;  // one layer's rows: row_count * (key + value row bytes)
    std::vector<Launch> pack, unpack;
    void *send[2] = {nullptr, nullptr};
    void *recv[2] = {nullptr, nullptr};
    void *host[2] = {nullptr, nullptr};
    hipStream_t stream[kStages] = {nullptr, nullptr, nullptr, nullptr};
    // start/end event per stage per layer
    std::vector<hipEvent_t> start, end;
    bool ran = false;

    hipEvent_t &ev_start(uint32_t l, int s) { return start[(size_t)l * kStages + s]; }
    hipEvent_t &ev_end(uint32_t l, int s) { return end[(size_t)l * kStages + s]; }
    hipEvent_t ev_start(uint32_t l, int s) const { return start[(size_t)l * kStages + s]; }
    hipEvent_t ev_end(uint32_t l, int s) const { return end[(size_t)l * kStages + s]; }

    void release() {
        for (hipEvent_t e : start)
            if (e) (void)hipEventDestroy(e);
        for (hipEvent_t e : end)
            if (e) (void)hipEventDestroy(e);
        start.clear();
        end.clear();
        for (hipStream_t &s : stream)
            if (s) {
                (void)hipStreamDestroy(s);
                s = nullptr;
            }
    }
};

namespace {

// Rows view of one layer inside a [tensor][row][row bytes of the tensor]
// buffer (tensor 1's plane follows tensor 0's rows).
sgl_kv_rows_view layer_rows(void *base, uint64_t byte_len, uint32_t tensors, uint64_t rows,
                            const uint64_t row_bytes[2]) {
    sgl_kv_rows_view v;
    memset(&v, 0, sizeof v);
    uint64_t at = 0;
    for (uint32_t t = 0; t < tensors; ++t) {
        v.planes[t] = static_cast<char *>(base) + at;
        v.plane_bytes[t] = byte_len > at ? byte_len - at : 0;
        v.row_stride[t] = row_bytes[t];
        at += rows * row_bytes[t];
    }
    return v;
}

int32_t check_buffer(const char *name, const void *ptr, uint64_t have, uint64_t need) {
    if (!ptr) return fail(SGL_KV_INVALID_ARGUMENT, name, 0, 0, 0, "null staging buffer %s", name);
    if (have < need)
        return fail(SGL_KV_ALLOCATION_OUT_OF_BOUNDS, name, 0, need, have,
                    "staging buffer %s holds %llu bytes, a layer needs %llu", name,
                    (unsigned long long)have, (unsigned long long)need);
    return SGL_KV_OK;
}

}  // namespace

extern "C" int32_t sgl_rocm_kv_pipeline_create(sgl_rocm_kv_ctx *ctx, const sgl_kv_pipeline_desc *d,
                                               sgl_rocm_kv_pipeline **out) {
    if (!ctx || !d || !out)
        return fail(SGL_KV_INVALID_ARGUMENT, "ctx/desc/out", 0, 0, 0, "null argument");
    *out = nullptr;
    if (d->layers == 0 || !d->src_layers || !d->dst_layers)
        return fail(SGL_KV_INVALID_ARGUMENT, "layers", d->layers, 0, 0,
                    "a pipeline needs at least one layer and both layer view arrays");
    const sgl_kv_pool_view &first = d->src_layers[0];
    const uint32_t tensors = first.tensor_count;
    const uint64_t row_bytes[2] = {first.row_bytes, view_row_bytes(first, 1)};
    uint64_t layer_bytes = 0;
    for (uint32_t t = 0; t < tensors && t < 2; ++t) {
        uint64_t plane;
        if (mul_ovf(d->row_count, row_bytes[t], &plane) || add_ovf(layer_bytes, plane, &layer_bytes))
            return fail(SGL_KV_SHAPE_OVERFLOW, nullptr, 0, 0, 0, "KV copy tensor shape overflowed");
    }
    int32_t rc;
    for (int b = 0; b < 2; ++b) {
        static const char *const send_names[2] = {"send[0]", "send[1]"};
        static const char *const recv_names[2] = {"recv[0]", "recv[1]"};
        static const char *const host_names[2] = {"host[0]", "host[1]"};
        if ((rc = check_buffer(send_names[b], d->send[b].ptr, d->send[b].byte_len, layer_bytes)))
            return rc;
        if (d->staged) {
            if ((rc = check_buffer(recv_names[b], d->recv[b].ptr, d->recv[b].byte_len, layer_bytes)) ||
                (rc = check_buffer(host_names[b], d->host[b], d->host_bytes, layer_bytes)))
                return rc;
        }
    }
    sgl_rocm_kv_pipeline *p = new sgl_rocm_kv_pipeline();
    p->ctx = ctx;
    p->layers = d->layers;
    p->staged = d->staged != 0;
    p->layer_bytes = layer_bytes;
    for (int b = 0; b < 2; ++b) {
        p->send[b] = d->send[b].ptr;
        p->recv[b] = p->staged ? d->recv[b].ptr : d->send[b].ptr;
        p->host[b] = d->host[b];
    }
    p->pack.resize(d->layers);
    p->unpack.resize(d->layers);
    for (uint32_t l = 0; l < d->layers; ++l) {
        const sgl_kv_pool_view &sv = d->src_layers[l];
        const sgl_kv_pool_view &dv = d->dst_layers[l];
        if (sv.tensor_count != tensors || sv.row_bytes != row_bytes[0] ||
            view_row_bytes(sv, 1) != row_bytes[1] || dv.tensor_count != tensors ||
            dv.row_bytes != row_bytes[0] || view_row_bytes(dv, 1) != row_bytes[1]) {
            delete p;
            return fail(SGL_KV_INVALID_ARGUMENT, "layers", l, 0, 0,
                        "layer %u's views differ in row shape from layer 0", l);
        }
        const int b = l % 2;
        const sgl_kv_rows_view send = layer_rows(p->send[b], d->send[b].byte_len, tensors,
                                                 d->row_count, row_bytes);
        const sgl_kv_rows_view recv = layer_rows(
            p->recv[b], p->staged ? d->recv[b].byte_len : d->send[b].byte_len, tensors, d->row_count,
            row_bytes);
        if ((rc = prepare_pack(ctx, &sv, &d->src_slots, d->row_count, &send, &p->pack[l])) ||
            (rc = prepare_unpack(ctx, &recv, d->row_count, &dv, &d->dst_slots, &p->unpack[l]))) {
            delete p;
            return rc;
        }
    }
    DeviceScope scope(ctx->device);
    hipError_t err = scope.status();
    for (int s = 0; s < kStages && err == hipSuccess; ++s) err = hipStreamCreate(&p->stream[s]);
    p->start.assign((size_t)d->layers * kStages, nullptr);
    p->end.assign((size_t)d->layers * kStages, nullptr);
    for (size_t i = 0; i < p->start.size() && err == hipSuccess; ++i) {
        err = hipEventCreate(&p->start[i]);
        if (err == hipSuccess) err = hipEventCreate(&p->end[i]);
    }
    if (err != hipSuccess) {
        p->release();
        delete p;
        return hip_fail(err, "sgl_rocm_kv_pipeline_create");
    }
    *out = p;
    return ok();
}

#define SGLKV_PIPE_HIP(call)                                   \
    do {                                                       \
        hipError_t e_ = (call);                                \
        if (e_ != hipSuccess) return hip_fail(e_, #call);      \
    } while (0)

extern "C" int32_t sgl_rocm_kv_pipeline_run(sgl_rocm_kv_pipeline *p, void *after) {
    if (!p) return fail(SGL_KV_INVALID_ARGUMENT, "pipeline", 0, 0, 0, "null pipeline");
    DeviceScope scope(p->ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    hipStream_t sp = p->stream[kPack], sd = p->stream[kD2H], sh = p->stream[kH2D],
                su = p->stream[kUnpack];
    if (after) SGLKV_PIPE_HIP(hipStreamWaitEvent(sp, static_cast<hipEvent_t>(after), 0));
    // A previous run's last unpacks may still read send/recv buffers.
    if (p->ran) {
        for (uint32_t l = p->layers >= 2 ? p->layers - 2 : 0; l < p->layers; ++l)
            SGLKV_PIPE_HIP(hipStreamWaitEvent(sp, p->ev_end(l, kUnpack), 0));
    }
    int32_t rc;
    for (uint32_t l = 0; l < p->layers; ++l) {
        const int b = l % 2;
        if (l >= 2)  // send[b] is free once its previous reader finished
            SGLKV_PIPE_HIP(hipStreamWaitEvent(sp, p->ev_end(l - 2, p->staged ? kD2H : kUnpack), 0));
        SGLKV_PIPE_HIP(hipEventRecord(p->ev_start(l, kPack), sp));
        if ((rc = submit_launch(p->ctx, p->pack[l], sp))) return rc;
        SGLKV_PIPE_HIP(hipEventRecord(p->ev_end(l, kPack), sp));
        if (p->staged) {
            SGLKV_PIPE_HIP(hipStreamWaitEvent(sd, p->ev_end(l, kPack), 0));
            if (l >= 2) SGLKV_PIPE_HIP(hipStreamWaitEvent(sd, p->ev_end(l - 2, kH2D), 0));
            SGLKV_PIPE_HIP(hipEventRecord(p->ev_start(l, kD2H), sd));
            SGLKV_PIPE_HIP(hipMemcpyAsync(p->host[b], p->send[b], p->layer_bytes,
                                          hipMemcpyDeviceToHost, sd));
            SGLKV_PIPE_HIP(hipEventRecord(p->ev_end(l, kD2H), sd));
            SGLKV_PIPE_HIP(hipStreamWaitEvent(sh, p->ev_end(l, kD2H), 0));
            if (l >= 2) SGLKV_PIPE_HIP(hipStreamWaitEvent(sh, p->ev_end(l - 2, kUnpack), 0));
            SGLKV_PIPE_HIP(hipEventRecord(p->ev_start(l, kH2D), sh));
            SGLKV_PIPE_HIP(hipMemcpyAsync(p->recv[b], p->host[b], p->layer_bytes,
                                          hipMemcpyHostToDevice, sh));
            SGLKV_PIPE_HIP(hipEventRecord(p->ev_end(l, kH2D), sh));
            SGLKV_PIPE_HIP(hipStreamWaitEvent(su, p->ev_end(l, kH2D), 0));
        } else {
            SGLKV_PIPE_HIP(hipStreamWaitEvent(su, p->ev_end(l, kPack), 0));
        }
        SGLKV_PIPE_HIP(hipEventRecord(p->ev_start(l, kUnpack), su));
        if ((rc = submit_launch(p->ctx, p->unpack[l], su))) return rc;
        SGLKV_PIPE_HIP(hipEventRecord(p->ev_end(l, kUnpack), su));
    }
    p->ran = true;
    return ok();
}

extern "C" int32_t sgl_rocm_kv_pipeline_wait(sgl_rocm_kv_pipeline *p) {
    if (!p) return fail(SGL_KV_INVALID_ARGUMENT, "pipeline", 0, 0, 0, "null pipeline");
    DeviceScope scope(p->ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    for (hipStream_t s : p->stream) SGLKV_PIPE_HIP(hipStreamSynchronize(s));
    return sgl_rocm_kv_check_errors(p->ctx, p->stream[kUnpack]);
}

extern "C" int32_t sgl_rocm_kv_pipeline_layer_times(const sgl_rocm_kv_pipeline *p, uint32_t layer,
                                                    float *ms) {
    if (!p || !ms) return fail(SGL_KV_INVALID_ARGUMENT, "pipeline/ms", 0, 0, 0, "null argument");
    if (layer >= p->layers)
        return fail(SGL_KV_LAYOUT_LAYER_OUT_OF_RANGE, nullptr, layer, p->layers, 0,
                    "KV cache layer index %u is outside %u layers", layer, p->layers);
    if (!p->ran) return fail(SGL_KV_INVALID_ARGUMENT, "pipeline", 0, 0, 0, "the pipeline has not run");
    DeviceScope scope(p->ctx->device);
    for (int s = 0; s < kStages; ++s) {
        ms[s] = 0.0f;
        if (!p->staged && (s == kD2H || s == kH2D)) continue;
        SGLKV_PIPE_HIP(hipEventElapsedTime(&ms[s], p->ev_start(layer, s), p->ev_end(layer, s)));
    }
    SGLKV_PIPE_HIP(hipEventElapsedTime(&ms[4], p->ev_start(layer, kPack), p->ev_end(layer, kUnpack)));
    return ok();
}

extern "C" int32_t sgl_rocm_kv_pipeline_elapsed(const sgl_rocm_kv_pipeline *p, float *ms) {
    if (!p || !ms) return fail(SGL_KV_INVALID_ARGUMENT, "pipeline/ms", 0, 0, 0, "null argument");
    if (!p->ran) return fail(SGL_KV_INVALID_ARGUMENT, "pipeline", 0, 0, 0, "the pipeline has not run");
    DeviceScope scope(p->ctx->device);
    SGLKV_PIPE_HIP(hipEventElapsedTime(ms, p->ev_start(0, kPack), p->ev_end(p->layers - 1, kUnpack)));
    return ok();
}

extern "C" int32_t sgl_rocm_kv_pipeline_destroy(sgl_rocm_kv_pipeline *p) {
    if (!p) return ok();
    {
        DeviceScope scope(p->ctx->device);
        for (hipStream_t s : p->stream)
            if (s) (void)hipStreamSynchronize(s);
        p->release();
    }
    delete p;
    return ok();
}

// The stream of a pipeline's last stage (its unpacks): work recorded there
// after a run completes after every layer of that run.
hipStream_t sglkv::pipeline_final_stream(sgl_rocm_kv_pipeline *p) { return p->stream[kUnpack]; }

// Points every launch of the pipeline at `flag` (a transfer backend gives
// each span its own error word).
void sglkv::pipeline_set_error_word(sgl_rocm_kv_pipeline *p, uint32_t *flag) {
    for (Launch &l : p->pack) set_launch_flag(l, flag);
    for (Launch &l : p->unpack) set_launch_flag(l, flag);
}
