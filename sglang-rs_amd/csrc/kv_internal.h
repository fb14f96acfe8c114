// kv_internal.h -- helpers shared by the host sources of libsgl_rocm_kv.
#ifndef SGLKV_INTERNAL_H
#define SGLKV_INTERNAL_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "kv_params.h"

// The C ABI is the library's only exported surface (built with
// -fvisibility=hidden); the declarations carry default visibility.
#pragma GCC visibility push(default)
#include "sgl_rocm_kv.h"
#pragma GCC visibility pop

namespace sglkv {

// Records the calling thread's failure detail and returns `code`.
int32_t fail(int32_t code, const char *name, uint64_t a, uint64_t b, uint64_t c,
             const char *fmt, ...) __attribute__((format(printf, 6, 7)));
// Clears the detail record and returns SGL_KV_OK.
int32_t ok();
// Sets the fourth field of the detail record of the last failure.
void set_detail_d(uint64_t d);

// Geometry common to both sides of a copy.
struct RowShape {
    uint64_t row_bytes[2];  // per tensor (equal unless a pair of unequal widths)
    uint32_t tensors;
    uint32_t heads;  // > 1 only when a side is head-major
    bool split;      // some side is HND: copy head chunk by head chunk
    uint64_t chunk(uint32_t t) const { return split ? row_bytes[t] / heads : row_bytes[t]; }
};

// Bytes per (token, tensor t) of a pool view: value_row_bytes 0 means both
// tensors are row_bytes wide.
inline uint64_t view_row_bytes(const sgl_kv_pool_view &v, uint32_t t) {
    return t == 1 && v.value_row_bytes ? v.value_row_bytes : v.row_bytes;
}

// A validated copy launch: kernel parameters plus launch geometry.
struct Launch {
    sglkv_copy_params params;
    sglkv_realign_params realign;  // used when `realigned`
    RowShape shape;
    int kind;         // 0 pool->rows, 1 rows->pool, 2 pool->pool
    int width_index;  // vector width 16, 8, 4, 2, 1
    bool realigned;   // the byte-realigning kernel (16-byte accesses at any alignment)
    uint32_t lds_bytes;  // dynamic LDS of the realigning kernel
    uint64_t rows;
    uint64_t grid;
    uint32_t layers;  // grid y: one layer per row of workgroups
    uint32_t block_x, block_y;
};

// Replaces the device error word a validated launch raises (default: the
// context's copy word).
inline void set_launch_flag(Launch &l, uint32_t *flag) {
    l.params.flag = flag;
    l.realign.flag = flag;
}

// Layer span of a multi-layer launch: `count` layers, each side's data
// `pool_stride` / `rows_stride` bytes after the previous layer's.
struct LayerSpan {
    uint32_t count;
    uint64_t pool_stride;
    uint64_t rows_stride;
};

int32_t prepare_pack(const sgl_rocm_kv_ctx *ctx, const sgl_kv_pool_view *src,
                     const sgl_kv_device_buffer *slots, uint64_t row_count,
                     const sgl_kv_rows_view *dst, Launch *l, LayerSpan span = {1, 0, 0});
int32_t prepare_unpack(const sgl_rocm_kv_ctx *ctx, const sgl_kv_rows_view *src, uint64_t row_count,
                       const sgl_kv_pool_view *dst, const sgl_kv_device_buffer *slots, Launch *l,
                       LayerSpan span = {1, 0, 0});
int32_t prepare_transfer(const sgl_rocm_kv_ctx *ctx, const sgl_kv_pool_view *src,
                         const sgl_kv_device_buffer *src_slots, uint64_t row_count,
                         const sgl_kv_pool_view *dst, const sgl_kv_device_buffer *dst_slots,
                         Launch *l, uint32_t layers, uint64_t src_layer_stride,
                         uint64_t dst_layer_stride);
int32_t submit_launch(sgl_rocm_kv_ctx *ctx, Launch &l, hipStream_t stream);
hipStream_t pipeline_final_stream(sgl_rocm_kv_pipeline *pipe);
void pipeline_set_error_word(sgl_rocm_kv_pipeline *pipe, uint32_t *flag);
// The no-allocation entry point's workspace on one device (kv_scratch.hip):
// `lock` makes a call's wait + launch + record one step among host threads,
// `last` is recorded after the last call that used the workspace.
struct NoallocOrder {
    std::mutex lock;
    hipEvent_t last = nullptr;
};
// The device address of the static no-allocation workspace on `device` and
// its ordering (resolved once per device).
int32_t noalloc_workspace(int device, void **out, NoallocOrder **order);
int32_t hip_fail(hipError_t err, const char *call);
int32_t flag_status(uint32_t flag);
int32_t attention_flag_status(uint32_t flag);

inline int32_t too_large_dim(const char *name, uint64_t value, uint64_t maximum) {
    return fail(SGL_KV_DIMENSION_TOO_LARGE, name, value, maximum, 0,
                "KV dimension %s=%llu exceeds maximum %llu", name, (unsigned long long)value,
                (unsigned long long)maximum);
}

inline int32_t too_large_rows(uint64_t rows, uint64_t maximum) {
    return too_large_dim("row_count", rows, maximum);
}

// CudaKvPairCopyKernels::validate_device (cuda_kv_kernels.rs:625-642):
// DeviceMismatch unless `b` lives on the context's device.
int32_t check_device(const sgl_rocm_kv_ctx *ctx, const char *name, const sgl_kv_device_buffer &b);

#define SGLKV_CHECK_HIP(call)                                              \
    do {                                                                   \
        hipError_t e_ = (call);                                            \
        if (e_ != hipSuccess) return ::sglkv::hip_fail(e_, #call);         \
    } while (0)

inline bool mul_ovf(uint64_t a, uint64_t b, uint64_t *out) { return __builtin_mul_overflow(a, b, out); }
inline bool add_ovf(uint64_t a, uint64_t b, uint64_t *out) { return __builtin_add_overflow(a, b, out); }

}  // namespace sglkv

// The per-device context (opaque in the C ABI).
struct sgl_rocm_kv_ctx {
    int device;
    int cu_count;
    hipModule_t module;
    hipFunction_t copy[5][3];
    hipFunction_t realign[3];       // byte-realigning copies: pool->rows, rows->pool, pool->pool
    hipFunction_t resolve;
    hipFunction_t take_flags;       // atomic read-and-clear of error words
    hipFunction_t fill;
    hipFunction_t requests;
    hipFunction_t pair_slots[2];    // key+value slot writes: 16-byte, 1-byte pieces
    hipFunction_t stream_fn[3];     // streaming ceilings: copy, read, write
    // 16-byte vector / element-wise / pipelined dims 128 / pipelined dims <= 128 /
    // wide (K <= 576, V <= 512) / wide dims <= 128 / latent (MLA: K <= 576, V <= 512) /
    // staged (dims 128, rows in LDS) / staged (dims 64) / latent with hi + lo weights /
    // staged (dims 256) / staged (dims 128, K in registers: head-major pages)
    hipFunction_t attention[12];
    hipFunction_t attention_combine;
    hipFunction_t attention_combine_h;    // the latent body's scaled fp16 records
    uint32_t attention_occupancy[12];     // resident workgroups per CU of attention[i] ...
    uint32_t attention_occupancy_lds[12]; // ... at this LDS size (0 = not yet queried)
    int max_lds_per_block;                // device limit on a workgroup's LDS bytes
    // Device error words, at the start of a small zeroed block: one per
    // consumer, as the reference keeps one flag per kernels object
    // (cuda_kv_kernels.rs:421, 460-461; cuda_attention.rs:667, 706-707), so that one
    // consumer's read-and-clear never takes another's bits.
    uint32_t *flag;                 // asynchronous copies, span resolution, page requests
    uint32_t *attn_flag;            // asynchronous paged attention
    uint32_t *pair_flag;            // the synchronous pair scatter/gather drop-ins
    uint32_t *sync_attn_flag;       // the synchronous paged attention
    const uint8_t *zero_row;        // SGLKV_ZERO_ROW_BYTES of zeros inside that block
    void *attention_partial;        // split records, grown on demand
    uint64_t attention_partial_bytes;
    void *noalloc_workspace;        // this device's static workspace (SGL_KV_NOALLOC_WORKSPACE_BYTES)
    sglkv::NoallocOrder *noalloc_order;  // its ordering across streams and contexts
    uint32_t rows_per_thread;  // from the code object
    uint32_t max_tile_rows;
    uint32_t realign_rows_per_thread;
};

namespace sglkv {

// Makes the context's device current for one call and restores the
// caller's device afterwards (the reference pushes and pops its CUDA
// context around every call, crates/sglang-kernel/src/cuda.rs:559-586).
class DeviceScope {
  public:
    explicit DeviceScope(int device) : prev_(-1), device_(device), err_(hipSuccess) {
        err_ = hipGetDevice(&prev_);
        if (err_ == hipSuccess && prev_ != device) err_ = hipSetDevice(device);
    }
    ~DeviceScope() {
        if (prev_ >= 0 && prev_ != device_) (void)hipSetDevice(prev_);
    }
    hipError_t status() const { return err_; }

  private:
    int prev_, device_;
    hipError_t err_;
};

}  // namespace sglkv

#endif
