// kv_runtime.cpp -- kernel entry points of libsgl_rocm_kv (group 2 of
// sgl_rocm_kv.h): context set-up, host validation and launches of the
// gfx950 kernels in sgl_rocm_kv_gfx950.co.
//
// Validation happens on the host before any launch, with the reference's
// error variants (CudaKvPairCopyError, crates/sglang-kernel/src/
// cuda_kv_kernels.rs:304-338, and CudaError::AllocationOutOfBounds,
// crates/sglang-kernel/src/cuda.rs:895-916). What only the device can see
// (a slot or page-table entry outside the pool) is reported through the
// context's error word.
#include <dlfcn.h>
#include <hip/hip_runtime.h>
#include <string.h>

#include <string>

#include "kv_internal.h"
#include "kv_params.h"

using namespace sglkv;

namespace {

constexpr int kWidths[5] = {16, 8, 4, 2, 1};
constexpr int kPoolRows = 0, kRowsPool = 1, kPoolPool = 2;
// Rows per launch: the kernels index rows in 32 bits, and the last tile of a
// launch (at most 512 rows) must still end below 2^32.
constexpr uint64_t kMaxRows = UINT32_MAX - 4096u;
const char *const kKindNames[3] = {"pool_rows", "rows_pool", "pool_pool"};

}  // namespace

int32_t sglkv::hip_fail(hipError_t err, const char *call) {
    return fail(SGL_KV_HIP, call, (uint64_t)err, 0, 0, "%s failed: %s (%d)", call,
                hipGetErrorString(err), (int)err);
}

namespace {

#define SGLKV_HIP(call)                                     \
    do {                                                    \
        hipError_t e_ = (call);                             \
        if (e_ != hipSuccess) return hip_fail(e_, #call);   \
    } while (0)

int32_t out_of_bounds(const char *name, uint64_t offset, uint64_t len, uint64_t have) {
    return fail(SGL_KV_ALLOCATION_OUT_OF_BOUNDS, name, offset, len, have,
                "allocation %s range [%llu, +%llu) exceeds its %llu bytes", name,
                (unsigned long long)offset, (unsigned long long)len, (unsigned long long)have);
}

int32_t too_large(const char *name, uint64_t value, uint64_t maximum) {
    return fail(SGL_KV_DIMENSION_TOO_LARGE, name, value, maximum, 0,
                "KV copy dimension %s=%llu exceeds maximum %llu", name, (unsigned long long)value,
                (unsigned long long)maximum);
}

int32_t shape_overflow() {
    return fail(SGL_KV_SHAPE_OVERFLOW, nullptr, 0, 0, 0, "KV copy tensor shape overflowed");
}

// Validates one pool side and fills its kernel description.
int32_t pool_side(const sgl_kv_pool_view *v, const sgl_kv_device_buffer *slots, uint64_t rows,
                  const RowShape &shape, sglkv_side *out) {
    if (!v || !v->base) return fail(SGL_KV_INVALID_ARGUMENT, "pool", 0, 0, 0, "null pool view");
    if (!slots || !slots->ptr)
        return fail(SGL_KV_INVALID_ARGUMENT, "slot_indices", 0, 0, 0, "null slot map");
    uint64_t need;
    if (mul_ovf(rows, 8, &need)) return shape_overflow();
    if (need > slots->byte_len) return out_of_bounds("slot_indices", 0, need, slots->byte_len);
    uint64_t slot_count, tensor_page_bytes[2] = {0, 0};
    if (mul_ovf(v->page_size, v->page_count, &slot_count)) return shape_overflow();
    for (uint32_t t = 0; t < v->tensor_count; ++t)
        if (mul_ovf(v->page_size, view_row_bytes(*v, t), &tensor_page_bytes[t])) return shape_overflow();
    if (slot_count > UINT32_MAX) return too_large("slot_count", slot_count, UINT32_MAX);
    const char *names[2] = {v->tensor_count == 2 ? "key" : "latent", "value"};
    uint64_t ends[2] = {0, 0};
    for (uint32_t t = 0; t < v->tensor_count; ++t) {
        if (add_ovf(v->tensor_offset[t], tensor_page_bytes[t], &ends[t])) return shape_overflow();
        if (ends[t] > v->page_stride_bytes)
            return fail(SGL_KV_TENSOR_PAGE_REGION_OUT_OF_BOUNDS, names[t], v->tensor_offset[t],
                        tensor_page_bytes[t], v->page_stride_bytes,
                        "KV copy %s page region [%llu, %llu) exceeds page stride %llu", names[t],
                        (unsigned long long)v->tensor_offset[t], (unsigned long long)ends[t],
                        (unsigned long long)v->page_stride_bytes);
    }
    if (v->tensor_count == 2 && v->tensor_offset[0] < ends[1] && v->tensor_offset[1] < ends[0])
        return fail(SGL_KV_TENSOR_PAGE_REGIONS_OVERLAP, nullptr, v->tensor_offset[0],
                    v->tensor_offset[1], tensor_page_bytes[0],
                    "KV copy key/value page regions overlap: key offset %llu, value offset %llu, "
                    "tensor page size %llu bytes",
                    (unsigned long long)v->tensor_offset[0], (unsigned long long)v->tensor_offset[1],
                    (unsigned long long)tensor_page_bytes[0]);
    // The pool must reach the end of the last slot's last tensor row
    // (CudaKvPairCopyPlan's pool_required_bytes, cuda_kv_kernels.rs:220-234).
    const uint64_t last_end = ends[0] > ends[1] ? ends[0] : ends[1];
    uint64_t required;
    if (mul_ovf(v->page_count - 1, v->page_stride_bytes, &required) ||
        add_ovf(required, last_end, &required))
        return shape_overflow();
    if (required > v->byte_len) return out_of_bounds("pool", 0, required, v->byte_len);

    const bool hnd = v->head_layout == SGL_KV_HND;
    memset(out, 0, sizeof *out);
    const uint64_t base = (uint64_t)(uintptr_t)v->base;
    out->plane[0] = base + v->tensor_offset[0];
    out->plane[1] = base + (v->tensor_count == 2 ? v->tensor_offset[1] : v->tensor_offset[0]);
    out->stride[0] = out->stride[1] = v->page_stride_bytes;
    out->slots = static_cast<const uint64_t *>(slots->ptr);
    for (uint32_t t = 0; t < 2; ++t) {
        const uint32_t vt = t < v->tensor_count ? t : 0;
        const uint64_t chunk = shape.chunk(vt);
        out->pos_mult[t] = hnd ? chunk : view_row_bytes(*v, vt);
        out->head_stride[t] = hnd ? v->page_size * chunk : chunk;
    }
    out->slot_count = slot_count;
    out->page_size = (uint32_t)v->page_size;
    return SGL_KV_OK;
}

int32_t check_pool_shape(const sgl_kv_pool_view *v) {
    if (!v || !v->base) return fail(SGL_KV_INVALID_ARGUMENT, "pool", 0, 0, 0, "null pool view");
    const struct {
        const char *name;
        uint64_t value;
    } dims[] = {{"page_size", v->page_size},
                {"page_stride_bytes", v->page_stride_bytes},
                {"page_count", v->page_count},
                {"row_bytes", v->row_bytes},
                {"tensor_count", v->tensor_count},
                {"heads", v->heads}};
    for (const auto &d : dims)
        if (d.value == 0)
            return fail(SGL_KV_ZERO_DIMENSION, d.name, 0, 0, 0, "KV copy dimension %s must be non-zero",
                        d.name);
    if (v->tensor_count > 2)
        return fail(SGL_KV_INVALID_ARGUMENT, "tensor_count", v->tensor_count, 2, 0,
                    "a pool view holds one or two tensors, not %u", v->tensor_count);
    if (v->tensor_count == 1 && v->value_row_bytes)
        return fail(SGL_KV_INVALID_ARGUMENT, "value_row_bytes", v->value_row_bytes, 0, 0,
                    "a one-tensor pool view has no value width (%llu)",
                    (unsigned long long)v->value_row_bytes);
    if (v->head_layout > SGL_KV_HND)
        return fail(SGL_KV_INVALID_ARGUMENT, "head_layout", v->head_layout, 0, 0,
                    "unknown head layout %u", v->head_layout);
    if (v->page_size > UINT32_MAX) return too_large("page_size", v->page_size, UINT32_MAX);
    for (uint32_t t = 0; t < v->tensor_count; ++t)
        if (v->head_layout == SGL_KV_HND && view_row_bytes(*v, t) % v->heads)
            return fail(SGL_KV_INVALID_ARGUMENT, "heads", v->heads, view_row_bytes(*v, t), 0,
                        "%u heads do not split a %llu-byte row evenly", v->heads,
                        (unsigned long long)view_row_bytes(*v, t));
    return SGL_KV_OK;
}

// The row geometry a pool view fixes for a copy.
RowShape shape_of(const sgl_kv_pool_view &v, bool split, uint32_t heads) {
    RowShape s;
    s.row_bytes[0] = v.row_bytes;
    s.row_bytes[1] = v.tensor_count == 2 ? view_row_bytes(v, 1) : v.row_bytes;
    s.tensors = v.tensor_count;
    s.heads = split ? heads : 1u;
    s.split = split;
    return s;
}

// Validates a transfer-rows side; `names` label the planes in errors.
int32_t rows_side(const sgl_kv_rows_view *v, uint64_t rows, const RowShape &shape,
                  const char *const names[2], sglkv_side *out) {
    if (!v) return fail(SGL_KV_INVALID_ARGUMENT, "rows", 0, 0, 0, "null rows view");
    memset(out, 0, sizeof *out);
    for (uint32_t t = 0; t < shape.tensors; ++t) {
        const uint64_t rb = shape.row_bytes[t];
        if (!v->planes[t]) return fail(SGL_KV_INVALID_ARGUMENT, names[t], 0, 0, 0, "null plane");
        if (v->row_stride[t] < rb)
            return fail(SGL_KV_ROW_STRIDE_TOO_SMALL, names[t], rb, v->row_stride[t], 0,
                        "KV copy %s row stride %llu bytes is smaller than row width %llu bytes",
                        names[t], (unsigned long long)v->row_stride[t], (unsigned long long)rb);
        uint64_t need;
        if (mul_ovf(rows - 1, v->row_stride[t], &need) || add_ovf(need, rb, &need))
            return shape_overflow();
        if (need > v->plane_bytes[t]) return out_of_bounds(names[t], 0, need, v->plane_bytes[t]);
        out->plane[t] = (uint64_t)(uintptr_t)v->planes[t];
        out->stride[t] = v->row_stride[t];
        out->head_stride[t] = shape.chunk(t);
    }
    if (shape.tensors == 1) {
        out->plane[1] = out->plane[0];
        out->stride[1] = out->stride[0];
        out->head_stride[1] = out->head_stride[0];
    }
    return SGL_KV_OK;
}

// Widest power-of-two access (<= 16 bytes) that divides every address and
// stride either side computes.
int vector_bytes(const sglkv_side &s, const sglkv_side &d, const RowShape &shape) {
    uint64_t bits = shape.chunk(0) | shape.chunk(shape.tensors - 1);
    for (const sglkv_side *x : {&s, &d})
        bits |= x->plane[0] | x->plane[1] | x->stride[0] | x->stride[1] | x->pos_mult[0] |
                x->pos_mult[1] | x->head_stride[0] | x->head_stride[1];
    int vb = 16;
    while (vb > 1 && (bits & (uint64_t)(vb - 1))) vb >>= 1;
    return vb;
}

}  // namespace

namespace {

std::string default_code_object() {
    Dl_info info;
    if (dladdr(reinterpret_cast<void *>(&sgl_rocm_kv_init), &info) && info.dli_fname) {
        std::string path(info.dli_fname);
        const size_t slash = path.rfind('/');
        return (slash == std::string::npos ? std::string(".") : path.substr(0, slash)) +
               "/sgl_rocm_kv_gfx950.co";
    }
    return "sgl_rocm_kv_gfx950.co";
}

// Fills the launch geometry of a validated copy (vector width, tile) from
// the context's code-object constants.
// The byte-realigning kernel's launch: one thread per LDS vector of a row
// (blockDim.x = vrow), the code object's realign rows per thread.
// Returns false when a row's LDS footprint is too wide for it.
bool plan_realign(const sgl_rocm_kv_ctx *ctx, Launch *l) {
    const RowShape &shape = l->shape;
    sglkv_realign_params &r = l->realign;
    const uint64_t chunks = shape.split ? shape.heads : 1u;
    uint64_t vrow = 0, vt0 = 0;
    for (uint32_t t = 0; t < shape.tensors; ++t) {
        const uint64_t c = shape.chunk(t);
        const uint64_t seg = (c + 30) / 16;  // vectors covering c bytes at any alignment
        if (c > UINT32_MAX || seg * chunks > SGLKV_REALIGN_MAX_ROW_VECTORS) return false;
        r.chunk[t] = (uint32_t)c;
        r.seg[t] = (uint32_t)seg;
        vrow += seg * chunks;
        if (t == 0) vt0 = vrow;
    }
    if (vrow > SGLKV_REALIGN_MAX_ROW_VECTORS) return false;
    if (shape.tensors == 1) {
        r.chunk[1] = r.chunk[0];
        r.seg[1] = r.seg[0];
    }
    r.src = l->params.src;
    r.dst = l->params.dst;
    r.flag = ctx->flag;
    r.scale_src = l->params.scale_src;
    r.scale_dst = l->params.scale_dst;
    r.scale_count = l->params.scale_count;
    r.rows = (uint32_t)l->rows;
    r.vt0 = (uint32_t)vt0;
    r.vrow = (uint32_t)vrow;
    r.rows_per_thread = ctx->realign_rows_per_thread;
    r.zero = ctx->zero_row;
    l->block_x = (uint32_t)vrow;
    l->block_y = SGLKV_BLOCK_THREADS / l->block_x;
    // Tiles of at most 512 rows.
    if (l->block_y * r.rows_per_thread > 512) l->block_y = 512 / r.rows_per_thread;
    r.tile_rows = l->block_y * r.rows_per_thread;
    l->lds_bytes = SGLKV_REALIGN_LDS_BYTES(r.tile_rows, r.vrow);
    if (l->lds_bytes > (uint32_t)ctx->max_lds_per_block) return false;
    l->grid = (l->rows + r.tile_rows - 1) / r.tile_rows;
    l->realigned = true;
    return true;
}

int32_t finish_launch(const sgl_rocm_kv_ctx *ctx, Launch *l) {
    sglkv_copy_params &p = l->params;
    const RowShape &shape = l->shape;
    if (l->rows > kMaxRows) return too_large("row_count", l->rows, kMaxRows);
    const int vb = vector_bytes(p.src, p.dst, shape);
    uint64_t row_vectors = 0;
    for (uint32_t t = 0; t < shape.tensors; ++t) row_vectors += shape.row_bytes[t] / vb;
    if (row_vectors > (1ull << 31)) return too_large("row_bytes", shape.row_bytes[0], 1ull << 30);
    int wi = 0;
    while (kWidths[wi] != vb) ++wi;
    l->width_index = wi;
    l->realigned = false;
    l->lds_bytes = 0;
    p.flag = ctx->flag;
    p.rows = (uint32_t)l->rows;
    // Rows that do not fall on 16-byte vectors move through the realigning
    // kernel: its accesses stay 16 bytes wide where the plain kernel's would
    // narrow to the common alignment (down to single bytes for the odd
    // 649-byte packed-MLA rows).
    if (vb < 16 && plan_realign(ctx, l)) {
        // A dispatch counts its work-items in 32 bits.
        const uint64_t max_grid = UINT32_MAX / ((uint64_t)l->block_x * l->block_y);
        if (l->grid > max_grid) return too_large("grid blocks", l->grid, max_grid);
        return SGL_KV_OK;
    }
    p.vpr = (uint32_t)row_vectors;
    p.vpt = (uint32_t)(shape.row_bytes[0] / vb);
    p.vpc[0] = (uint32_t)(shape.chunk(0) / vb);
    p.vpc[1] = (uint32_t)(shape.chunk(shape.tensors - 1) / vb);
    l->block_x = p.vpr < SGLKV_BLOCK_THREADS ? p.vpr : SGLKV_BLOCK_THREADS;
    uint32_t by = SGLKV_BLOCK_THREADS / l->block_x;
    if (by > ctx->max_tile_rows / ctx->rows_per_thread) by = ctx->max_tile_rows / ctx->rows_per_thread;
    l->block_y = by;
    p.tile_rows = by * ctx->rows_per_thread;
    // A pool side with head-major pages whose head chunks are whole 16-byte
    // vectors under a cache line (e.g. 64 bytes: fp8 x 64 dims, bf16 x 32):
    // regroup the lanes so that a line's consecutive positions share a wave.
    const uint64_t cb = shape.chunk(0);
    auto head_major = [&](const sglkv_side &s) { return s.slots && s.head_stride[0] != cb; };
    p.line_rows = 0;
    if (vb == 16 && (head_major(p.src) || head_major(p.dst)) && cb < 128 && 128 % cb == 0 &&
        shape.chunk(shape.tensors - 1) == cb && l->block_x == p.vpr && l->block_y % (128 / cb) == 0)
        p.line_rows = (uint32_t)(128 / cb);
    l->grid = (l->rows + p.tile_rows - 1) / p.tile_rows;
    const uint64_t max_grid = UINT32_MAX / ((uint64_t)l->block_x * l->block_y);  // 32-bit work-item count
    if (l->grid > max_grid) return too_large("grid blocks", l->grid, max_grid);
    return SGL_KV_OK;
}

void attach_scales(sglkv_copy_params &p, float *src, float *dst, uint32_t tensors) {
    if (src && dst) {
        p.scale_src = src;
        p.scale_dst = dst;
        p.scale_count = tensors;
    }
}

int32_t check_ctx(const sgl_rocm_kv_ctx *ctx) {
    if (!ctx) return fail(SGL_KV_INVALID_ARGUMENT, "ctx", 0, 0, 0, "null context");
    return SGL_KV_OK;
}

int32_t device_of(const void *ptr, int *device) {
    hipPointerAttribute_t attr;
    memset(&attr, 0, sizeof attr);
    hipError_t err = hipPointerGetAttributes(&attr, ptr);
    if (err != hipSuccess) {
        (void)hipGetLastError();
        *device = -1;
        return SGL_KV_OK;
    }
    *device = attr.type == hipMemoryTypeHost ? -1 : attr.device;
    return SGL_KV_OK;
}

// CudaKvPairCopyKernels::validate_device (cuda_kv_kernels.rs:625-642).
int32_t validate_device(const sgl_rocm_kv_ctx *ctx, const char *name, const sgl_kv_device_buffer &b) {
    int dev;
    device_of(b.ptr, &dev);
    if (dev != ctx->device)
        return fail(SGL_KV_DEVICE_MISMATCH, name, (uint64_t)ctx->device, (uint64_t)(int64_t)dev, 0,
                    "KV copy allocation %s is on device %d, expected device %d", name, dev,
                    ctx->device);
    return SGL_KV_OK;
}

}  // namespace

int32_t sglkv::check_device(const sgl_rocm_kv_ctx *ctx, const char *name, const sgl_kv_device_buffer &b) {
    return validate_device(ctx, name, b);
}

namespace {

// CudaDeviceAllocation::device_ptr_at (cuda.rs:895-916).
int32_t ptr_at(const char *name, const sgl_kv_device_buffer &b, uint64_t offset, uint64_t len,
               uint64_t *out) {
    uint64_t end;
    if (add_ovf(offset, len, &end) || end > b.byte_len) return out_of_bounds(name, offset, len, b.byte_len);
    *out = (uint64_t)(uintptr_t)b.ptr + offset;
    return SGL_KV_OK;
}

// Launch, synchronise, read the error word (CudaKvPairCopyKernels::launch,
// cuda_kv_kernels.rs:541-623).
int32_t pair_copy(sgl_rocm_kv_ctx *ctx, const sgl_kv_pair_copy_plan *plan,
                  const sgl_kv_pair_copy_buffers *b, hipStream_t stream, bool scatter) {
    int32_t rc = check_ctx(ctx);
    if (rc) return rc;
    if (!plan || !b) return fail(SGL_KV_INVALID_ARGUMENT, "plan/buffers", 0, 0, 0, "null argument");
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    // Same check order as the reference: scatter validates keys, values,
    // slots, pool; gather validates pool, slots, keys, values.
    struct Buf {
        const char *name;
        const sgl_kv_device_buffer *buf;
        uint64_t offset, required;
        uint64_t *addr;
    };
    uint64_t keys = 0, values = 0, slots = 0, pool = 0;
    const Buf k{"keys", &b->keys, b->keys_offset, plan->key_rows_required_bytes, &keys};
    const Buf v{"values", &b->values, b->values_offset, plan->value_rows_required_bytes, &values};
    const Buf s{"slot_indices", &b->slot_indices, b->slot_indices_offset,
                plan->slot_indices_required_bytes, &slots};
    const Buf q{"pool", &b->pool, b->pool_offset, plan->pool_required_bytes, &pool};
    const Buf scatter_order[4] = {k, v, s, q};
    const Buf gather_order[4] = {q, s, k, v};
    const Buf *order = scatter ? scatter_order : gather_order;
    for (int i = 0; i < 4; ++i)
        if ((rc = validate_device(ctx, order[i].name, *order[i].buf))) return rc;
    for (int i = 0; i < 4; ++i)
        if ((rc = ptr_at(order[i].name, *order[i].buf, order[i].offset, order[i].required,
                         order[i].addr)))
            return rc;
    if (plan->slot_count > UINT32_MAX) return too_large("slot_count", plan->slot_count, UINT32_MAX);
    if (plan->layout.page_size > UINT32_MAX)
        return too_large("page_size", plan->layout.page_size, UINT32_MAX);

    Launch l;
    memset(&l, 0, sizeof l);
    const uint64_t rb = plan->layout.row_bytes;
    l.shape = RowShape{{rb, rb}, 2, 1, false};
    l.kind = scatter ? kRowsPool : kPoolRows;
    l.rows = plan->row_count;
    sglkv_copy_params &p = l.params;
    sglkv_side &ps = scatter ? p.dst : p.src;
    sglkv_side &rs = scatter ? p.src : p.dst;
    ps.plane[0] = pool + plan->layout.key_in_page_offset;
    ps.plane[1] = pool + plan->layout.value_in_page_offset;
    ps.stride[0] = ps.stride[1] = plan->layout.page_stride_bytes;
    ps.slots = reinterpret_cast<const uint64_t *>(slots);
    ps.pos_mult[0] = ps.pos_mult[1] = rb;
    ps.head_stride[0] = ps.head_stride[1] = rb;
    ps.slot_count = plan->slot_count;
    ps.page_size = (uint32_t)plan->layout.page_size;
    rs.plane[0] = keys;
    rs.plane[1] = values;
    rs.stride[0] = plan->key_row_stride_bytes;
    rs.stride[1] = plan->value_row_stride_bytes;
    rs.head_stride[0] = rs.head_stride[1] = rb;
    if ((rc = finish_launch(ctx, &l))) return rc;
    // These drop-ins own an error word, as the reference's kernels object
    // owns its flag (cuda_kv_kernels.rs:421, 550-551): clearing and reading
    // it never touches the bits of the asynchronous calls.
    set_launch_flag(l, ctx->pair_flag);

    SGLKV_HIP(hipMemsetAsync(ctx->pair_flag, 0, sizeof(uint32_t), stream));
    if ((rc = submit_launch(ctx, l, stream))) return rc;
    SGLKV_HIP(hipStreamSynchronize(stream));
    uint32_t flag = 0;
    SGLKV_HIP(hipMemcpy(&flag, ctx->pair_flag, sizeof flag, hipMemcpyDeviceToHost));
    if (flag)
        return fail(SGL_KV_DEVICE_SLOT_INDEX_OUT_OF_RANGE, nullptr, plan->slot_count, 0, 0,
                    "KV copy device slot map contains an index outside %llu slots",
                    (unsigned long long)plan->slot_count);
    return ok();
}

}  // namespace

extern "C" int32_t sgl_rocm_kv_init(int32_t device, const char *code_object_path,
                                    sgl_rocm_kv_ctx **out) {
    if (!out) return fail(SGL_KV_INVALID_ARGUMENT, "out", 0, 0, 0, "null argument");
    *out = nullptr;
    int count = 0;
    hipError_t err = hipGetDeviceCount(&count);
    if (err != hipSuccess) return hip_fail(err, "hipGetDeviceCount");
    if (device < 0 || device >= count)
        return fail(SGL_KV_INVALID_ARGUMENT, "device", (uint64_t)(int64_t)device, (uint64_t)count, 0,
                    "device %d is not one of the %d visible devices", device, count);
    DeviceScope scope(device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    const std::string path = code_object_path ? std::string(code_object_path) : default_code_object();
    sgl_rocm_kv_ctx *ctx = new sgl_rocm_kv_ctx();
    ctx->device = device;
    err = hipModuleLoad(&ctx->module, path.c_str());
    if (err != hipSuccess) {
        delete ctx;
        return fail(SGL_KV_MODULE, "hipModuleLoad", (uint64_t)err, 0, 0,
                    "cannot load code object %s: %s", path.c_str(), hipGetErrorString(err));
    }
    for (int w = 0; w < 5; ++w)
        for (int k = 0; k < 3; ++k) {
            char name[64];
            snprintf(name, sizeof name, "sglkv_copy_%s_v%d", kKindNames[k], kWidths[w]);
            err = hipModuleGetFunction(&ctx->copy[w][k], ctx->module, name);
            if (err != hipSuccess) {
                (void)hipModuleUnload(ctx->module);
                delete ctx;
                return fail(SGL_KV_MODULE, name, (uint64_t)err, 0, 0,
                            "code object %s lacks kernel %s", path.c_str(), name);
            }
        }
    const char *const realign_names[3] = {"sglkv_realign_pool_rows", "sglkv_realign_rows_pool",
                                          "sglkv_realign_pool_pool"};
    err = hipSuccess;
    for (int k = 0; k < 3 && err == hipSuccess; ++k)
        err = hipModuleGetFunction(&ctx->realign[k], ctx->module, realign_names[k]);
    if (err == hipSuccess) err = hipModuleGetFunction(&ctx->resolve, ctx->module, "sglkv_resolve_spans");
    if (err == hipSuccess) err = hipModuleGetFunction(&ctx->take_flags, ctx->module, "sglkv_take_flags");
    if (err == hipSuccess) err = hipModuleGetFunction(&ctx->fill, ctx->module, "sglkv_fill_synthetic");
    const char *const stream_names[3] = {"sglkv_stream_copy", "sglkv_stream_read", "sglkv_stream_write"};
    for (int i = 0; i < 3 && err == hipSuccess; ++i)
        err = hipModuleGetFunction(&ctx->stream_fn[i], ctx->module, stream_names[i]);
    if (err == hipSuccess) err = hipModuleGetFunction(&ctx->requests, ctx->module, "sglkv_copy_requests");
    if (err == hipSuccess)
        err = hipModuleGetFunction(&ctx->pair_slots[0], ctx->module, "sglkv_write_pair_slots_v16");
    if (err == hipSuccess)
        err = hipModuleGetFunction(&ctx->pair_slots[1], ctx->module, "sglkv_write_pair_slots_v1");
    if (err == hipSuccess)
        err = hipModuleGetFunction(&ctx->attention[0], ctx->module, "sglkv_paged_attention_v16");
    if (err == hipSuccess)
        err = hipModuleGetFunction(&ctx->attention[1], ctx->module, "sglkv_paged_attention_v2");
    if (err == hipSuccess)
        err = hipModuleGetFunction(&ctx->attention[2], ctx->module, "sglkv_paged_attention_pipe128");
    if (err == hipSuccess)
        err = hipModuleGetFunction(&ctx->attention[3], ctx->module, "sglkv_paged_attention_pipe");
    if (err == hipSuccess)
        err = hipModuleGetFunction(&ctx->attention[4], ctx->module, "sglkv_paged_attention_wide576");
    if (err == hipSuccess)
        err = hipModuleGetFunction(&ctx->attention[5], ctx->module, "sglkv_paged_attention_wide128");
    if (err == hipSuccess)
        err = hipModuleGetFunction(&ctx->attention[6], ctx->module, "sglkv_paged_attention_latent");
    if (err == hipSuccess)
        err = hipModuleGetFunction(&ctx->attention[7], ctx->module, "sglkv_paged_attention_staged128");
    if (err == hipSuccess)
        err = hipModuleGetFunction(&ctx->attention[8], ctx->module, "sglkv_paged_attention_staged64");
    if (err == hipSuccess)
        err = hipModuleGetFunction(&ctx->attention[9], ctx->module, "sglkv_paged_attention_latent_exact");
    if (err == hipSuccess)
        err = hipModuleGetFunction(&ctx->attention[10], ctx->module, "sglkv_paged_attention_staged256");
    if (err == hipSuccess)
        err = hipModuleGetFunction(&ctx->attention[11], ctx->module, "sglkv_paged_attention_staged128k");
    if (err == hipSuccess)
        err = hipDeviceGetAttribute(&ctx->max_lds_per_block, hipDeviceAttributeMaxSharedMemoryPerBlock, device);
    if (err == hipSuccess)
        err = hipModuleGetFunction(&ctx->attention_combine, ctx->module, "sglkv_paged_attention_combine");
    if (err == hipSuccess)
        err = hipModuleGetFunction(&ctx->attention_combine_h, ctx->module, "sglkv_paged_attention_combine_h");
    if (err == hipSuccess) err = hipDeviceGetAttribute(&ctx->cu_count, hipDeviceAttributeMultiprocessorCount, device);
    // The tile constants the kernels were compiled with.
    const char *const constants[3] = {"sglkv_rows_per_thread", "sglkv_max_tile_rows",
                                      "sglkv_realign_rows_per_thread"};
    uint32_t *const values[3] = {&ctx->rows_per_thread, &ctx->max_tile_rows, &ctx->realign_rows_per_thread};
    for (int i = 0; i < 3 && err == hipSuccess; ++i) {
        hipDeviceptr_t addr = nullptr;
        size_t bytes = 0;
        err = hipModuleGetGlobal(&addr, &bytes, ctx->module, constants[i]);
        if (err == hipSuccess && bytes != sizeof(uint32_t)) err = hipErrorInvalidSymbol;
        if (err == hipSuccess) err = hipMemcpyDtoH(values[i], addr, sizeof(uint32_t));
    }
    if (err == hipSuccess && (ctx->rows_per_thread == 0 || ctx->rows_per_thread > ctx->max_tile_rows ||
                              ctx->realign_rows_per_thread == 0 || ctx->realign_rows_per_thread > 32))
        err = hipErrorInvalidImage;
    // One small block: the error words at offsets 0, 64, 128 and 256
    // (separate lines), check_errors' readout at 192, the zero row at 320.
    constexpr size_t kFlagBlock = 320 + SGLKV_ZERO_ROW_BYTES;
    if (err == hipSuccess) err = hipMalloc(reinterpret_cast<void **>(&ctx->flag), kFlagBlock);
    if (err == hipSuccess) err = hipMemset(ctx->flag, 0, kFlagBlock);
    if (err == hipSuccess) {
        ctx->attn_flag = ctx->flag + 16;
        ctx->pair_flag = ctx->flag + 32;
        ctx->sync_attn_flag = ctx->flag + 64;
        ctx->zero_row = reinterpret_cast<const uint8_t *>(ctx->flag) + 320;
    }
    if (err != hipSuccess) {
        if (ctx->flag) (void)hipFree(ctx->flag);
        (void)hipModuleUnload(ctx->module);
        delete ctx;
        return hip_fail(err, "sgl_rocm_kv_init");
    }
    // The no-allocation entry point's workspace on this device, resolved
    // here once so that the entry point itself does no set-up.
    int32_t rc = noalloc_workspace(device, &ctx->noalloc_workspace, &ctx->noalloc_order);
    if (rc) {
        (void)hipFree(ctx->flag);
        (void)hipModuleUnload(ctx->module);
        delete ctx;
        return rc;
    }
    *out = ctx;
    return ok();
}

extern "C" int32_t sgl_rocm_kv_destroy(sgl_rocm_kv_ctx *ctx) {
    if (!ctx) return ok();
    DeviceScope scope(ctx->device);
    if (ctx->attention_partial) (void)hipFree(ctx->attention_partial);
    hipError_t e1 = hipFree(ctx->flag);
    hipError_t e2 = hipModuleUnload(ctx->module);
    delete ctx;
    if (e1 != hipSuccess) return hip_fail(e1, "hipFree");
    if (e2 != hipSuccess) return hip_fail(e2, "hipModuleUnload");
    return ok();
}

extern "C" int32_t sgl_rocm_kv_device(const sgl_rocm_kv_ctx *ctx) { return ctx ? ctx->device : -1; }

extern "C" int32_t sgl_rocm_kv_cu_count(const sgl_rocm_kv_ctx *ctx) { return ctx ? ctx->cu_count : 0; }

extern "C" int32_t sgl_rocm_kv_pair_scatter(sgl_rocm_kv_ctx *ctx, const sgl_kv_pair_copy_plan *plan,
                                            const sgl_kv_pair_copy_buffers *buffers, void *stream) {
    return pair_copy(ctx, plan, buffers, static_cast<hipStream_t>(stream), true);
}

extern "C" int32_t sgl_rocm_kv_pair_gather(sgl_rocm_kv_ctx *ctx, const sgl_kv_pair_copy_plan *plan,
                                           const sgl_kv_pair_copy_buffers *buffers, void *stream) {
    return pair_copy(ctx, plan, buffers, static_cast<hipStream_t>(stream), false);
}

namespace sglkv {

// Validates the last layer of a multi-layer launch (the first is validated
// by the caller) and that the destination's layers do not overlap.
int32_t check_layer_span(const sgl_kv_pool_view *pool, bool pool_is_dst,
                         const sgl_kv_rows_view *rows, const LayerSpan &span, uint64_t row_count,
                         const RowShape &shape, const sgl_kv_device_buffer *slots) {
    if (span.count == 0 || span.count > 65535)
        return fail(SGL_KV_INVALID_ARGUMENT, "layer_count", span.count, 65535, 0,
                    "a launch covers 1 to 65535 layers, not %u", span.count);
    if (span.count == 1) return SGL_KV_OK;
    const uint64_t n = span.count - 1;
    uint64_t pool_shift, rows_shift;
    if (mul_ovf(n, span.pool_stride, &pool_shift) || mul_ovf(n, span.rows_stride, &rows_shift))
        return shape_overflow();
    // The last layer, as a view of its own.
    sgl_kv_pool_view last_pool = *pool;
    for (uint32_t t = 0; t < pool->tensor_count; ++t)
        if (add_ovf(last_pool.tensor_offset[t], pool_shift, &last_pool.tensor_offset[t]))
            return shape_overflow();
    sgl_kv_rows_view last_rows = *rows;
    const char *names[2] = {shape.tensors == 2 ? "keys" : "rows", "values"};
    for (uint32_t t = 0; t < shape.tensors; ++t) {
        if (rows->plane_bytes[t] < rows_shift)
            return out_of_bounds(names[t], rows_shift, 0, rows->plane_bytes[t]);
        last_rows.planes[t] = static_cast<char *>(rows->planes[t]) + rows_shift;
        last_rows.plane_bytes[t] = rows->plane_bytes[t] - rows_shift;
    }
    sglkv_side scratch;
    int32_t rc;
    if ((rc = pool_side(&last_pool, slots, row_count, shape, &scratch)) ||
        (rc = rows_side(&last_rows, row_count, shape, names, &scratch)))
        return rc;
    // Layers written by the launch must not overlap one another.
    uint64_t lo = UINT64_MAX, hi = 0;
    if (pool_is_dst) {
        for (uint32_t t = 0; t < pool->tensor_count; ++t) {
            lo = pool->tensor_offset[t] < lo ? pool->tensor_offset[t] : lo;
            const uint64_t end = pool->tensor_offset[t] + pool->page_size * view_row_bytes(*pool, t);
            hi = end > hi ? end : hi;
        }
        if (span.pool_stride < hi - lo)
            return fail(SGL_KV_INVALID_ARGUMENT, "pool_layer_stride", span.pool_stride, hi - lo, 0,
                        "destination layers %llu bytes apart overlap their %llu-byte regions",
                        (unsigned long long)span.pool_stride, (unsigned long long)(hi - lo));
    } else {
        for (uint32_t t = 0; t < shape.tensors; ++t) {
            const uint64_t b = (uint64_t)(uintptr_t)rows->planes[t];
            const uint64_t end = b + (row_count - 1) * rows->row_stride[t] + shape.row_bytes[t];
            lo = b < lo ? b : lo;
            hi = end > hi ? end : hi;
        }
        if (span.rows_stride < hi - lo)
            return fail(SGL_KV_INVALID_ARGUMENT, "rows_layer_stride", span.rows_stride, hi - lo, 0,
                        "destination layers %llu bytes apart overlap their %llu-byte rows",
                        (unsigned long long)span.rows_stride, (unsigned long long)(hi - lo));
    }
    return SGL_KV_OK;
}

int32_t prepare_pack(const sgl_rocm_kv_ctx *ctx, const sgl_kv_pool_view *src,
                     const sgl_kv_device_buffer *slots, uint64_t row_count,
                     const sgl_kv_rows_view *dst, Launch *l, LayerSpan span) {
    // Row counts are checked first: the limit holds whatever the context.
    if (row_count > kMaxRows) return too_large("row_count", row_count, kMaxRows);
    int32_t rc = check_ctx(ctx);
    if (!rc) rc = check_pool_shape(src);
    if (rc) return rc;
    if (!dst) return fail(SGL_KV_INVALID_ARGUMENT, "rows", 0, 0, 0, "null rows view");
    memset(l, 0, sizeof *l);
    l->kind = kPoolRows;
    l->rows = row_count;
    l->layers = span.count;
    if (row_count == 0) return SGL_KV_OK;
    const bool split = src->head_layout == SGL_KV_HND;
    l->shape = shape_of(*src, split, src->heads);
    const char *names[2] = {src->tensor_count == 2 ? "keys" : "rows", "values"};
    if ((rc = pool_side(src, slots, row_count, l->shape, &l->params.src)) ||
        (rc = rows_side(dst, row_count, l->shape, names, &l->params.dst)) ||
        (rc = check_layer_span(src, false, dst, span, row_count, l->shape, slots)))
        return rc;
    l->params.src.layer_stride = span.pool_stride;
    l->params.dst.layer_stride = span.rows_stride;
    attach_scales(l->params, src->scale, dst->scale, src->tensor_count);
    return finish_launch(ctx, l);
}

int32_t prepare_unpack(const sgl_rocm_kv_ctx *ctx, const sgl_kv_rows_view *src, uint64_t row_count,
                       const sgl_kv_pool_view *dst, const sgl_kv_device_buffer *slots, Launch *l,
                       LayerSpan span) {
    // Row counts are checked first: the limit holds whatever the context.
    if (row_count > kMaxRows) return too_large("row_count", row_count, kMaxRows);
    int32_t rc = check_ctx(ctx);
    if (!rc) rc = check_pool_shape(dst);
    if (rc) return rc;
    if (!src) return fail(SGL_KV_INVALID_ARGUMENT, "rows", 0, 0, 0, "null rows view");
    memset(l, 0, sizeof *l);
    l->kind = kRowsPool;
    l->rows = row_count;
    l->layers = span.count;
    if (row_count == 0) return SGL_KV_OK;
    const bool split = dst->head_layout == SGL_KV_HND;
    l->shape = shape_of(*dst, split, dst->heads);
    const char *names[2] = {dst->tensor_count == 2 ? "keys" : "rows", "values"};
    if ((rc = rows_side(src, row_count, l->shape, names, &l->params.src)) ||
        (rc = pool_side(dst, slots, row_count, l->shape, &l->params.dst)) ||
        (rc = check_layer_span(dst, true, src, span, row_count, l->shape, slots)))
        return rc;
    l->params.src.layer_stride = span.rows_stride;
    l->params.dst.layer_stride = span.pool_stride;
    attach_scales(l->params, src->scale, dst->scale, dst->tensor_count);
    return finish_launch(ctx, l);
}

int32_t submit_launch(sgl_rocm_kv_ctx *ctx, Launch &l, hipStream_t stream) {
    if (l.rows == 0) return SGL_KV_OK;
    if (l.realigned) {
        void *args[] = {&l.realign};
        SGLKV_HIP(hipModuleLaunchKernel(ctx->realign[l.kind], (unsigned)l.grid, l.layers ? l.layers : 1, 1,
                                        l.block_x, l.block_y, 1, l.lds_bytes, stream, args, nullptr));
        return SGL_KV_OK;
    }
    void *args[] = {&l.params};
    SGLKV_HIP(hipModuleLaunchKernel(ctx->copy[l.width_index][l.kind], (unsigned)l.grid,
                                    l.layers ? l.layers : 1, 1, l.block_x, l.block_y, 1, 0, stream,
                                    args, nullptr));
    return SGL_KV_OK;
}

}  // namespace sglkv

extern "C" int32_t sgl_rocm_kv_pack_layer(sgl_rocm_kv_ctx *ctx, const sgl_kv_pool_view *src,
                                          const sgl_kv_device_buffer *slots, uint64_t row_count,
                                          const sgl_kv_rows_view *dst, void *stream) {
    Launch l;
    int32_t rc = prepare_pack(ctx, src, slots, row_count, dst, &l);
    if (rc) return rc;
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    rc = submit_launch(ctx, l, static_cast<hipStream_t>(stream));
    return rc ? rc : ok();
}

extern "C" int32_t sgl_rocm_kv_unpack_layer(sgl_rocm_kv_ctx *ctx, const sgl_kv_rows_view *src,
                                            uint64_t row_count, const sgl_kv_pool_view *dst,
                                            const sgl_kv_device_buffer *slots, void *stream) {
    Launch l;
    int32_t rc = prepare_unpack(ctx, src, row_count, dst, slots, &l);
    if (rc) return rc;
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    rc = submit_launch(ctx, l, static_cast<hipStream_t>(stream));
    return rc ? rc : ok();
}

extern "C" int32_t sgl_rocm_kv_pack_layers(sgl_rocm_kv_ctx *ctx, const sgl_kv_pool_view *src,
                                           uint64_t pool_layer_stride, uint32_t layer_count,
                                           const sgl_kv_device_buffer *slots, uint64_t row_count,
                                           const sgl_kv_rows_view *dst, uint64_t rows_layer_stride,
                                           void *stream) {
    Launch l;
    int32_t rc = prepare_pack(ctx, src, slots, row_count, dst, &l,
                              LayerSpan{layer_count, pool_layer_stride, rows_layer_stride});
    if (rc) return rc;
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    rc = submit_launch(ctx, l, static_cast<hipStream_t>(stream));
    return rc ? rc : ok();
}

extern "C" int32_t sgl_rocm_kv_unpack_layers(sgl_rocm_kv_ctx *ctx, const sgl_kv_rows_view *src,
                                             uint64_t rows_layer_stride, uint32_t layer_count,
                                             uint64_t row_count, const sgl_kv_pool_view *dst,
                                             uint64_t pool_layer_stride,
                                             const sgl_kv_device_buffer *slots, void *stream) {
    Launch l;
    int32_t rc = prepare_unpack(ctx, src, row_count, dst, slots, &l,
                                LayerSpan{layer_count, pool_layer_stride, rows_layer_stride});
    if (rc) return rc;
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    rc = submit_launch(ctx, l, static_cast<hipStream_t>(stream));
    return rc ? rc : ok();
}

namespace {

// One tensor of one layer, `count` slots, between a pool described by its
// PagedKvCacheLayout and strided rows: the batched form of
// CudaKvStorage::write_tensor_slot_from_device / read_tensor_slot_to_device
// (cuda_kv_cache.rs:258-294), which copy one slot per cuMemcpyDtoD (the MLA
// forward pass calls them per token, cuda_mla.rs:256-271).
int32_t tensor_slots(sgl_rocm_kv_ctx *ctx, const sgl_kv_paged_layout *layout,
                     const sgl_kv_device_buffer *pool, uint64_t layer, uint64_t tensor,
                     const sgl_kv_device_buffer *slots, uint64_t count,
                     const sgl_kv_device_buffer *rows, uint64_t rows_offset, uint64_t rows_stride,
                     bool write, void *stream) {
    int32_t rc = check_ctx(ctx);
    if (rc) return rc;
    if (!layout || !pool || !rows)
        return fail(SGL_KV_INVALID_ARGUMENT, "layout/pool/rows", 0, 0, 0, "null argument");
    if (pool->byte_len < layout->total_byte_len)
        return out_of_bounds("pool", 0, layout->total_byte_len, pool->byte_len);
    sgl_kv_pool_view v;
    if ((rc = sgl_kv_pool_view_for_layer(layout, pool->ptr, pool->byte_len, SGL_KV_NHD, 1, layer,
                                         tensor, 1, &v)))
        return rc;
    if (rows_offset > rows->byte_len) return out_of_bounds(write ? "source" : "destination",
                                                           rows_offset, 0, rows->byte_len);
    sgl_kv_rows_view r;
    memset(&r, 0, sizeof r);
    r.planes[0] = rows->ptr ? static_cast<char *>(rows->ptr) + rows_offset : nullptr;
    r.plane_bytes[0] = rows->byte_len - rows_offset;
    r.row_stride[0] = rows_stride;
    Launch l;
    rc = write ? prepare_unpack(ctx, &r, count, &v, slots, &l) : prepare_pack(ctx, &v, slots, count, &r, &l);
    if (rc) return rc;
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    rc = submit_launch(ctx, l, static_cast<hipStream_t>(stream));
    return rc ? rc : ok();
}

}  // namespace

extern "C" int32_t sgl_rocm_kv_write_tensor_slots(sgl_rocm_kv_ctx *ctx, const sgl_kv_paged_layout *layout,
                                                  const sgl_kv_device_buffer *pool, uint64_t layer,
                                                  uint64_t tensor, const sgl_kv_device_buffer *slots,
                                                  uint64_t count, const sgl_kv_device_buffer *source,
                                                  uint64_t source_offset, uint64_t source_row_stride,
                                                  void *stream) {
    return tensor_slots(ctx, layout, pool, layer, tensor, slots, count, source, source_offset,
                        source_row_stride, true, stream);
}

extern "C" int32_t sgl_rocm_kv_write_tensor_pair_slots(
    sgl_rocm_kv_ctx *ctx, const sgl_kv_paged_layout *layout, const sgl_kv_device_buffer *pool, uint64_t layer,
    const sgl_kv_device_buffer *slots, uint64_t count, const sgl_kv_device_buffer *keys, uint64_t keys_offset,
    uint64_t keys_row_stride, const sgl_kv_device_buffer *values, uint64_t values_offset,
    uint64_t values_row_stride, void *stream) {
    int32_t rc = check_ctx(ctx);
    if (rc) return rc;
    if (!layout || !pool || !slots || !keys || !values)
        return fail(SGL_KV_INVALID_ARGUMENT, "layout/pool/slot_indices/keys/values", 0, 0, 0, "null argument");
    if (pool->byte_len < layout->total_byte_len)
        return out_of_bounds("pool", 0, layout->total_byte_len, pool->byte_len);
    sgl_kv_pool_view v[2];
    for (uint32_t t = 0; t < 2; ++t)
        if ((rc = sgl_kv_pool_view_for_layer(layout, pool->ptr, pool->byte_len, SGL_KV_NHD, 1, layer, t, 1,
                                             &v[t])))
            return rc;
    if (count == 0) return ok();
    if (!pool->ptr) return fail(SGL_KV_INVALID_ARGUMENT, "pool", 0, 0, 0, "null pool");
    if (!slots->ptr) return fail(SGL_KV_INVALID_ARGUMENT, "slot_indices", 0, 0, 0, "null slot map");
    uint64_t need;
    if (mul_ovf(count, sizeof(uint64_t), &need)) return shape_overflow();
    if (need > slots->byte_len) return out_of_bounds("slot_indices", 0, need, slots->byte_len);
    const sgl_kv_device_buffer *rows[2] = {keys, values};
    const uint64_t offs[2] = {keys_offset, values_offset}, strides[2] = {keys_row_stride, values_row_stride};
    const char *const names[2] = {"keys", "values"};
    sglkv_pair_slots_params p;
    memset(&p, 0, sizeof p);
    uint64_t bits = (uint64_t)(uintptr_t)pool->ptr | v[0].page_stride_bytes;
    for (uint32_t t = 0; t < 2; ++t) {
        if (!rows[t]->ptr) return fail(SGL_KV_INVALID_ARGUMENT, names[t], 0, 0, 0, "null rows");
        if (strides[t] < v[t].row_bytes)
            return fail(SGL_KV_ROW_STRIDE_TOO_SMALL, names[t], v[t].row_bytes, strides[t], 0,
                        "KV copy %s row stride %llu bytes is smaller than row width %llu bytes", names[t],
                        (unsigned long long)strides[t], (unsigned long long)v[t].row_bytes);
        if (mul_ovf(count - 1, strides[t], &need) || add_ovf(need, v[t].row_bytes, &need) ||
            add_ovf(need, offs[t], &need))
            return shape_overflow();
        if (need > rows[t]->byte_len) return out_of_bounds(names[t], offs[t], need - offs[t], rows[t]->byte_len);
        p.offset[t] = v[t].tensor_offset[0];
        p.row_bytes[t] = v[t].row_bytes;
        p.rows[t] = static_cast<const uint8_t *>(rows[t]->ptr) + offs[t];
        p.row_stride[t] = strides[t];
        bits |= p.offset[t] | p.row_bytes[t] | (uint64_t)(uintptr_t)p.rows[t] | p.row_stride[t];
    }
    const uint32_t w = (bits & 15u) == 0 ? 16u : 1u;
    p.slots = static_cast<const uint64_t *>(slots->ptr);
    p.count = count;
    p.pool = static_cast<uint8_t *>(pool->ptr);
    p.page_size = v[0].page_size;
    p.page_stride = v[0].page_stride_bytes;
    if (mul_ovf(v[0].page_size, v[0].page_count, &p.slot_count)) return shape_overflow();
    p.pieces[0] = p.row_bytes[0] / w;
    p.pieces[1] = p.row_bytes[1] / w;
    p.flag = ctx->flag;
    uint64_t threads;
    if (mul_ovf(count, p.pieces[0] + p.pieces[1], &threads)) return shape_overflow();
    const uint64_t grid = threads / SGLKV_BLOCK_THREADS + (threads % SGLKV_BLOCK_THREADS ? 1 : 0);
    if (grid > INT32_MAX) return too_large("grid blocks", grid, INT32_MAX);
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    void *args[] = {&p};
    SGLKV_HIP(hipModuleLaunchKernel(ctx->pair_slots[w == 16 ? 0 : 1], (unsigned)grid, 1, 1, SGLKV_BLOCK_THREADS,
                                    1, 1, 0, static_cast<hipStream_t>(stream), args, nullptr));
    return ok();
}

extern "C" int32_t sgl_rocm_kv_read_tensor_slots(sgl_rocm_kv_ctx *ctx, const sgl_kv_paged_layout *layout,
                                                 const sgl_kv_device_buffer *pool, uint64_t layer,
                                                 uint64_t tensor, const sgl_kv_device_buffer *slots,
                                                 uint64_t count, const sgl_kv_device_buffer *destination,
                                                 uint64_t destination_offset,
                                                 uint64_t destination_row_stride, void *stream) {
    return tensor_slots(ctx, layout, pool, layer, tensor, slots, count, destination,
                        destination_offset, destination_row_stride, false, stream);
}

namespace sglkv {

// Pool -> pool over `layers` consecutive layers (layer i of a side: its
// view with every tensor offset advanced by i * stride).
int32_t prepare_transfer(const sgl_rocm_kv_ctx *ctx, const sgl_kv_pool_view *src,
                         const sgl_kv_device_buffer *src_slots, uint64_t row_count,
                         const sgl_kv_pool_view *dst, const sgl_kv_device_buffer *dst_slots,
                         Launch *l, uint32_t layers, uint64_t src_layer_stride,
                         uint64_t dst_layer_stride) {
    if (row_count > kMaxRows) return too_large("row_count", row_count, kMaxRows);
    int32_t rc = check_ctx(ctx);
    if (!rc) rc = check_pool_shape(src);
    if (!rc) rc = check_pool_shape(dst);
    if (rc) return rc;
    if (src->tensor_count != dst->tensor_count || src->row_bytes != dst->row_bytes ||
        view_row_bytes(*src, 1) != view_row_bytes(*dst, 1))
        return fail(SGL_KV_INVALID_ARGUMENT, "dst", dst->row_bytes, src->row_bytes, 0,
                    "destination rows (%llu + %llu bytes x %u tensors) differ from source rows "
                    "(%llu + %llu x %u)",
                    (unsigned long long)dst->row_bytes, (unsigned long long)view_row_bytes(*dst, 1),
                    dst->tensor_count, (unsigned long long)src->row_bytes,
                    (unsigned long long)view_row_bytes(*src, 1), src->tensor_count);
    const bool split = src->head_layout == SGL_KV_HND || dst->head_layout == SGL_KV_HND;
    if (split && src->heads != dst->heads)
        return fail(SGL_KV_INVALID_ARGUMENT, "heads", dst->heads, src->heads, 0,
                    "head-major relayout needs equal head counts (%u vs %u)", dst->heads, src->heads);
    for (uint32_t t = 0; t < src->tensor_count; ++t)
        if (split && view_row_bytes(*src, t) % src->heads)
            return fail(SGL_KV_INVALID_ARGUMENT, "heads", src->heads, view_row_bytes(*src, t), 0,
                        "%u heads do not split a %llu-byte row evenly", src->heads,
                        (unsigned long long)view_row_bytes(*src, t));
    if (layers == 0 || layers > 65535)
        return fail(SGL_KV_INVALID_ARGUMENT, "layer_count", layers, 65535, 0,
                    "a launch covers 1 to 65535 layers, not %u", layers);
    memset(l, 0, sizeof *l);
    l->kind = kPoolPool;
    l->rows = row_count;
    l->layers = layers;
    if (row_count == 0) return SGL_KV_OK;
    l->shape = shape_of(*src, split, src->heads);
    if ((rc = pool_side(src, src_slots, row_count, l->shape, &l->params.src)) ||
        (rc = pool_side(dst, dst_slots, row_count, l->shape, &l->params.dst)))
        return rc;
    if (layers > 1) {
        // The last layer of each side, as views of their own.
        sgl_kv_pool_view last[2] = {*src, *dst};
        const uint64_t strides[2] = {src_layer_stride, dst_layer_stride};
        const sgl_kv_device_buffer *slots[2] = {src_slots, dst_slots};
        sglkv_side scratch;
        for (int side = 0; side < 2; ++side) {
            uint64_t shift;
            if (mul_ovf(layers - 1, strides[side], &shift)) return shape_overflow();
            for (uint32_t t = 0; t < last[side].tensor_count; ++t)
                if (add_ovf(last[side].tensor_offset[t], shift, &last[side].tensor_offset[t]))
                    return shape_overflow();
            if ((rc = pool_side(&last[side], slots[side], row_count, l->shape, &scratch))) return rc;
        }
        uint64_t lo = UINT64_MAX, hi = 0;
        for (uint32_t t = 0; t < dst->tensor_count; ++t) {
            lo = dst->tensor_offset[t] < lo ? dst->tensor_offset[t] : lo;
            const uint64_t end = dst->tensor_offset[t] + dst->page_size * view_row_bytes(*dst, t);
            hi = end > hi ? end : hi;
        }
        if (dst_layer_stride < hi - lo)
            return fail(SGL_KV_INVALID_ARGUMENT, "dst_layer_stride", dst_layer_stride, hi - lo, 0,
                        "destination layers %llu bytes apart overlap their %llu-byte regions",
                        (unsigned long long)dst_layer_stride, (unsigned long long)(hi - lo));
    }
    l->params.src.layer_stride = src_layer_stride;
    l->params.dst.layer_stride = dst_layer_stride;
    attach_scales(l->params, src->scale, dst->scale, src->tensor_count);
    return finish_launch(ctx, l);
}

}  // namespace sglkv

extern "C" int32_t sgl_rocm_kv_transfer_layer(sgl_rocm_kv_ctx *ctx, const sgl_kv_pool_view *src,
                                              const sgl_kv_device_buffer *src_slots,
                                              uint64_t row_count, const sgl_kv_pool_view *dst,
                                              const sgl_kv_device_buffer *dst_slots, void *stream) {
    return sgl_rocm_kv_transfer_layers(ctx, src, 0, 1, src_slots, row_count, dst, 0, dst_slots, stream);
}

extern "C" int32_t sgl_rocm_kv_transfer_layers(sgl_rocm_kv_ctx *ctx, const sgl_kv_pool_view *src,
                                               uint64_t src_layer_stride, uint32_t layer_count,
                                               const sgl_kv_device_buffer *src_slots,
                                               uint64_t row_count, const sgl_kv_pool_view *dst,
                                               uint64_t dst_layer_stride,
                                               const sgl_kv_device_buffer *dst_slots, void *stream) {
    Launch l;
    int32_t rc = prepare_transfer(ctx, src, src_slots, row_count, dst, dst_slots, &l, layer_count,
                                  src_layer_stride, dst_layer_stride);
    if (rc) return rc;
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    rc = submit_launch(ctx, l, static_cast<hipStream_t>(stream));
    return rc ? rc : ok();
}

extern "C" int32_t sgl_rocm_kv_resolve_spans(sgl_rocm_kv_ctx *ctx, uint64_t page_size,
                                             uint64_t page_count, const sgl_kv_device_buffer *spans,
                                             uint64_t span_count,
                                             const sgl_kv_device_buffer *page_table,
                                             uint64_t page_table_len, uint64_t row_count,
                                             const sgl_kv_device_buffer *out_slots, void *stream) {
    int32_t rc = check_ctx(ctx);
    if (rc) return rc;
    if (page_size == 0) return fail(SGL_KV_ZERO_DIMENSION, "page_size", 0, 0, 0, "KV copy dimension page_size must be non-zero");
    if (page_size > UINT32_MAX) return too_large("page_size", page_size, UINT32_MAX);
    if (span_count > UINT32_MAX) return too_large("span_count", span_count, UINT32_MAX);
    if (row_count > UINT32_MAX) return too_large("row_count", row_count, UINT32_MAX);
    if (row_count == 0) return ok();
    if (!spans || !page_table || !out_slots || !out_slots->ptr || (span_count && !spans->ptr) ||
        (page_table_len && !page_table->ptr))
        return fail(SGL_KV_INVALID_ARGUMENT, "spans/page_table/out_slots", 0, 0, 0, "null buffer");
    uint64_t need;
    if (mul_ovf(span_count, sizeof(sgl_kv_span), &need)) return shape_overflow();
    if (need > spans->byte_len) return out_of_bounds("spans", 0, need, spans->byte_len);
    if (mul_ovf(page_table_len, 4, &need)) return shape_overflow();
    if (need > page_table->byte_len) return out_of_bounds("page_table", 0, need, page_table->byte_len);
    if (mul_ovf(row_count, 8, &need)) return shape_overflow();
    if (need > out_slots->byte_len) return out_of_bounds("out_slots", 0, need, out_slots->byte_len);
    static_assert(sizeof(sgl_kv_span) == sizeof(sglkv_span), "span layouts differ");
    sglkv_resolve_params p;
    memset(&p, 0, sizeof p);
    p.spans = static_cast<const sglkv_span *>(spans->ptr);
    p.page_table = static_cast<const int32_t *>(page_table->ptr);
    p.out_slots = static_cast<uint64_t *>(out_slots->ptr);
    p.flag = ctx->flag;
    p.page_table_len = page_table_len;
    p.page_count = page_count;
    p.span_count = (uint32_t)span_count;
    p.page_size = (uint32_t)page_size;
    p.rows = (uint32_t)row_count;
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    void *args[] = {&p};
    const uint64_t grid = (row_count + SGLKV_BLOCK_THREADS - 1) / SGLKV_BLOCK_THREADS;
    SGLKV_HIP(hipModuleLaunchKernel(ctx->resolve, (unsigned)grid, 1, 1, SGLKV_BLOCK_THREADS, 1, 1, 0,
                                    static_cast<hipStream_t>(stream), args, nullptr));
    return ok();
}

// Maps the device error word to the status (and detail record) it reports.
// Span resolution's bits come first: a row it could not resolve also
// reaches the copies as a bad slot, and the page table is the cause.
int32_t sglkv::flag_status(uint32_t flag) {
    if (flag & SGLKV_FLAG_PAGE)
        return fail(SGL_KV_DEVICE_PAGE_INDEX_OUT_OF_RANGE, nullptr, 0, flag, 0,
                    "KV transfer page table holds an entry outside the table or the pool");
    if (flag & SGLKV_FLAG_SPAN)
        return fail(SGL_KV_DEVICE_SPAN_OUT_OF_RANGE, nullptr, 0, flag, 0,
                    "KV transfer row is not covered by any span");
    if (flag & SGLKV_FLAG_SLOT)
        return fail(SGL_KV_DEVICE_SLOT_INDEX_OUT_OF_RANGE, nullptr, 0, flag, 0,
                    "KV copy device slot map contains an index outside the pool's slots");
    if (flag & SGLKV_FLAG_REQUEST)
        return fail(SGL_KV_DEVICE_REQUEST_OUT_OF_RANGE, nullptr, 0, flag, 0,
                    "KV page request lies outside its source or target region");
    return attention_flag_status(flag);
}

extern "C" int32_t sgl_rocm_kv_check_errors(sgl_rocm_kv_ctx *ctx, void *stream) {
    int32_t rc = check_ctx(ctx);
    if (rc) return rc;
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    hipStream_t s = static_cast<hipStream_t>(stream);
    // The copy word and the attention word (the asynchronous attention's
    // metadata errors surface here too), each read and cleared atomically
    // on `stream` after the work queued there.
    uint32_t *out = ctx->flag + 48;
    void *args[] = {&ctx->flag, &ctx->attn_flag, &out};
    SGLKV_HIP(hipModuleLaunchKernel(ctx->take_flags, 1, 1, 1, 64, 1, 1, 0, s, args, nullptr));
    uint32_t flags[2] = {0, 0};
    SGLKV_HIP(hipMemcpyAsync(flags, out, sizeof flags, hipMemcpyDeviceToHost, s));
    SGLKV_HIP(hipStreamSynchronize(s));
    return flag_status(flags[0] | flags[1]);
}

extern "C" int32_t sgl_rocm_kv_fill_synthetic(sgl_rocm_kv_ctx *ctx, const sgl_kv_device_buffer *buffer,
                                              uint64_t seed, uint32_t kind, void *stream) {
    int32_t rc = check_ctx(ctx);
    if (rc) return rc;
    if (!buffer || !buffer->ptr) return fail(SGL_KV_INVALID_ARGUMENT, "buffer", 0, 0, 0, "null buffer");
    if (buffer->byte_len % 8)
        return fail(SGL_KV_INVALID_ARGUMENT, "buffer", buffer->byte_len, 8, 0,
                    "fill length %llu is not a multiple of 8 bytes",
                    (unsigned long long)buffer->byte_len);
    if (kind > SGL_KV_FILL_BF16_UNIFORM)
        return fail(SGL_KV_INVALID_ARGUMENT, "kind", kind, 0, 0, "unknown fill kind %u", kind);
    uint64_t words = buffer->byte_len / 8;
    if (words == 0) return ok();
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    uint64_t blocks = (words + SGLKV_BLOCK_THREADS - 1) / SGLKV_BLOCK_THREADS;
    const uint64_t cap = (uint64_t)(ctx->cu_count > 0 ? ctx->cu_count : 1) * 32;
    if (blocks > cap) blocks = cap;
    void *ptr = buffer->ptr;
    void *args[] = {&ptr, &words, &seed, &kind};
    SGLKV_HIP(hipModuleLaunchKernel(ctx->fill, (unsigned)blocks, 1, 1, SGLKV_BLOCK_THREADS, 1, 1, 0,
                                    static_cast<hipStream_t>(stream), args, nullptr));
    return ok();
}

extern "C" int32_t sgl_rocm_kv_stream(sgl_rocm_kv_ctx *ctx, uint32_t kind, const sgl_kv_device_buffer *src,
                                      const sgl_kv_device_buffer *dst, uint64_t bytes, void *stream) {
    int32_t rc = check_ctx(ctx);
    if (rc) return rc;
    if (kind > SGL_KV_STREAM_WRITE) return fail(SGL_KV_INVALID_ARGUMENT, "kind", kind, 0, 0, "unknown stream kind %u", kind);
    if (bytes % 16)
        return fail(SGL_KV_INVALID_ARGUMENT, "bytes", bytes, 16, 0, "stream length %llu is not a multiple of 16 bytes",
                    (unsigned long long)bytes);
    // copy and read need the source; copy and write need `bytes` of
    // destination, read needs 16 (its keep-alive store).
    const uint64_t need_dst = kind == SGL_KV_STREAM_READ ? 16 : bytes;
    if (kind != SGL_KV_STREAM_WRITE && (!src || !src->ptr || src->byte_len < bytes))
        return fail(SGL_KV_ALLOCATION_OUT_OF_BOUNDS, "src", 0, bytes, src ? src->byte_len : 0,
                    "stream source shorter than %llu bytes", (unsigned long long)bytes);
    if (!dst || !dst->ptr || dst->byte_len < need_dst)
        return fail(SGL_KV_ALLOCATION_OUT_OF_BOUNDS, "dst", 0, need_dst, dst ? dst->byte_len : 0,
                    "stream destination shorter than %llu bytes", (unsigned long long)need_dst);
    if (bytes == 0) return ok();
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    // Workgroups per CU of the fastest settings measured: 16 for the copy, 8
    // for the read and the write.
    const uint64_t cus = (uint64_t)(ctx->cu_count > 0 ? ctx->cu_count : 256);
    const unsigned blocks = (unsigned)((kind == SGL_KV_STREAM_COPY ? 16 : 8) * cus);
    const void *s = kind == SGL_KV_STREAM_WRITE ? dst->ptr : src->ptr;
    void *d = dst->ptr;
    uint64_t vecs = bytes / 16;
    void *args[] = {&s, &d, &vecs};
    SGLKV_HIP(hipModuleLaunchKernel(ctx->stream_fn[kind], blocks, 1, 1, SGLKV_BLOCK_THREADS, 1, 1, 0,
                                    static_cast<hipStream_t>(stream), args, nullptr));
    return ok();
}

extern "C" int32_t sgl_rocm_kv_execute_page_requests(sgl_rocm_kv_ctx *ctx,
                                                     const sgl_kv_device_buffer *requests,
                                                     uint64_t count, uint64_t max_length,
                                                     const sgl_kv_device_buffer *source_region,
                                                     const sgl_kv_device_buffer *target_region,
                                                     uint32_t offsets_are_addresses, void *stream) {
    int32_t rc = check_ctx(ctx);
    if (rc) return rc;
    if (count == 0) return ok();
    if (!requests || !requests->ptr || !source_region || !source_region->ptr || !target_region ||
        !target_region->ptr)
        return fail(SGL_KV_INVALID_ARGUMENT, "requests/source_region/target_region", 0, 0, 0,
                    "null buffer");
    static_assert(sizeof(sgl_kv_page_request) == sizeof(sglkv_request), "request layouts differ");
    uint64_t need;
    if (mul_ovf(count, sizeof(sglkv_request), &need)) return shape_overflow();
    if (need > requests->byte_len) return out_of_bounds("requests", 0, need, requests->byte_len);
    if (max_length == 0) return fail(SGL_KV_ZERO_DIMENSION, "max_length", 0, 0, 0,
                                     "KV copy dimension max_length must be non-zero");
    const uint64_t chunks = max_length / SGLKV_REQUEST_CHUNK + (max_length % SGLKV_REQUEST_CHUNK ? 1 : 0);
    uint64_t grid;
    if (mul_ovf(count, chunks, &grid) || grid > INT32_MAX) return too_large("grid blocks", grid, INT32_MAX);
    sglkv_request_params p;
    memset(&p, 0, sizeof p);
    p.requests = static_cast<const sglkv_request *>(requests->ptr);
    p.flag = ctx->flag;
    p.count = count;
    p.chunks = chunks;
    p.source_lo = (uint64_t)(uintptr_t)source_region->ptr;
    p.target_lo = (uint64_t)(uintptr_t)target_region->ptr;
    if (add_ovf(p.source_lo, source_region->byte_len, &p.source_hi) ||
        add_ovf(p.target_lo, target_region->byte_len, &p.target_hi))
        return shape_overflow();
    p.target_base = offsets_are_addresses ? 0 : p.target_lo;
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    void *args[] = {&p};
    SGLKV_HIP(hipModuleLaunchKernel(ctx->requests, (unsigned)grid, 1, 1, SGLKV_BLOCK_THREADS, 1, 1, 0,
                                    static_cast<hipStream_t>(stream), args, nullptr));
    return ok();
}
