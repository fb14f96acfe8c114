// kv_scratch.hip -- the device workspace of the entry point that allocates
// nothing (sgl_rocm_kv_paged_attention_async_noalloc): a file-scope device
// array that the HIP runtime places on every device the library runs on when
// this object's code is loaded there, and keeps until the process ends.
//
// Built by hipcc (host and gfx950 device code) and linked into
// libsgl_rocm_kv.so beside the host sources. The array's name is only a
// host-side handle: its device address, which differs per device, comes from
// hipGetSymbolAddress with that device current, once per device, at context
// set-up (sgl_rocm_kv_init); host code only ever passes that address on.
#include <hip/hip_runtime.h>

#include <mutex>

#include "kv_internal.h"

namespace {

static __device__ __align__(256) uint8_t scratch[SGL_KV_NOALLOC_WORKSPACE_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_lock;
void *g_address[kMaxDevices];
sglkv::NoallocOrder g_order[kMaxDevices];

}  // namespace

int32_t sglkv::noalloc_workspace(int device, void **out, NoallocOrder **order) {
    *out = nullptr;
    *order = nullptr;
    if (device < 0 || device >= kMaxDevices)
        return fail(SGL_KV_INVALID_ARGUMENT, "device", (uint64_t)(int64_t)device, kMaxDevices, 0,
                    "device %d is past the %d devices the workspace table covers", device, kMaxDevices);
    std::lock_guard<std::mutex> guard(g_lock);
    if (!g_address[device]) {
        DeviceScope scope(device);
        if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
        void *ptr = nullptr;
        const hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (err != hipSuccess) return hip_fail(err, "hipGetSymbolAddress");
        if (!ptr) return fail(SGL_KV_MODULE, "hipGetSymbolAddress", 0, 0, 0, "the workspace has no device address");
        // The ordering event, created once here so that the entry point
        // itself creates nothing; kept, like the workspace, until the
        // process ends.
        hipEvent_t last = nullptr;
        const hipError_t eerr = hipEventCreateWithFlags(&last, hipEventDisableTiming);
        if (eerr != hipSuccess) return hip_fail(eerr, "hipEventCreateWithFlags");
        g_order[device].last = last;
        g_address[device] = ptr;
    }
    *out = g_address[device];
    *order = &g_order[device];
    return SGL_KV_OK;
}
