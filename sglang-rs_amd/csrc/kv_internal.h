// kv_internal.h -- helpers shared by the host sources of libsgl_rocm_kv.
#ifndef SGLKV_INTERNAL_H
#define SGLKV_INTERNAL_H

#include <stdint.h>

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

inline bool mul_ovf(uint64_t a, uint64_t b, uint64_t *out) { return __builtin_mul_overflow(a, b, out); }
inline bool add_ovf(uint64_t a, uint64_t b, uint64_t *out) { return __builtin_add_overflow(a, b, out); }

}  // namespace sglkv

#endif
