// Host-side helpers of the C ABI: thread-local error message, argument checks, launch checks.
#pragma once
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "sisa_hip.h"

namespace sisa {

void set_error(const char* fmt, ...);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int elem_size(int dtype) {
    switch (dtype) {
        case SISA_F32: return 4;
        case SISA_BF16: return 2;
        case SISA_F16: return 2;
        case SISA_F64: return 8;
        default: return 0;
    }
}

// A (B,H,L,w) view whose rows can be read with 16-byte vector loads.
inline bool view_ok(const sisa_view& v, int dtype) {
    const int es = elem_size(dtype);
    if (!v.ptr || es == 0) return false;
    if (!aligned16(v.ptr)) return false;
    return (v.sb * es) % 16 == 0 && (v.sh * es) % 16 == 0 && (v.sl * es) % 16 == 0;
}

inline int launch_status(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("%s: launch failed: %s", what, hipGetErrorString(e));
        return SISA_ERR_LAUNCH;
    }
    return SISA_OK;
}

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace sisa

#define SISA_REQUIRE(cond, ...)                     \
    do {                                            \
        if (!(cond)) {                              \
            ::sisa::set_error(__VA_ARGS__);         \
            return SISA_ERR_INVALID;                \
        }                                           \
    } while (0)
