// Shared helpers for the molnex HIP library (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/molnex.h"

namespace mnx {

// Records a formatted message as the thread's last error and returns `code`.
int set_error(int code, const char* fmt, ...);
void clear_error();

#define MNX_HIP_TRY(expr)                                                             \
    do {                                                                              \
        hipError_t _e = (expr);                                                       \
        if (_e != hipSuccess)                                                         \
            return ::mnx::set_error(MNX_ERR_HIP, "%s failed: %s (%s:%d)", #expr,      \
                                    hipGetErrorString(_e), __FILE__, __LINE__);       \
    } while (0)

#define MNX_CHECK_LAUNCH()                                                            \
    do {                                                                              \
        hipError_t _e = hipGetLastError();                                            \
        if (_e != hipSuccess)                                                         \
            return ::mnx::set_error(MNX_ERR_HIP, "kernel launch failed: %s (%s:%d)",  \
                                    hipGetErrorString(_e), __FILE__, __LINE__);       \
    } while (0)

#define MNX_REQUIRE(cond, ...)                                                        \
    do {                                                                              \
        if (!(cond)) return ::mnx::set_error(MNX_ERR_INVALID, __VA_ARGS__);           \
    } while (0)

constexpr int kWave = 64;

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Aligned bump allocator over a caller-provided workspace.
struct Workspace {
    char* base;
    size_t size;
    size_t used = 0;
    template <typename T>
    T* take(size_t count) {
        size_t off = (used + 255) & ~size_t(255);
        used = off + count * sizeof(T);
        return base ? reinterpret_cast<T*>(base + off) : nullptr;
    }
    bool fits() const { return used <= size; }
};

}  // namespace mnx
