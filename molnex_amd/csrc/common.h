// Shared helpers for the molnex HIP library (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <mutex>
#include <unordered_map>

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

// Workgroups of `threads` threads of `kernel` that the current device holds at once
// (compute units x resident workgroups per unit, cached per kernel and device), capped
// at `need`; -1 if the runtime cannot tell.  Grid size of persistent (grid-strided)
// kernels.
inline int64_t device_fill_grid(const void* kernel, int threads, int64_t need) {
    static std::mutex mu;
    static std::unordered_map<const void*, int> per_cu[64];
    static int cus[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return -1;
    std::lock_guard<std::mutex> lock(mu);
    if (cus[dev] == 0 && hipDeviceGetAttribute(&cus[dev], hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return -1;
    auto it = per_cu[dev].find(kernel);
    if (it == per_cu[dev].end()) {
        int b = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, kernel, threads, 0) != hipSuccess) return -1;
        it = per_cu[dev].emplace(kernel, std::max(b, 1)).first;
    }
    return std::min<int64_t>(need, int64_t(it->second) * cus[dev]);
}

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
