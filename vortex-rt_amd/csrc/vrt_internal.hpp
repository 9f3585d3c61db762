// vrt_internal.hpp -- host-side internals shared by the C-ABI translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include "vrt_hip.h"

struct vrt_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    vrt_device_info info{};
    // Scratch for the standalone reductions (argmax partials). Kernels on one context are
    // stream-ordered, so calls never overlap on it.
    void* scratch = nullptr;
    size_t scratch_bytes = 0;
    // This device's address of the static workspace of vrt_q8_ffn_noalloc (hipGetSymbolAddress).
    float* ffn_scratch = nullptr;
};

namespace vrt {

int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

#define VRT_HIP_CHECK(expr)                                                                  \
    do {                                                                                     \
        hipError_t _e = (expr);                                                              \
        if (_e != hipSuccess)                                                                \
            return ::vrt::set_error(VRT_ERR_HIP, "%s failed: %s", #expr, hipGetErrorString(_e)); \
    } while (0)

#define VRT_REQUIRE(cond, ...)                                                               \
    do {                                                                                     \
        if (!(cond)) return ::vrt::set_error(VRT_ERR_INVALID, __VA_ARGS__);                  \
    } while (0)

// Matvec launch shape for a given K: S lanes per row slot, NB blocks per lane.
struct MvShape {
    int S;
    int NB;
};
bool mv_shape(uint32_t input_dim, MvShape* out);

// Launches the generic Q8_0 matvec over a virtual row space on `stream`.
// x: device fp32[K]; y: device fp32[total rows] (virtual-row order).
int launch_matvec(hipStream_t stream, const uint8_t* const* bases, const uint32_t* rows, uint32_t nseg,
                  int interleave, uint32_t K, const uint8_t* w_end, const float* x, float* y);

}  // namespace vrt
