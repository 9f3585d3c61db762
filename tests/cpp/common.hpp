// Shared helpers of the C++ tests: fixtures quantised on the device by the quantiser of record
// (vrt_q8_quantize, bit-exact), and a host dequant for the references.
#pragma once

#include "vortexrt/buffer.hpp"
#include "vortexrt/gguf.hpp"
#include "vrt_hip.h"

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <vector>

namespace vt = vortexrt;

#define EXPECT(cond)                                                                  \
    do {                                                                              \
        if (!(cond)) {                                                                \
            std::fprintf(stderr, "%s:%d: check failed: %s\n", __FILE__, __LINE__, #cond); \
            std::exit(1);                                                             \
        }                                                                             \
    } while (0)

// rows x k floats -> Q8_0 bytes with the given quantiser variant (0: src/q8_test_main.cpp,
// 1: src/ffn_test_main.cpp), computed on the device.
inline std::vector<std::uint8_t> quantize(vt::DeviceContext& ctx, const std::vector<float>& w, std::uint32_t variant) {
    vt::Buffer src(ctx, w.size() * 4u, vt::kBufferUsageStorage, vt::kMemoryDeviceLocal);
    const std::size_t nb = w.size() / 32u;
    vt::Buffer dst(ctx, nb * 34u, vt::kBufferUsageStorage, vt::kMemoryDeviceLocal);
    src.upload(w.data(), w.size() * 4u);
    vt::check_vrt(vrt_q8_quantize(ctx.handle(), static_cast<const float*>(src.handle()), w.size(), variant, dst.handle()));
    std::vector<std::uint8_t> out(nb * 34u);
    dst.download(out.data(), out.size());
    return out;
}

// Sequential fp32 reference of one row: sum of (scale * q) * x in block order.
inline float row_dot(const std::uint8_t* row, const float* x, std::uint32_t k) {
    float acc = 0.0f;
    for (std::uint32_t b = 0; b < k / 32u; ++b) {
        const std::uint8_t* blk = row + b * 34u;
        const float s = vt::f16_to_f32(static_cast<std::uint16_t>(blk[0] | (blk[1] << 8)));
        for (int j = 0; j < 32; ++j) acc += s * static_cast<float>(static_cast<std::int8_t>(blk[2 + j])) * x[b * 32u + j];
    }
    return acc;
}

template <typename F>
inline bool throws(F&& f) {
    try {
        f();
    } catch (const std::exception&) {
        return true;
    }
    return false;
}
