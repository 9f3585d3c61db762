// The reference's fused FFN test (src/ffn_test_main.cpp:254-441) against vortexrt:: on the
// HIP path: 64 -> 96 -> 64 with variant-B quantised gate/up/down, 5e-3 absolute bound against
// a float64 host reference on the dequantised weights, replay within 1e-6.
#include "common.hpp"

#include "vortexrt/q8_matvec.hpp"

#include <cmath>
#include <iostream>

namespace {

std::vector<float> fixture(std::uint32_t rows, std::uint32_t k, std::uint32_t seed) {
    std::vector<float> w(static_cast<std::size_t>(rows) * k);
    for (std::uint32_t r = 0; r < rows; ++r)
        for (std::uint32_t i = 0; i < k; ++i)
            w[std::size_t(r) * k + i] = std::sin(float(r * 31 + i * 7 + seed * 101) * 0.013f) * 0.05f;
    return w;
}

std::vector<double> matvec(const std::vector<std::uint8_t>& q, const std::vector<double>& x, std::uint32_t rows) {
    const auto k = static_cast<std::uint32_t>(x.size());
    std::vector<double> y(rows, 0.0);
    for (std::uint32_t r = 0; r < rows; ++r)
        for (std::uint32_t b = 0; b < k / 32u; ++b) {
            const std::uint8_t* blk = q.data() + (std::size_t(r) * (k / 32u) + b) * 34u;
            const double s = vt::f16_to_f32(static_cast<std::uint16_t>(blk[0] | (blk[1] << 8)));
            for (int j = 0; j < 32; ++j) y[r] += s * static_cast<std::int8_t>(blk[2 + j]) * x[b * 32u + j];
        }
    return y;
}

}  // namespace

int main() {
    vt::DeviceContext ctx;
    constexpr std::uint32_t kIn = 64, kFfn = 96, kOut = 64;
    const auto qg = quantize(ctx, fixture(kFfn, kIn, 1), 1);
    const auto qu = quantize(ctx, fixture(kFfn, kIn, 2), 1);
    const auto qd = quantize(ctx, fixture(kOut, kFfn, 3), 1);
    std::vector<std::uint8_t> enc;
    enc.insert(enc.end(), qg.begin(), qg.end());
    enc.insert(enc.end(), qu.begin(), qu.end());
    enc.insert(enc.end(), qd.begin(), qd.end());
    while (enc.size() % 4u) enc.push_back(0);
    std::vector<float> x(kIn);
    std::vector<double> xd(kIn);
    for (std::uint32_t i = 0; i < kIn; ++i) xd[i] = x[i] = std::sin(float(i) * 0.071f) * 0.8f;
    auto g = matvec(qg, xd, kFfn);
    const auto u = matvec(qu, xd, kFfn);
    for (std::uint32_t i = 0; i < kFfn; ++i) {
        const double a = g[i];
        g[i] = 0.5 * a * (1.0 + std::tanh(0.7978845608028654 * (a + 0.044715 * a * a * a))) * u[i];
    }
    const auto ref = matvec(qd, g, kOut);

    vt::Q8MatVecPipeline pipe(ctx, "", "", "");
    EXPECT(pipe.ffn_available());
    vt::Buffer weights(ctx, enc.size(), vt::kBufferUsageStorage, vt::kMemoryDeviceLocal);
    vt::Buffer in(ctx, kIn * 4u, vt::kBufferUsageStorage, vt::kMemoryDeviceLocal);
    vt::Buffer ws(ctx, 16384, vt::kBufferUsageStorage, vt::kMemoryDeviceLocal);
    vt::Buffer st_in(ctx, kIn * 4u, vt::kBufferUsageTransferSrc, vt::kMemoryHostVisible | vt::kMemoryHostCoherent);
    vt::Buffer st_out(ctx, kOut * 4u, vt::kBufferUsageTransferDst, vt::kMemoryHostVisible | vt::kMemoryHostCoherent);
    weights.upload(enc.data(), enc.size());
    const auto og = 0u, ou = static_cast<std::uint32_t>(qg.size()), od = static_cast<std::uint32_t>(qg.size() + qu.size());
    std::vector<float> y(kOut), y2(kOut);
    pipe.run_staged_ffn(weights, in, ws, st_in, st_out, x.data(), kIn * 4u, y.data(), kOut * 4u, og, ou, od, kIn, kFfn, kOut);
    pipe.run_staged_ffn(weights, in, ws, st_in, st_out, x.data(), kIn * 4u, y2.data(), kOut * 4u, og, ou, od, kIn, kFfn, kOut);
    double err = 0.0, replay = 0.0;
    for (std::uint32_t i = 0; i < kOut; ++i) {
        err = std::max(err, std::fabs(y[i] - ref[i]));
        replay = std::max(replay, std::fabs(double(y[i]) - double(y2[i])));
    }
    std::cout << "Vortex-RT Q8_0 fused FFN\n  max abs error: " << err << ", replay " << replay << "\n";
    EXPECT(err <= 5e-3 && replay <= 1e-6);
    EXPECT(throws([&] {
        pipe.run_staged_ffn(weights, in, ws, st_in, st_out, x.data(), kIn * 4u, y.data(), kOut * 4u, 2, ou, od, kIn, kFfn, kOut);
    }));
    EXPECT(throws([&] {
        pipe.run_staged_ffn(weights, in, ws, st_in, st_out, x.data(), kIn * 4u, y.data(), kOut * 4u, og, ou, od, kIn, 100, kOut);
    }));
    std::cout << "ffn_test ok\n";
    return 0;
}
