// The reference's Q8_0 matvec test (src/q8_test_main.cpp:78-616) against vortexrt:: on the
// HIP path: 257 x 640 fixture, 2e-3 absolute bound, staged run, the pair/triplet fixture
// (three copies of the matrix at offsets 0, s, 2s; packed output equals the single output
// three times, replay within 1e-6), and the argument errors.
#include "common.hpp"

#include "vortexrt/q8_matvec.hpp"

#include <algorithm>
#include <array>
#include <cmath>
#include <cstring>
#include <iostream>

int main() {
    vt::DeviceContext ctx;
    constexpr std::uint32_t kIn = 640, kOut = 257, kBlocks = kIn / 32;
    std::vector<float> x(kIn), w(static_cast<std::size_t>(kOut) * kIn);
    for (std::uint32_t i = 0; i < kIn; ++i) x[i] = std::sin(float(i) * 0.031f) * 0.75f;
    for (std::uint32_t r = 0; r < kOut; ++r)
        for (std::uint32_t b = 0; b < kBlocks; ++b)
            for (std::uint32_t k = 0; k < 32; ++k)
                w[(std::size_t(r) * kBlocks + b) * 32 + k] = std::cos(float(r * 13 + b * 32 + k) * 0.017f) * 0.5f;
    auto q = quantize(ctx, w, 0);
    std::vector<float> ref(kOut);
    for (std::uint32_t r = 0; r < kOut; ++r) ref[r] = row_dot(q.data() + std::size_t(r) * kBlocks * 34u, x.data(), kIn);
    while (q.size() % 4u) q.push_back(0);

    vt::Q8MatVecPipeline pipe(ctx, "");
    vt::Buffer weights(ctx, q.size(), vt::kBufferUsageStorage, vt::kMemoryDeviceLocal);
    vt::Buffer in(ctx, kIn * 4u, vt::kBufferUsageStorage, vt::kMemoryDeviceLocal);
    vt::Buffer out(ctx, kOut * 4u * 3u, vt::kBufferUsageStorage, vt::kMemoryDeviceLocal);
    vt::Buffer st_in(ctx, kIn * 4u, vt::kBufferUsageTransferSrc, vt::kMemoryHostVisible | vt::kMemoryHostCoherent);
    vt::Buffer st_out(ctx, kOut * 4u * 3u, vt::kBufferUsageTransferDst, vt::kMemoryHostVisible | vt::kMemoryHostCoherent);
    weights.upload(q.data(), q.size());
    in.upload(x.data(), kIn * 4u);

    std::vector<float> y(kOut);
    pipe.run(weights, in, out, 0, kIn, kOut);
    out.download(y.data(), kOut * 4u);
    float max_err = 0.0f;
    for (std::uint32_t r = 0; r < kOut; ++r) max_err = std::max(max_err, std::fabs(y[r] - ref[r]));
    std::cout << "Vortex-RT Q8_0 matvec\n  GPU: " << ctx.capabilities().name << " (" << ctx.capabilities().arch << ")\n"
              << "  max abs error: " << max_err << "\n";
    EXPECT(max_err <= 2e-3f);

    std::vector<float> y2(kOut);
    pipe.run_staged(weights, in, out, st_in, st_out, x.data(), kIn * 4u, y2.data(), kOut * 4u, 0, kIn, kOut);
    EXPECT(std::memcmp(y.data(), y2.data(), kOut * 4u) == 0);

    // pair / triplet over three copies
    const std::size_t mat = q.size();
    std::vector<std::uint8_t> q3(mat * 3u);
    for (int c = 0; c < 3; ++c) std::copy(q.begin(), q.end(), q3.begin() + c * mat);
    vt::Buffer weights3(ctx, q3.size(), vt::kBufferUsageStorage, vt::kMemoryDeviceLocal);
    weights3.upload(q3.data(), q3.size());
    const auto s = static_cast<std::uint32_t>(mat);
    std::vector<float> y3(kOut * 3u), y3b(kOut * 3u);
    pipe.run_staged_triplet(weights3, in, out, st_in, st_out, x.data(), kIn * 4u, y3.data(), y3.size() * 4u,
                            {0u, s, 2u * s}, kIn, {kOut, kOut, kOut});
    pipe.run_staged_triplet(weights3, in, out, st_in, st_out, x.data(), kIn * 4u, y3b.data(), y3b.size() * 4u,
                            {0u, s, 2u * s}, kIn, {kOut, kOut, kOut});
    float tri_err = 0.0f, replay = 0.0f;
    for (std::uint32_t i = 0; i < kOut * 3u; ++i) {
        tri_err = std::max(tri_err, std::fabs(y3[i] - ref[i % kOut]));
        replay = std::max(replay, std::fabs(y3[i] - y3b[i]));
    }
    std::vector<float> y2p(kOut * 2u);
    pipe.run_staged_pair(weights3, in, out, st_in, st_out, x.data(), kIn * 4u, y2p.data(), y2p.size() * 4u, {s, 2u * s},
                         kIn, {kOut, kOut});
    float pair_err = 0.0f;
    for (std::uint32_t i = 0; i < kOut * 2u; ++i) pair_err = std::max(pair_err, std::fabs(y2p[i] - ref[i % kOut]));
    std::cout << "  triplet max abs error: " << tri_err << ", replay " << replay << ", pair " << pair_err << "\n";
    EXPECT(tri_err <= 2e-3f && pair_err <= 2e-3f && replay <= 1e-6f);

    // argument errors (src/q8_matvec.cpp:801-820)
    EXPECT(throws([&] { pipe.run(weights, in, out, 2, kIn, kOut); }));          // misaligned offset
    EXPECT(throws([&] { pipe.run(weights, in, out, 0, 48, kOut); }));           // K % 32
    EXPECT(throws([&] { pipe.run(weights, in, out, 0, kIn, 0); }));             // zero rows
    EXPECT(throws([&] { pipe.run(weights, in, out, 0, kIn, kOut + 64); }));     // weights too small
    EXPECT(throws([&] { in.upload(x.data(), kIn * 4u, 4); }));                  // Buffer::upload out of range
    std::cout << "q8_matvec_test ok\n";
    return 0;
}
