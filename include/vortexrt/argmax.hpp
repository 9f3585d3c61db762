// Greedy argmax (include/vortexrt/argmax.hpp:12-32 of Vortex-RT).
#pragma once

#include "vortexrt/buffer.hpp"

#include <cstdint>
#include <string>

namespace vortexrt {

struct ArgmaxResult {
    std::uint32_t index = 0;
    float value = 0.0f;
};

static_assert(sizeof(ArgmaxResult) == 8);

class ArgmaxPipeline {
public:
    // The shader path is accepted for signature compatibility; the kernel is built in.
    ArgmaxPipeline(DeviceContext& context, const std::string& spirv_path = {});
    ~ArgmaxPipeline() = default;

    ArgmaxPipeline(const ArgmaxPipeline&) = delete;
    ArgmaxPipeline& operator=(const ArgmaxPipeline&) = delete;

    // output[0] = {index, value} of the largest of element_count floats of input: NaN never
    // wins, equal values go to the lower index (shaders/argmax.comp). Synchronous.
    void run(Buffer& input, Buffer& output, std::uint32_t element_count);

private:
    DeviceContext& context_;
};

}  // namespace vortexrt
