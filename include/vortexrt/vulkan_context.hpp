// Device context of the HIP build (include/vortexrt/vulkan_context.hpp:45-70 of Vortex-RT).
// The reference's class is VulkanContext; here the same role is DeviceContext over one HIP
// device and one stream, and VulkanContext names it so existing callers keep compiling.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>

struct vrt_ctx;

namespace vortexrt {

// DeviceCapabilities (reference :13-32), HIP fields.
struct DeviceCapabilities {
    std::string name;
    std::string arch;                  // e.g. "gfx950"
    std::uint32_t device_index = 0;
    std::uint32_t vendor_id = 0;
    std::uint32_t device_id = 0;
    std::uint32_t subgroup_size = 0;   // wavefront size (64)
    std::uint32_t compute_units = 0;
    bool fp16 = false;
    bool int8 = false;
    bool storage8 = false;
    bool storage16 = false;
    std::uint64_t device_local_bytes = 0;
    std::uint64_t l2_bytes = 0;
};

class DeviceContext {
public:
    // device_selector: "" (then env VORTEXRT_DEVICE, then device 0), a decimal index, or a
    // case-insensitive substring of the device name (reference src/vulkan_context.cpp:116-317).
    explicit DeviceContext(std::string device_selector = {});
    ~DeviceContext();

    DeviceContext(const DeviceContext&) = delete;
    DeviceContext& operator=(const DeviceContext&) = delete;

    [[nodiscard]] const DeviceCapabilities& capabilities() const noexcept { return caps_; }
    [[nodiscard]] vrt_ctx* handle() const noexcept { return ctx_; }
    // The hipStream_t every kernel of this context is launched on.
    [[nodiscard]] void* stream() const;
    // Waits for all work on the stream (the reference's fence waits).
    void synchronize();

private:
    vrt_ctx* ctx_ = nullptr;
    DeviceCapabilities caps_{};
};

using VulkanContext = DeviceContext;

// Throws std::runtime_error(vrt_last_error()) when rc is not VRT_OK.
void check_vrt(int rc);

}  // namespace vortexrt
