// Device or pinned-host buffer (include/vortexrt/buffer.hpp:11-42 of Vortex-RT).
#pragma once

#include "vortexrt/vulkan_context.hpp"

#include <cstddef>
#include <cstdint>

namespace vortexrt {

// Memory property bits with the values of the Vulkan flags they replace.
using MemoryPropertyFlags = std::uint32_t;
inline constexpr MemoryPropertyFlags kMemoryDeviceLocal = 0x1;    // -> hipMalloc
inline constexpr MemoryPropertyFlags kMemoryHostVisible = 0x2;    // -> pinned hipHostMalloc
inline constexpr MemoryPropertyFlags kMemoryHostCoherent = 0x4;
// Usage bits are accepted for signature compatibility; HIP memory needs none.
using BufferUsageFlags = std::uint32_t;
inline constexpr BufferUsageFlags kBufferUsageStorage = 0x20;
inline constexpr BufferUsageFlags kBufferUsageTransferSrc = 0x1;
inline constexpr BufferUsageFlags kBufferUsageTransferDst = 0x2;

class Buffer {
public:
    // Host-visible memory is pinned host memory the device reads directly; otherwise the
    // buffer is device memory. Either way the allocation starts zero-filled.
    Buffer(DeviceContext& context, std::uint64_t size, BufferUsageFlags usage, MemoryPropertyFlags memory_properties);
    ~Buffer();

    Buffer(const Buffer&) = delete;
    Buffer& operator=(const Buffer&) = delete;

    // Device-accessible address of the first byte.
    [[nodiscard]] void* handle() const noexcept { return ptr_; }
    [[nodiscard]] std::uint64_t size() const noexcept { return size_; }
    [[nodiscard]] bool host_visible() const noexcept { return (props_ & kMemoryHostVisible) != 0; }
    [[nodiscard]] bool host_coherent() const noexcept { return (props_ & kMemoryHostCoherent) != 0; }
    [[nodiscard]] DeviceContext& context() const noexcept { return context_; }

    // Synchronous copies (reference src/buffer.cpp:85-160; same range checks and messages).
    void upload(const void* data, std::size_t bytes, std::uint64_t offset = 0);
    void download(void* data, std::size_t bytes, std::uint64_t offset = 0) const;

private:
    DeviceContext& context_;
    void* ptr_ = nullptr;
    std::uint64_t size_ = 0;
    MemoryPropertyFlags props_ = 0;
};

}  // namespace vortexrt
