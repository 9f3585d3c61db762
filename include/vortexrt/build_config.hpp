// Constant names of the reference's generated build_config.hpp (include/vortexrt/
// build_config.hpp.in:3-26). Kernels are compiled into libvrt_hip.so, so there are no shader
// files: every path is empty, which the pipelines accept.
#pragma once

namespace vortexrt::build_config {

inline constexpr const char* vector_add_spv = "";
inline constexpr const char* q8_matvec_spv = "";
inline constexpr const char* q8_matvec_u8_spv = "";
inline constexpr const char* q8_matvec_32_spv = "";
inline constexpr const char* q8_matvec_u8_32_spv = "";
inline constexpr const char* q8_matvec_16_spv = "";
inline constexpr const char* q8_matvec_u8_16_spv = "";
inline constexpr const char* q8_matvec_8_spv = "";
inline constexpr const char* q8_matvec_u8_8_spv = "";
inline constexpr const char* argmax_spv = "";
inline constexpr const char* gelu_mul_spv = "";

}  // namespace vortexrt::build_config
