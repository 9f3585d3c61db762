// vrt_g3_errors.hpp -- how the device state a decode launch leaves behind maps to the errors the
// reference throws (src/gemma3.cpp:1609-1696 softmax, :1857-1863 non-finite hidden state).
// Host-only and dependency-free, so the mapping is unit-tested on the CPU.
#pragma once

#include <cstdint>
#include <cstdio>

#include "vrt_hip.h"

namespace vrt {

// G3State::nonfinite codes. The device keeps the minimum of every code raised during a launch,
// and the codes are ordered as the reference's checks run: block l's softmax check comes before
// block l's non-finite check, which comes before anything in block l + 1. So the minimum is the
// error the reference throws first.
constexpr uint32_t kG3NoFailure = 0xffffffffu;
constexpr uint32_t kG3HandoffLost = 0x20000000u;  // a persistent-kernel hand-off was abandoned
constexpr uint32_t g3_code_softmax(uint32_t block) { return 2u * block; }        // :1666-1670
constexpr uint32_t g3_code_nonfinite(uint32_t block) { return 2u * block + 1u; }  // :1857-1863

struct G3Failure {
    int code = VRT_OK;
    char msg[160] = {0};
};

// nonfinite: G3State::nonfinite after the launch; abort_flag: the persistent kernel's abort
// word (0 when the multi-kernel path ran). Any raised abort flag is reported, whatever code the
// minimum kept, so a launch never ends with an abort flag nobody reports (the caller clears it).
inline G3Failure g3_map_failure(uint32_t nonfinite, uint32_t abort_flag) {
    G3Failure f;
    const bool lost = abort_flag != 0u || nonfinite == kG3HandoffLost;
    const char* also = lost ? " (a device hand-off was also abandoned)" : "";
    if (nonfinite < kG3HandoffLost && (nonfinite & 1u)) {
        f.code = VRT_ERR_NUMERIC;
        std::snprintf(f.msg, sizeof f.msg, "Non-finite value after Gemma 3 block %u%s", nonfinite >> 1, also);
    } else if (nonfinite < kG3HandoffLost) {
        f.code = VRT_ERR_NUMERIC;
        std::snprintf(f.msg, sizeof f.msg, "Gemma 3 attention softmax failed%s", also);
    } else if (lost) {
        f.code = VRT_ERR_HIP;
        std::snprintf(f.msg, sizeof f.msg, "Gemma 3 decode: device hand-off timed out");
    }
    return f;
}

}  // namespace vrt
