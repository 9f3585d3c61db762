// Prints the error each device state maps to (vrt_g3_errors.hpp): one line per
// "nonfinite abort_flag" pair read from stdin, as "code|message".
#include <cstdint>
#include <cstdio>

#include "vrt_g3_errors.hpp"

int main() {
    unsigned long long nf = 0, ab = 0;
    while (std::scanf("%llx %llx", &nf, &ab) == 2) {
        const vrt::G3Failure f = vrt::g3_map_failure(static_cast<uint32_t>(nf), static_cast<uint32_t>(ab));
        std::printf("%d|%s\n", f.code, f.msg);
    }
    return 0;
}
