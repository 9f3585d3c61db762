// GgufFile (vortexrt:: C++ reader) on a file: prints its header, tensor directory and the
// dequantised Q8_0 rows asked for, as JSON. No GPU. Usage: gguf_test file [tensor row]...
#include "vortexrt/gguf.hpp"

#include <cstdio>
#include <exception>
#include <string>

int main(int argc, char** argv) {
    if (argc < 2) return 2;
    try {
        vortexrt::GgufFile f(argv[1]);
        f.validate();
        std::printf("{\"version\": %u, \"data_offset\": %llu, \"alignment\": %u, \"arch\": \"%s\", \"n_meta\": %zu, \"tensors\": {",
                    f.version(), static_cast<unsigned long long>(f.data_offset()), f.alignment(),
                    f.metadata_string("general.architecture").value_or("").c_str(), f.metadata().size());
        bool first = true;
        for (const auto& t : f.tensors()) {
            std::printf("%s\"%s\": [%u, %llu, %llu", first ? "" : ", ", t.name.c_str(), t.type,
                        static_cast<unsigned long long>(t.offset),
                        static_cast<unsigned long long>(f.tensor_byte_size(t).value_or(0)));
            for (const auto d : t.dimensions) std::printf(", %llu", static_cast<unsigned long long>(d));
            std::printf("]");
            first = false;
        }
        std::printf("}, \"rows\": [");
        for (int i = 2; i + 1 < argc; i += 2) {
            const auto* t = f.find_tensor(argv[i]);
            const auto row = f.read_q8_0_row(*t, std::stoull(argv[i + 1]));
            std::printf("%s[", i > 2 ? ", " : "");
            for (std::size_t j = 0; j < row.size(); ++j) std::printf("%s%.9g", j ? ", " : "", row[j]);
            std::printf("]");
        }
        std::printf("]}\n");
    } catch (const std::exception& e) {
        std::printf("{\"error\": \"%s\"}\n", e.what());
        return 1;
    }
    return 0;
}
