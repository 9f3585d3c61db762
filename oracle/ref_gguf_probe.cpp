// ref_gguf_probe.cpp -- TEST INFRASTRUCTURE. Driver linked against the reference's own
// GGUF parser (src/gguf.cpp, built by `make ref` into oracle/_ref/). It prints what
// vortexrt::GgufFile sees in a file, so tests can pin this repository's GGUF writer and
// reader (and the Q8_0 row dequant, src/gguf.cpp:546-638) against the reference.
//
//   ref_gguf_probe FILE [TENSOR ROW]...
// Output lines:
//   header <version> <data_offset> <alignment> <n_metadata> <n_tensors>
//   meta <key> <type> <u64|i64|f64|str|array-length>
//   tensor <name> <type> <offset> <bytes> <dim0> [dim1 ...]
//   row <tensor> <row> <hex float bits ...>
#include "vortexrt/gguf.hpp"

#include <cinttypes>
#include <cstdio>
#include <cstring>
#include <exception>
#include <string>

int main(int argc, char** argv) {
    if (argc < 2) {
        std::fprintf(stderr, "usage: %s FILE [TENSOR ROW]...\n", argv[0]);
        return 2;
    }
    try {
        vortexrt::GgufFile f(argv[1]);
        std::printf("header %u %" PRIu64 " %u %zu %zu\n", f.version(), f.data_offset(), f.alignment(),
                    f.metadata().size(), f.tensors().size());
        for (const auto& kv : f.metadata()) {
            const auto& v = kv.value;
            std::printf("meta %s %u ", kv.key.c_str(), static_cast<unsigned>(v.type));
            if (v.is_array()) std::printf("%zu\n", v.array.size());
            else if (auto s = v.as_string()) std::printf("%s\n", s->c_str());
            else if (auto d = v.as_f64()) std::printf("%.17g\n", *d);
            else if (auto u = v.as_u64()) std::printf("%" PRIu64 "\n", *u);
            else if (auto i = v.as_i64()) std::printf("%" PRId64 "\n", *i);
            else if (auto b = v.as_bool()) std::printf("%d\n", *b ? 1 : 0);
            else std::printf("?\n");
        }
        for (const auto& t : f.tensors()) {
            const auto nb = f.tensor_byte_size(t);
            std::printf("tensor %s %u %" PRIu64 " %" PRIu64, t.name.c_str(), t.type, t.offset, nb ? *nb : 0);
            for (auto d : t.dimensions) std::printf(" %" PRIu64, d);
            std::printf("\n");
        }
        for (int a = 2; a + 1 < argc; a += 2) {
            const auto* t = f.find_tensor(argv[a]);
            if (!t) { std::printf("row %s missing\n", argv[a]); continue; }
            const auto row = std::stoull(argv[a + 1]);
            const auto vals = f.read_q8_0_row(*t, row);
            std::printf("row %s %llu", argv[a], static_cast<unsigned long long>(row));
            for (float v : vals) {
                uint32_t u;
                std::memcpy(&u, &v, 4);
                std::printf(" %08x", u);
            }
            std::printf("\n");
        }
    } catch (const std::exception& e) {
        std::printf("error %s\n", e.what());
        return 1;
    }
    return 0;
}
