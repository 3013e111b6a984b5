// Host checks of the loader's GGUF pieces, built by tests/test_gguf_host.py
// against vkml-framework_amd/src/gguf.cpp alone:
//   halves            every f16 bit pattern widened (65536 lines of f32 bits)
//   narrow <file>     f32 bit patterns (one hex word a line) narrowed to f16
//   config <gguf>     the header of a GGUF file, or the error it raises
#include <cinttypes>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <string>

#include "../../vkml-framework_amd/src/gguf.hpp"
#include "vkml/error.hpp"

int main(int argc, char** argv) {
    using namespace vkml::detail;
    if (argc < 2) return 2;
    const std::string what = argv[1];
    if (what == "halves") {
        for (std::uint32_t h = 0; h < 65536; ++h) {
            const float f = f16_to_float(static_cast<std::uint16_t>(h));
            std::uint32_t b;
            std::memcpy(&b, &f, 4);
            std::printf("%08" PRIx32 "\n", b);
        }
        return 0;
    }
    if (what == "narrow" && argc == 3) {
        std::ifstream in(argv[2]);
        std::string line;
        while (std::getline(in, line)) {
            const auto b = static_cast<std::uint32_t>(std::stoul(line, nullptr, 16));
            float f;
            std::memcpy(&f, &b, 4);
            std::printf("%04x\n", float_to_f16(f));
        }
        return 0;
    }
    if (what == "config" && argc == 3) {
        try {
            const Gguf g{argv[2]};
            std::printf("version %u\n", g.version());
            for (const auto& [key, value] : g.metadata()) {
                if (value.is_number()) std::printf("meta %s %.17g\n", key.c_str(), value.number());
                else if (value.is_string()) std::printf("meta %s \"%s\"\n", key.c_str(), value.str().c_str());
                else std::printf("meta %s [array]\n", key.c_str());
            }
            return 0;
        } catch (const vkml::Error& e) {
            std::printf("error %s\n", e.what());
            return 1;
        }
    }
    return 2;
}
