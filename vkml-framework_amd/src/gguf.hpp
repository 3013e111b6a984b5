// gguf.hpp -- GGUF v2/v3 files (llama.cpp's format), the reader behind
// Llama::load and LlamaConfig::from_gguf (the reference's src/io/gguf.hpp:
// 22-71 is its counterpart). Metadata values are kept as numbers, strings,
// or arrays of them; tensor data is viewed in place in a read-only mapping
// of the file.
#pragma once

#include <cstdint>
#include <filesystem>
#include <map>
#include <memory>
#include <span>
#include <string>
#include <variant>
#include <vector>

#include "vkml/tensor.hpp"

namespace vkml::detail {

struct GgufValue {
    std::variant<std::monostate, double, std::string, std::vector<GgufValue>> v;
    bool is_number() const { return std::holds_alternative<double>(v); }
    bool is_string() const { return std::holds_alternative<std::string>(v); }
    double number() const { return std::get<double>(v); }
    const std::string& str() const { return std::get<std::string>(v); }
};

// ggml type numbers (src/io/gguf.cpp:30-40).
enum GgmlType : std::uint32_t {
    kGgmlF32 = 0, kGgmlF16 = 1, kGgmlQ4_0 = 2, kGgmlQ4_1 = 3, kGgmlQ5_0 = 6, kGgmlQ5_1 = 7, kGgmlQ8_0 = 8,
    kGgmlQ2_K = 10, kGgmlQ3_K = 11, kGgmlQ4_K = 12, kGgmlQ5_K = 13, kGgmlQ6_K = 14, kGgmlBF16 = 30
};

class Gguf {
public:
    explicit Gguf(const std::filesystem::path& path);

    std::uint32_t version() const noexcept { return version_; }
    const std::map<std::string, GgufValue>& metadata() const noexcept { return metadata_; }
    bool has(const std::string& key) const { return metadata_.count(key) != 0; }
    double number(const std::string& key, double fallback) const;
    std::string string(const std::string& key, const std::string& fallback) const;

    struct Entry {
        Shape shape;  // row-major (GGUF lists dimensions fastest first)
        std::uint32_t type;
        std::uint64_t offset;
        std::uint64_t bytes;
    };
    bool contains(const std::string& name) const { return entries_.count(name) != 0; }
    const Entry& entry(const std::string& name) const;
    const Shape& shape(const std::string& name) const { return entry(name).shape; }
    std::string type_name(const std::string& name) const;

    // The raw bytes of a tensor, in the file's mapping (valid while this
    // Gguf, or a copy of it, lives).
    std::span<const std::uint8_t> bytes(const std::string& name) const;
    const std::filesystem::path& path() const noexcept { return path_; }

private:
    struct Mapping;
    std::filesystem::path path_;
    std::shared_ptr<Mapping> map_;
    std::uint32_t version_ = 0;
    std::map<std::string, GgufValue> metadata_;
    std::map<std::string, Entry> entries_;
    std::uint64_t data_start_ = 0;
};

// ggml's name of a type ("q4_K"), and (values, bytes) per block; {0, 0} if unknown.
const char* ggml_type_name(std::uint32_t type);
std::pair<std::uint64_t, std::uint64_t> ggml_block(std::uint32_t type);

// Host 16-bit conversions (src/io/host_quant.cpp:74-114).
float f16_to_float(std::uint16_t h);
std::uint16_t float_to_f16(float f);

// Decodes whole blocks of q8_0, q4_0, q4_1, q4_K or q6_K to f32 (src/io/gguf.cpp:117-228).
void dequantize_blocks(std::uint32_t type, const std::uint8_t* blocks, std::size_t count, float* out);

// Requantizes a [rows, cols] matrix of any decodable type to Q8_0 with f16
// scales on the host, every core (src/io/host_quant.cpp:116-159):
// words [rows * cols / 4], halves [rows * cols / 32].
void requantize_q8(std::uint32_t type, const std::uint8_t* data, std::int64_t rows, std::int64_t cols, std::uint32_t* words,
                   std::uint16_t* halves);

// Runs body(begin, end) over [0, n) split across up to 16 host threads.
template <class Body>
void parallel_for(std::size_t n, const Body& body);

}  // namespace vkml::detail

#include <algorithm>
#include <thread>

template <class Body>
void vkml::detail::parallel_for(std::size_t n, const Body& body) {
    const std::size_t threads = std::clamp<std::size_t>(std::thread::hardware_concurrency(), 1, 16);
    const std::size_t per = std::max<std::size_t>((n + threads - 1) / threads, 1);
    std::vector<std::thread> pool;
    for (std::size_t begin = per; begin < n; begin += per) pool.emplace_back([&body, begin, end = std::min(n, begin + per)] { body(begin, end); });
    body(0, std::min(n, per));
    for (auto& t : pool) t.join();
}
