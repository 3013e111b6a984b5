// gguf.cpp -- GGUF reading and host decoding for the loader.
#include "gguf.hpp"

#include <array>
#include <cmath>
#include <cstring>
#include <fstream>

#include "vkml/error.hpp"

namespace vkml::detail {

namespace {

constexpr std::uint64_t kMaxDimension = std::uint64_t{1} << 40;
constexpr std::uint64_t kMaxString = std::uint64_t{1} << 30;
constexpr std::uint64_t kMaxArray = std::uint64_t{1} << 28;

class Reader {
public:
    Reader(std::ifstream& in, std::string where) : in_(in), where_(std::move(where)) {}
    template <class T>
    T get() {
        T v{};
        bytes(&v, sizeof v);
        return v;
    }
    std::string str() {
        const auto size = get<std::uint64_t>();
        if (size > kMaxString) fail("a string of " + std::to_string(size) + " bytes");
        std::string s(size, '\0');
        bytes(s.data(), size);
        return s;
    }
    void bytes(void* out, std::uint64_t n) {
        if (!in_.read(static_cast<char*>(out), static_cast<std::streamsize>(n))) throw Error(where_ + ": truncated");
    }
    std::uint64_t position() { return static_cast<std::uint64_t>(in_.tellg()); }
    [[noreturn]] void fail(const std::string& what) { throw Error(where_ + ": malformed header: " + what); }

    // Metadata value of type t (0-12: u8 i8 u16 i16 u32 i32 f32 bool string array u64 i64 f64).
    GgufValue value(std::uint32_t t, int depth = 0) {
        switch (t) {
            case 0: return {double(get<std::uint8_t>())};
            case 1: return {double(get<std::int8_t>())};
            case 2: return {double(get<std::uint16_t>())};
            case 3: return {double(get<std::int16_t>())};
            case 4: return {double(get<std::uint32_t>())};
            case 5: return {double(get<std::int32_t>())};
            case 6: return {double(get<float>())};
            case 7: return {double(get<std::uint8_t>() != 0)};
            case 8: return {str()};
            case 9: {
                if (depth > 4) fail("arrays nested too deep");
                const auto element = get<std::uint32_t>();
                const auto count = get<std::uint64_t>();
                if (count > kMaxArray) fail("an array of " + std::to_string(count) + " values");
                std::vector<GgufValue> out;
                out.reserve(static_cast<std::size_t>(std::min<std::uint64_t>(count, 1 << 20)));
                for (std::uint64_t i = 0; i < count; ++i) out.push_back(value(element, depth + 1));
                return {std::move(out)};
            }
            case 10: return {double(get<std::uint64_t>())};
            case 11: return {double(get<std::int64_t>())};
            case 12: return {get<double>()};
            default: fail("a value of unknown type " + std::to_string(t));
        }
    }

private:
    std::ifstream& in_;
    std::string where_;
};

std::uint16_t rd16(const std::uint8_t* p) {
    std::uint16_t v;
    std::memcpy(&v, p, 2);
    return v;
}

void scale_min_k4(int j, const std::uint8_t* q, std::uint8_t& sc, std::uint8_t& m) {
    if (j < 4) {
        sc = q[j] & 63;
        m = q[j + 4] & 63;
    } else {
        sc = std::uint8_t((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        m = std::uint8_t((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

void block_q8_0(const std::uint8_t* b, float* y) {
    const float d = f16_to_float(rd16(b));
    for (int j = 0; j < 32; ++j) y[j] = float(std::int8_t(b[2 + j])) * d;
}

void block_q4(const std::uint8_t* b, float* y, bool offset) {
    const float d = f16_to_float(rd16(b));
    const float m = offset ? f16_to_float(rd16(b + 2)) : 0.0f;
    const std::uint8_t* qs = b + (offset ? 4 : 2);
    for (int j = 0; j < 16; ++j) {
        const int q0 = qs[j] & 0x0F, q1 = qs[j] >> 4;
        y[j] = offset ? float(q0) * d + m : float(q0 - 8) * d;
        y[j + 16] = offset ? float(q1) * d + m : float(q1 - 8) * d;
    }
}

void block_q4_k(const std::uint8_t* b, float* y) {
    const float d = f16_to_float(rd16(b)), dmin = f16_to_float(rd16(b + 2));
    const std::uint8_t* q = b + 16;
    for (int j = 0, is = 0; j < 256; j += 64, is += 2) {
        std::uint8_t sc, m;
        scale_min_k4(is, b + 4, sc, m);
        const float d1 = d * float(sc), m1 = dmin * float(m);
        scale_min_k4(is + 1, b + 4, sc, m);
        const float d2 = d * float(sc), m2 = dmin * float(m);
        for (int l = 0; l < 32; ++l) *y++ = d1 * float(q[l] & 0xF) - m1;
        for (int l = 0; l < 32; ++l) *y++ = d2 * float(q[l] >> 4) - m2;
        q += 32;
    }
}

void block_q6_k(const std::uint8_t* b, float* y) {
    const std::uint8_t* ql = b;
    const std::uint8_t* qh = b + 128;
    const auto* sc = reinterpret_cast<const std::int8_t*>(b + 192);
    const float d = f16_to_float(rd16(b + 208));
    for (int n = 0; n < 256; n += 128) {
        for (int l = 0; l < 32; ++l) {
            const int is = l / 16;
            const int q1 = ((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
            const int q2 = ((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
            const int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            const int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            y[l] = d * float(sc[is]) * float(q1);
            y[l + 32] = d * float(sc[is + 2]) * float(q2);
            y[l + 64] = d * float(sc[is + 4]) * float(q3);
            y[l + 96] = d * float(sc[is + 6]) * float(q4);
        }
        y += 128;
        ql += 64;
        qh += 32;
        sc += 8;
    }
}

// x rounded half to even for |x| < 2^22 by the 1.5 * 2^23 addition
// (src/io/host_quant.cpp:63-70); volatile keeps the two roundings.
float round_even(float x) {
    volatile float t = x + 12582912.0f;
    return t - 12582912.0f;
}

}  // namespace

float f16_to_float(std::uint16_t h) {
    const std::uint32_t sign = std::uint32_t(h & 0x8000u) << 16;
    const std::uint32_t exponent = (h >> 10) & 0x1Fu, mantissa = h & 0x3FFu;
    std::uint32_t bits;
    if (exponent == 0) {
        float f = float(mantissa) * 5.9604644775390625e-8f;
        std::memcpy(&bits, &f, 4);
        bits |= sign;
    } else if (exponent == 31) {
        bits = sign | 0x7F800000u | (mantissa << 13);
    } else {
        bits = sign | ((exponent + 112u) << 23) | (mantissa << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

std::uint16_t float_to_f16(float f) {
    std::uint32_t x;
    std::memcpy(&x, &f, 4);
    const std::uint32_t sign = (x >> 16) & 0x8000u;
    const std::uint32_t biased = (x >> 23) & 0xFFu;
    std::uint32_t mantissa = x & 0x7FFFFFu;
    if (biased == 0xFFu) return std::uint16_t(sign | 0x7C00u | (mantissa ? 0x200u : 0u));
    const int exponent = int(biased) - 127 + 15;
    if (exponent >= 31) return std::uint16_t(sign | 0x7C00u);
    const auto round = [](std::uint32_t value, int shift) {
        const std::uint32_t kept = value >> shift, rest = value & ((1u << shift) - 1);
        const std::uint32_t half = 1u << (shift - 1);
        return kept + (rest > half || (rest == half && (kept & 1u)) ? 1u : 0u);
    };
    if (exponent <= 0) {
        if (exponent < -10) return std::uint16_t(sign);
        mantissa |= 0x800000u;
        return std::uint16_t(sign | round(mantissa, 14 - exponent));
    }
    return std::uint16_t(sign | round((std::uint32_t(exponent) << 23) | mantissa, 13));
}

const char* ggml_type_name(std::uint32_t t) {
    switch (t) {
        case kGgmlF32: return "f32";
        case kGgmlF16: return "f16";
        case kGgmlQ4_0: return "q4_0";
        case kGgmlQ4_1: return "q4_1";
        case kGgmlQ5_0: return "q5_0";
        case kGgmlQ5_1: return "q5_1";
        case kGgmlQ8_0: return "q8_0";
        case 9: return "q8_1";
        case kGgmlQ2_K: return "q2_K";
        case kGgmlQ3_K: return "q3_K";
        case kGgmlQ4_K: return "q4_K";
        case kGgmlQ5_K: return "q5_K";
        case kGgmlQ6_K: return "q6_K";
        case 15: return "q8_K";
        case kGgmlBF16: return "bf16";
        default: return nullptr;
    }
}

std::pair<std::uint64_t, std::uint64_t> ggml_block(std::uint32_t t) {
    switch (t) {
        case kGgmlF32: return {1, 4};
        case kGgmlF16: case kGgmlBF16: return {1, 2};
        case kGgmlQ4_0: return {32, 18};
        case kGgmlQ4_1: return {32, 20};
        case kGgmlQ5_0: return {32, 22};
        case kGgmlQ5_1: return {32, 24};
        case kGgmlQ8_0: return {32, 34};
        case 9: return {32, 36};
        case kGgmlQ2_K: return {256, 84};
        case kGgmlQ3_K: return {256, 110};
        case kGgmlQ4_K: return {256, 144};
        case kGgmlQ5_K: return {256, 176};
        case kGgmlQ6_K: return {256, 210};
        case 15: return {256, 292};
        default: return {0, 0};
    }
}

Gguf::Gguf(const std::filesystem::path& path) : path_(path) {
    const std::string where = "gguf: " + path.string();
    std::ifstream in(path, std::ios::binary);
    if (!in) throw Error(where + ": cannot open file");
    std::error_code ec;
    const std::uint64_t file_size = std::filesystem::file_size(path, ec);
    if (ec) throw Error(where + ": cannot read file size");
    Reader r{in, where};
    std::array<char, 4> magic{};
    if (file_size < 4 || !in.read(magic.data(), 4) || std::string(magic.data(), 4) != "GGUF") throw Error(where + ": not a GGUF file");
    version_ = r.get<std::uint32_t>();
    if (version_ < 2 || version_ > 3) throw Error(where + ": GGUF version " + std::to_string(version_) + " is not supported (2 and 3 are)");
    const auto tensors = r.get<std::uint64_t>();
    const auto kvs = r.get<std::uint64_t>();
    if (tensors > (std::uint64_t{1} << 24) || kvs > (std::uint64_t{1} << 24)) {
        r.fail("counts of " + std::to_string(tensors) + " tensors and " + std::to_string(kvs) + " metadata entries");
    }
    for (std::uint64_t i = 0; i < kvs; ++i) {
        std::string key = r.str();
        const auto type = r.get<std::uint32_t>();
        metadata_[key] = r.value(type);
    }
    std::vector<std::pair<std::string, Entry>> infos;
    for (std::uint64_t i = 0; i < tensors; ++i) {
        std::string name = r.str();
        const auto dims = r.get<std::uint32_t>();
        if (dims > 4) r.fail("tensor " + name + " has " + std::to_string(dims) + " dimensions");
        Shape shape(dims);
        for (std::uint32_t d = 0; d < dims; ++d) {
            const auto n = r.get<std::uint64_t>();
            if (n > kMaxDimension) r.fail("tensor " + name + " has a dimension of " + std::to_string(n));
            shape[dims - 1 - d] = static_cast<std::int64_t>(n);
        }
        const auto type = r.get<std::uint32_t>();
        const auto offset = r.get<std::uint64_t>();
        infos.emplace_back(std::move(name), Entry{std::move(shape), type, offset, 0});
    }
    const auto align_it = metadata_.find("general.alignment");
    const std::uint64_t alignment = align_it != metadata_.end() && align_it->second.is_number() ? std::uint64_t(align_it->second.number()) : 32;
    if (alignment == 0 || alignment > (std::uint64_t{1} << 30)) r.fail("general.alignment is " + std::to_string(alignment));
    data_start_ = (r.position() + alignment - 1) / alignment * alignment;
    for (auto& [name, e] : infos) {
        const auto too_large = [&] { throw Error(where + ": tensor " + name + " is too large"); };
        std::uint64_t count = 1;
        for (const std::int64_t d : e.shape) {
            const auto n = static_cast<std::uint64_t>(d);
            if (n != 0 && count > UINT64_MAX / n) too_large();
            count *= n;
        }
        const auto [values, size] = ggml_block(e.type);
        if (values) {
            const std::uint64_t blocks = count / values + (count % values != 0);
            if (blocks > UINT64_MAX / size) too_large();
            e.bytes = blocks * size;
        }
        if (data_start_ > file_size || e.offset > file_size - data_start_ || e.bytes > file_size - data_start_ - e.offset) {
            throw Error(where + ": tensor " + name + " runs past the end of the file");
        }
        entries_.emplace(std::move(name), std::move(e));
    }
}

double Gguf::number(const std::string& key, double fallback) const {
    const auto it = metadata_.find(key);
    return it != metadata_.end() && it->second.is_number() ? it->second.number() : fallback;
}

std::string Gguf::string(const std::string& key, const std::string& fallback) const {
    const auto it = metadata_.find(key);
    return it != metadata_.end() && it->second.is_string() ? it->second.str() : fallback;
}

const Gguf::Entry& Gguf::entry(const std::string& name) const {
    const auto it = entries_.find(name);
    if (it == entries_.end()) throw Error("gguf: " + path_.string() + " has no tensor \"" + name + "\"");
    return it->second;
}

std::string Gguf::type_name(const std::string& name) const {
    const Entry& e = entry(name);
    const char* n = ggml_type_name(e.type);
    return n ? n : "type " + std::to_string(e.type);
}

std::vector<std::uint8_t> Gguf::read(const std::string& name) const {
    const Entry& e = entry(name);
    std::vector<std::uint8_t> out(e.bytes);
    std::ifstream in(path_, std::ios::binary);
    in.seekg(static_cast<std::streamoff>(data_start_ + e.offset));
    if (!in.read(reinterpret_cast<char*>(out.data()), static_cast<std::streamsize>(out.size()))) {
        throw Error("gguf: reading tensor \"" + name + "\" from " + path_.string() + " failed");
    }
    return out;
}

void dequantize_blocks(std::uint32_t type, const std::uint8_t* blocks, std::size_t count, float* out) {
    const auto [values, size] = ggml_block(type);
    for (std::size_t b = 0; b < count; ++b) {
        const std::uint8_t* p = blocks + b * size;
        float* y = out + b * values;
        switch (type) {
            case kGgmlQ8_0: block_q8_0(p, y); break;
            case kGgmlQ4_0: block_q4(p, y, false); break;
            case kGgmlQ4_1: block_q4(p, y, true); break;
            case kGgmlQ4_K: block_q4_k(p, y); break;
            case kGgmlQ6_K: block_q6_k(p, y); break;
            default: {
                const char* n = ggml_type_name(type);
                throw Error(std::string("gguf: decoding ") + (n ? n : "this type") +
                            " is not implemented (q8_0, q4_0, q4_1, q4_K and q6_K are)");
            }
        }
    }
}

void requantize_q8(std::uint32_t type, const std::uint8_t* data, std::int64_t rows, std::int64_t cols, std::uint32_t* words,
                   std::uint16_t* halves) {
    const auto [values, size] = ggml_block(type);
    const std::size_t count = std::size_t(rows * cols);
    if (values == 0 || cols % 32 != 0 || count % values != 0) {
        throw Error("requantize_q8: " + std::to_string(rows) + " x " + std::to_string(cols) + " values are not whole blocks");
    }
    if (type != kGgmlQ8_0 && type != kGgmlQ4_0 && type != kGgmlQ4_1 && type != kGgmlQ4_K && type != kGgmlQ6_K) {
        const char* n = ggml_type_name(type);
        throw Error(std::string("gguf: decoding ") + (n ? n : "this type") + " is not implemented (q8_0, q4_0, q4_1, q4_K and q6_K are)");
    }
    parallel_for(count / values, [&](std::size_t begin, std::size_t end) {
        std::array<float, 256> y;
        for (std::size_t u = begin; u < end; ++u) {
            dequantize_blocks(type, data + u * size, 1, y.data());
            for (std::size_t g = 0; g < values; g += 32) {
                const float* x = y.data() + g;
                float absmax = 0.0f;
                for (int i = 0; i < 32; ++i) absmax = std::max(absmax, std::abs(x[i]));
                const std::size_t group = (u * values + g) / 32;
                halves[group] = float_to_f16(absmax / 127.0f);
                const float d = f16_to_float(halves[group]);
                const float inv = d > 0.0f ? 1.0f / d : 0.0f;
                for (int w = 0; w < 8; ++w) {
                    std::uint32_t word = 0;
                    for (int k = 0; k < 4; ++k) {
                        const float v = std::clamp(round_even(x[4 * w + k] * inv), -127.0f, 127.0f);
                        word |= (std::uint32_t(std::int32_t(v)) & 0xFFu) << (8 * k);
                    }
                    words[group * 8 + w] = word;
                }
            }
        }
    });
}

}  // namespace vkml::detail
