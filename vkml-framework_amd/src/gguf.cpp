// gguf.cpp -- GGUF reading and host decoding for the loader.
//
// The file is mapped read-only and its header parsed in place through a
// cursor that checks every read against the mapping's end, so a damaged
// length or count shows up as "truncated" instead of a huge allocation.
// Tensor data is handed out as views of the mapping (no copy).
#include "gguf.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <array>
#include <bit>
#include <cmath>
#include <cstring>

#include "vkml/error.hpp"

namespace vkml::detail {

namespace {

// A read-only view of the header bytes with a position.
class Cursor {
public:
    Cursor(const std::uint8_t* begin, const std::uint8_t* end, const std::string& where) : at_(begin), end_(end), where_(where) {}

    std::uint64_t remaining() const { return static_cast<std::uint64_t>(end_ - at_); }
    const std::uint8_t* here() const { return at_; }

    // n bytes from here, or an error naming what was being read.
    const std::uint8_t* take(std::uint64_t n, const char* what) {
        if (n > remaining()) truncated(std::string("reading ") + what);
        const std::uint8_t* p = at_;
        at_ += n;
        return p;
    }
    // A little-endian unsigned integer of `width` bytes.
    std::uint64_t uint(unsigned width, const char* what) {
        const std::uint8_t* p = take(width, what);
        std::uint64_t v = 0;
        for (unsigned i = 0; i < width; ++i) v |= std::uint64_t(p[i]) << (8 * i);
        return v;
    }
    std::uint32_t u32(const char* what) { return static_cast<std::uint32_t>(uint(4, what)); }
    std::uint64_t u64(const char* what) { return uint(8, what); }
    // A GGUF string: u64 length, then that many bytes.
    std::string text(const char* what) {
        const std::uint64_t n = u64(what);
        const std::uint8_t* p = take(n, what);
        return std::string(reinterpret_cast<const char*>(p), static_cast<std::size_t>(n));
    }
    [[noreturn]] void malformed(const std::string& what) const { throw Error(where_ + ": malformed header: " + what); }
    [[noreturn]] void truncated(const std::string& what) const { throw Error(where_ + ": truncated (" + what + ")"); }

private:
    const std::uint8_t* at_;
    const std::uint8_t* end_;
    const std::string& where_;
};

// GGUF metadata value types 0..12 (gguf.md): for scalars, the width in bytes
// and how the bits read: u unsigned, i signed, f IEEE float, b bool; 8 is a
// string and 9 an array.
struct ValueKind {
    unsigned width;
    char kind;
};
constexpr std::array<ValueKind, 13> kValueKinds{{{1, 'u'}, {1, 'i'}, {2, 'u'}, {2, 'i'}, {4, 'u'}, {4, 'i'}, {4, 'f'}, {1, 'b'},
                                                 {0, 's'}, {0, 'a'}, {8, 'u'}, {8, 'i'}, {8, 'f'}}};
constexpr int kMaxArrayDepth = 8;
constexpr std::uint64_t kMaxArray = std::uint64_t{1} << 28;  // values in one array (the reference's bound, gguf.cpp)

GgufValue parse_value(Cursor& c, std::uint32_t type, int depth) {
    if (type >= kValueKinds.size()) c.malformed("a value of unknown type " + std::to_string(type));
    const ValueKind k = kValueKinds[type];
    if (k.kind == 's') return {c.text("a string value")};
    if (k.kind == 'a') {
        if (depth >= kMaxArrayDepth) c.malformed("arrays nested more than " + std::to_string(kMaxArrayDepth) + " deep");
        const std::uint32_t element = c.u32("an array's element type");
        const std::uint64_t count = c.u64("an array's length");
        if (element >= kValueKinds.size()) c.malformed("an array of unknown type " + std::to_string(element));
        // Every element takes at least this many bytes of the file (a
        // string its 8-byte length, an array its type and length), so a
        // damaged count is caught before anything is reserved for it.
        const std::uint64_t least = kValueKinds[element].kind == 's' ? 8 : kValueKinds[element].kind == 'a' ? 12 : kValueKinds[element].width;
        if (count > kMaxArray || count > c.remaining() / least) c.truncated("an array of " + std::to_string(count) + " values");
        std::vector<GgufValue> items;
        items.reserve(static_cast<std::size_t>(std::min<std::uint64_t>(count, std::uint64_t{1} << 20)));
        for (std::uint64_t i = 0; i < count; ++i) items.push_back(parse_value(c, element, depth + 1));
        return {std::move(items)};
    }
    const std::uint64_t raw = c.uint(k.width, "a number");
    switch (k.kind) {
        case 'b': return {raw != 0 ? 1.0 : 0.0};
        case 'i': {
            const unsigned shift = 64 - 8 * k.width;  // sign-extend from the value's width
            return {double(static_cast<std::int64_t>(raw << shift) >> shift)};
        }
        case 'f':
            return {k.width == 4 ? double(std::bit_cast<float>(static_cast<std::uint32_t>(raw))) : std::bit_cast<double>(raw)};
        default: return {double(raw)};
    }
}

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

}  // namespace

// IEEE binary16 <-> binary32. Widening is exact: normal halves move their
// exponent and fraction into place, subnormal ones are their fraction times
// 2^-24 (a float computes that exactly).
float f16_to_float(std::uint16_t h) {
    const std::uint32_t sign = std::uint32_t(h >> 15) << 31;
    const std::uint32_t exponent = (h >> 10) & 0x1Fu, fraction = h & 0x3FFu;
    if (exponent == 0x1Fu) return std::bit_cast<float>(sign | 0x7F800000u | (fraction << 13));
    if (exponent != 0) return std::bit_cast<float>(sign | ((exponent + 112u) << 23) | (fraction << 13));
    return std::bit_cast<float>(sign | std::bit_cast<std::uint32_t>(std::ldexp(float(fraction), -24)));
}

// Narrowing rounds to nearest, ties to even. Normal results: rebias the
// exponent and round the 23-bit fraction to 10 by adding just under half an
// ulp plus the kept ulp's low bit (a carry out of the fraction bumps the
// exponent, as it should). Subnormal results: the value times 2^24, which a
// float holds exactly, rounded to an integer in the default rounding mode.
// 65520 and above go to infinity; NaN stays a quiet NaN.
std::uint16_t float_to_f16(float f) {
    const std::uint32_t x = std::bit_cast<std::uint32_t>(f);
    const auto sign = static_cast<std::uint16_t>((x >> 16) & 0x8000u);
    const std::uint32_t magnitude = x & 0x7FFFFFFFu;
    if (magnitude > 0x7F800000u) return sign | 0x7E00u;    // NaN
    if (magnitude >= 0x477FF000u) return sign | 0x7C00u;   // 65520 and above, infinity
    if (magnitude < 0x38800000u) {                          // below 2^-14
        const float scaled = std::bit_cast<float>(magnitude) * 16777216.0f;
        return sign | static_cast<std::uint16_t>(std::nearbyint(scaled));
    }
    std::uint32_t r = magnitude - (112u << 23);
    r += 0xFFFu + ((r >> 13) & 1u);
    return sign | static_cast<std::uint16_t>(r >> 13);
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

// The file's bytes, mapped read-only for the life of the Gguf.
struct Gguf::Mapping {
    const std::uint8_t* data = nullptr;
    std::uint64_t size = 0;
    ~Mapping() {
        if (data) munmap(const_cast<std::uint8_t*>(data), static_cast<std::size_t>(size));
    }
};

Gguf::Gguf(const std::filesystem::path& path) : path_(path), map_(std::make_shared<Mapping>()) {
    const std::string where = "gguf: " + path.string();
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) throw Error(where + ": cannot open file");
    struct stat st {};
    if (fstat(fd, &st) != 0) {
        ::close(fd);
        throw Error(where + ": cannot read file size");
    }
    map_->size = static_cast<std::uint64_t>(st.st_size);
    if (map_->size > 0) {
        void* p = mmap(nullptr, static_cast<std::size_t>(map_->size), PROT_READ, MAP_PRIVATE, fd, 0);
        if (p == MAP_FAILED) {
            ::close(fd);
            throw Error(where + ": cannot map file");
        }
        map_->data = static_cast<const std::uint8_t*>(p);
    }
    ::close(fd);
    const std::uint8_t* base = map_->data;
    if (map_->size < 4 || std::memcmp(base, "GGUF", 4) != 0) throw Error(where + ": not a GGUF file");
    Cursor c(base + 4, base + map_->size, where);
    version_ = c.u32("the version");
    if (version_ < 2 || version_ > 3) throw Error(where + ": GGUF version " + std::to_string(version_) + " is not supported (2 and 3 are)");
    const std::uint64_t tensors = c.u64("the tensor count"), entries = c.u64("the metadata count");
    // every metadata entry and tensor record takes well over 8 bytes
    if (tensors > c.remaining() / 8 || entries > c.remaining() / 8) {
        throw Error(where + ": truncated (" + std::to_string(tensors) + " tensors and " + std::to_string(entries) +
                    " metadata entries do not fit the file)");
    }
    for (std::uint64_t i = 0; i < entries; ++i) {
        std::string key = c.text("a metadata key");
        const std::uint32_t type = c.u32("a metadata type");
        metadata_.insert_or_assign(std::move(key), parse_value(c, type, 0));
    }
    struct Record {
        std::string name;
        Entry entry;
    };
    std::vector<Record> records;
    records.reserve(static_cast<std::size_t>(tensors));
    for (std::uint64_t i = 0; i < tensors; ++i) {
        Record r;
        r.name = c.text("a tensor name");
        const std::uint32_t dims = c.u32("a tensor's rank");
        if (dims > 4) c.malformed("tensor " + r.name + " has " + std::to_string(dims) + " dimensions (at most 4 are allowed)");
        r.entry.shape.assign(dims, 0);
        // GGUF lists the fastest-varying dimension first; Shape is row-major.
        for (std::uint32_t d = 0; d < dims; ++d) {
            const std::uint64_t n = c.u64("a tensor dimension");
            if (n > std::uint64_t(INT64_MAX)) c.malformed("tensor " + r.name + " has a dimension of " + std::to_string(n));
            r.entry.shape[dims - 1 - d] = static_cast<std::int64_t>(n);
        }
        r.entry.type = c.u32("a tensor type");
        r.entry.offset = c.u64("a tensor offset");
        records.push_back(std::move(r));
    }
    std::uint64_t alignment = 32;
    if (const auto it = metadata_.find("general.alignment"); it != metadata_.end() && it->second.is_number()) {
        alignment = static_cast<std::uint64_t>(it->second.number());
        // Any alignment up to 2^30 bytes, as the reference takes (GGUF writes powers of two).
        if (alignment == 0 || alignment > (std::uint64_t{1} << 30)) c.malformed("general.alignment is " + std::to_string(alignment));
    }
    const auto header_end = static_cast<std::uint64_t>(c.here() - base);
    data_start_ = (header_end + alignment - 1) / alignment * alignment;
    const std::uint64_t data_bytes = data_start_ <= map_->size ? map_->size - data_start_ : 0;
    for (Record& r : records) {
        std::uint64_t count = 1;
        bool overflow = false;
        for (const std::int64_t d : r.entry.shape) overflow |= __builtin_mul_overflow(count, static_cast<std::uint64_t>(d), &count);
        const auto [per_block, block_bytes] = ggml_block(r.entry.type);
        if (per_block) {
            const std::uint64_t blocks = count / per_block + (count % per_block ? 1 : 0);
            overflow |= __builtin_mul_overflow(blocks, block_bytes, &r.entry.bytes);
        }
        if (overflow) throw Error(where + ": tensor " + r.name + " is too large");
        if (r.entry.offset > data_bytes || r.entry.bytes > data_bytes - r.entry.offset) {
            throw Error(where + ": tensor " + r.name + " runs past the end of the file");
        }
        entries_.insert_or_assign(std::move(r.name), std::move(r.entry));
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

std::span<const std::uint8_t> Gguf::bytes(const std::string& name) const {
    const Entry& e = entry(name);
    return {map_->data + data_start_ + e.offset, static_cast<std::size_t>(e.bytes)};
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
                        const float v = std::clamp(std::nearbyint(x[4 * w + k] * inv), -127.0f, 127.0f);
                        word |= (std::uint32_t(std::int32_t(v)) & 0xFFu) << (8 * k);
                    }
                    words[group * 8 + w] = word;
                }
            }
        }
    });
}

}  // namespace vkml::detail
