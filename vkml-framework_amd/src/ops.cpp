// ops.cpp -- vkml's ops over the C ABI (the reference's src/ops/*.cpp). Each
// validates shapes and dtypes as the reference does, with its messages, then
// launches the HIP kernel(s) of libvkml_hip.so on the context's stream.
#include <algorithm>
#include <cmath>
#include <numbers>
#include <numeric>
#include <string>

#include "runtime.hpp"
#include "vkml/ops.hpp"

namespace vkml {

using detail::check;
using detail::TensorAccess;

namespace {

constexpr std::int64_t kGemvMaxRows = 8;


Tensor like(const Tensor& t, Shape shape, DType dtype) { return TensorAccess::empty(TensorAccess::runtime(t), std::move(shape), dtype); }

std::uint32_t u32(std::int64_t v) {
    if (v < 0 || v > 0xFFFFFFFFll) throw Error("vkml: size " + std::to_string(v) + " does not fit 32 bits");
    return static_cast<std::uint32_t>(v);
}

void require_f32(const char* name, const Tensor& x) {
    if (x.dtype() != DType::F32) throw Error(std::string(name) + ": no kernel for " + std::string(to_string(x.dtype())) + " yet");
}

Tensor binary(const char* name, std::uint32_t op, const Tensor& a, const Tensor& b) {
    if (a.dtype() != DType::F32 || b.dtype() != DType::F32) {
        throw Error(std::string(name) + ": f32 only for now, got " + std::string(to_string(a.dtype())) + " and " +
                    std::string(to_string(b.dtype())));
    }
    const Shape& as = a.shape();
    const Shape& bs = b.shape();
    const bool trailing = bs.size() <= as.size() && std::equal(bs.rbegin(), bs.rend(), as.rbegin());
    if (!trailing || (b.numel() == 0 && a.numel() != 0)) {
        throw Error(std::string(name) + ": cannot broadcast " + to_string(bs) + " to " + to_string(as));
    }
    Tensor out = like(a, as, DType::F32);
    if (a.numel() == 0) return out;
    check(vkml_binary(op, u32(a.numel()), u32(b.numel()), static_cast<const float*>(a.data()),
                      static_cast<const float*>(b.data()), static_cast<float*>(out.data())),
          name);
    return out;
}

Tensor unary(const char* name, std::uint32_t op, const Tensor& x, float param = 0.0f) {
    require_f32(name, x);
    Tensor out = like(x, x.shape(), DType::F32);
    if (x.numel() == 0) return out;
    check(vkml_unary(op, u32(x.numel()), param, static_cast<const float*>(x.data()), static_cast<float*>(out.data())), name);
    return out;
}

struct Rows {
    std::uint32_t rows, cols;
};

Rows row_shape(const char* name, const Tensor& x) {
    if (x.shape().empty()) throw Error(std::string(name) + ": input must have at least 1 dimension, got a scalar");
    require_f32(name, x);
    const std::int64_t cols = x.shape().back();
    return {u32(cols == 0 ? 0 : x.numel() / cols), u32(cols)};
}

std::uint32_t quant_code(QuantType t) {
    switch (t) {
        case QuantType::q8_0: return VKML_Q8_0;
        case QuantType::q4_0: return VKML_Q4_0;
        case QuantType::q4_1: return VKML_Q4_1;
        case QuantType::q4_K: return VKML_Q4_K;
    }
    return VKML_Q8_0;
}

std::uint32_t scale_code(const QuantizedMatrix& q) { return q.type == QuantType::q4_K ? std::uint32_t(VKML_F16) : detail::type_code(q.scales.dtype()); }

std::int64_t product(const Shape& s, std::size_t count) {
    std::int64_t p = 1;
    for (std::size_t i = 0; i < count; ++i) p *= s[i];
    return p;
}

QuantizedMatrix quantize(const char* name, const Tensor& w, QuantType quant, DType scale_type = DType::F16) {
    const Shape& s = w.shape();
    if (s.size() != 2 || w.dtype() == DType::I32) {
        throw Error(std::string(name) + ": expected a float matrix, got " + std::string(to_string(w.dtype())) + " " + to_string(s));
    }
    if (s[1] % 32 != 0) throw Error(std::string(name) + ": columns must be a multiple of 32, got " + to_string(s));
    const std::int64_t per_word = quant == QuantType::q8_0 ? 4 : 8;
    QuantizedMatrix q{.values = like(w, {s[0], s[1] / per_word}, DType::I32),
                      .scales = like(w, quant == QuantType::q4_1 ? Shape{s[0], s[1] / 32, 2} : Shape{s[0], s[1] / 32}, scale_type),
                      .rows = s[0],
                      .cols = s[1],
                      .type = quant};
    if (w.numel() == 0) return q;
    const vkml_quantize_params p{u32(w.numel() / 32), detail::type_code(w.dtype()), quant_code(quant), detail::type_code(scale_type)};
    check(vkml_quantize(&p, w.data(), q.values.data(), q.scales.data()), name);
    return q;
}

}  // namespace

namespace detail {
QuantizedMatrix quantize_q8_f32(const Tensor& x) { return quantize("quantize_q8", x, QuantType::q8_0, DType::F32); }
}  // namespace detail

Tensor add(const Tensor& a, const Tensor& b) { return binary("add", 0, a, b); }
Tensor sub(const Tensor& a, const Tensor& b) { return binary("sub", 1, a, b); }
Tensor mul(const Tensor& a, const Tensor& b) { return binary("mul", 2, a, b); }
Tensor div(const Tensor& a, const Tensor& b) { return binary("div", 3, a, b); }
Tensor silu(const Tensor& x) { return unary("silu", 0, x); }
Tensor gelu(const Tensor& x) { return unary("gelu", 1, x); }
Tensor softcap(const Tensor& x, float cap) {
    if (!(cap > 0.0f)) throw Error("softcap: the cap must be positive, got " + std::to_string(cap));
    return unary("softcap", 2, x, cap);
}

Tensor softmax(const Tensor& x) {
    const Rows r = row_shape("softmax", x);
    Tensor out = like(x, x.shape(), DType::F32);
    if (out.numel() == 0) return out;
    const vkml_softmax_params p{r.rows, r.cols, 1.0f, 0, 1, 0, 0, 0.0f, 0};
    check(vkml_softmax(&p, static_cast<const float*>(x.data()), static_cast<float*>(out.data())), "softmax");
    return out;
}

Tensor argmax(const Tensor& x) {
    const Rows r = row_shape("argmax", x);
    if (r.cols == 0) throw Error("argmax: the last dimension is empty");
    Tensor out = like(x, Shape(x.shape().begin(), x.shape().end() - 1), DType::I32);
    if (out.numel() == 0) return out;
    check(vkml_argmax(r.rows, r.cols, static_cast<const float*>(x.data()), static_cast<std::int32_t*>(out.data())), "argmax");
    return out;
}

Tensor rms_norm(const Tensor& x, const Tensor& weight, float eps) {
    const Rows r = row_shape("rms_norm", x);
    if (weight.shape() != Shape{x.shape().back()} || weight.dtype() != DType::F32) {
        throw Error("rms_norm: weight must be f32 " + to_string(Shape{x.shape().back()}) + " to match x " + to_string(x.shape()) +
                    ", got " + std::string(to_string(weight.dtype())) + " " + to_string(weight.shape()));
    }
    Tensor out = like(x, x.shape(), DType::F32);
    if (out.numel() == 0) return out;
    const vkml_rms_norm_params p{r.rows, r.cols, eps};
    check(vkml_rms_norm(&p, static_cast<const float*>(x.data()), static_cast<const float*>(weight.data()), static_cast<float*>(out.data())),
          "rms_norm");
    return out;
}

Tensor cast(const Tensor& x, DType dtype) {
    const bool ok = (dtype == DType::F32 && x.dtype() != DType::I32) ||
                    (x.dtype() == DType::F32 && (dtype == DType::F16 || dtype == DType::BF16));
    if (!ok) {
        throw Error("cast: " + std::string(to_string(x.dtype())) + " to " + std::string(to_string(dtype)) + " is not implemented yet");
    }
    Tensor out = like(x, x.shape(), dtype);
    if (x.numel() == 0) return out;
    check(vkml_cast(u32(x.numel()), detail::type_code(x.dtype()), detail::type_code(dtype), x.data(), out.data()), "cast");
    return out;
}

Tensor permute(const Tensor& x, std::vector<int> dims) {
    const Shape& s = x.shape();
    if (dims.size() != s.size() || s.size() > 6 || s.empty()) {
        throw Error("permute: dims of " + std::to_string(dims.size()) + " entries for " + to_string(s) + " (up to 6 dimensions)");
    }
    if (element_size(x.dtype()) != 4) throw Error("permute: 32-bit dtypes only, got " + std::string(to_string(x.dtype())));
    std::vector<bool> seen(dims.size());
    for (int& d : dims) {
        if (d < 0) d += static_cast<int>(dims.size());
        if (d < 0 || d >= static_cast<int>(dims.size()) || seen[static_cast<std::size_t>(d)]) throw Error("permute: dims must be a permutation");
        seen[static_cast<std::size_t>(d)] = true;
    }
    Shape out_shape;
    for (int d : dims) out_shape.push_back(s[static_cast<std::size_t>(d)]);
    Tensor out = like(x, out_shape, x.dtype());
    if (x.numel() == 0) return out;
    vkml_permute_params p{};
    p.rank = u32(static_cast<std::int64_t>(s.size()));
    p.count = u32(x.numel());
    for (std::size_t i = 0; i < s.size(); ++i) {
        p.in_shape[i] = u32(s[i]);
        p.dims[i] = static_cast<std::uint32_t>(dims[i]);
    }
    check(vkml_permute(&p, x.data(), out.data()), "permute");
    return out;
}

Tensor transpose(const Tensor& x, int dim0, int dim1) {
    const int rank = static_cast<int>(x.shape().size());
    if (dim0 < 0) dim0 += rank;
    if (dim1 < 0) dim1 += rank;
    if (dim0 < 0 || dim1 < 0 || dim0 >= rank || dim1 >= rank) throw Error("transpose: dimension out of range for " + to_string(x.shape()));
    std::vector<int> dims(static_cast<std::size_t>(rank));
    std::iota(dims.begin(), dims.end(), 0);
    std::swap(dims[static_cast<std::size_t>(dim0)], dims[static_cast<std::size_t>(dim1)]);
    return permute(x, dims);
}

Tensor embedding(const Tensor& table, const Tensor& ids) {
    if (table.shape().size() != 2 || table.dtype() == DType::I32 || ids.dtype() != DType::I32) {
        throw Error("embedding: expected a float [vocab, dim] table and i32 ids, got " + std::string(to_string(table.dtype())) + " " +
                    to_string(table.shape()) + " and " + std::string(to_string(ids.dtype())) + " ids");
    }
    Shape out_shape = ids.shape();
    out_shape.push_back(table.shape()[1]);
    Tensor out = like(table, out_shape, DType::F32);
    if (out.numel() == 0) return out;
    const vkml_embedding_params p{u32(out.numel()), u32(table.shape()[1]), u32(table.shape()[0]), detail::type_code(table.dtype()), VKML_F16};
    check(vkml_embedding(&p, table.data(), nullptr, static_cast<const std::int32_t*>(ids.data()), static_cast<float*>(out.data())), "embedding");
    return out;
}

Tensor rope_table(Context& context, std::int64_t max_positions, std::int64_t head_dim, float theta, std::optional<RopeScaling> scaling,
                  std::span<const float> freq_factors, float magnitude) {
    if (head_dim <= 0 || head_dim % 2 != 0 || max_positions < 0) {
        throw Error("rope_table: head_dim must be positive and even and max_positions non-negative, got head_dim " +
                    std::to_string(head_dim) + ", max_positions " + std::to_string(max_positions));
    }
    const auto half = static_cast<std::size_t>(head_dim / 2);
    std::vector<double> inv_freq(half);
    for (std::size_t i = 0; i < half; ++i) inv_freq[i] = std::pow(double(theta), -2.0 * double(i) / double(head_dim));
    if (!freq_factors.empty()) {
        if (freq_factors.size() != half) {
            throw Error("rope_table: " + std::to_string(freq_factors.size()) + " frequency factors for " + std::to_string(half) + " frequencies");
        }
        for (std::size_t i = 0; i < half; ++i) inv_freq[i] /= double(freq_factors[i]);
    }
    if (scaling) {
        const RopeScaling& s = *scaling;
        if (!(s.factor > 0 && s.low_freq_factor > 0 && s.high_freq_factor > s.low_freq_factor && s.original_max_positions > 0)) {
            throw Error("rope_table: rope scaling needs factor > 0, 0 < low_freq_factor < high_freq_factor and original_max_positions > 0");
        }
        const double old_len = double(s.original_max_positions);
        const double low_wavelen = old_len / s.low_freq_factor, high_wavelen = old_len / s.high_freq_factor;
        for (double& f : inv_freq) {
            const double wavelen = 2 * std::numbers::pi / f;
            if (wavelen > low_wavelen) {
                f /= s.factor;
            } else if (wavelen >= high_wavelen) {
                const double smooth = (old_len / wavelen - s.low_freq_factor) / (s.high_freq_factor - s.low_freq_factor);
                f = (1 - smooth) * f / s.factor + smooth * f;
            }
        }
    }
    std::vector<float> data(static_cast<std::size_t>(max_positions) * half * 2);
    for (std::size_t pos = 0; pos < static_cast<std::size_t>(max_positions); ++pos) {
        for (std::size_t i = 0; i < half; ++i) {
            const double angle = double(pos) * inv_freq[i];
            data[(pos * half + i) * 2] = static_cast<float>(magnitude * std::cos(angle));
            data[(pos * half + i) * 2 + 1] = static_cast<float>(magnitude * std::sin(angle));
        }
    }
    return Tensor::from_data<float>(context, data, {max_positions, head_dim / 2, 2});
}

Tensor rope(const Tensor& x, const Tensor& table, std::int64_t start_pos, RopeStyle style) {
    const Shape& xs = x.shape();
    if (xs.size() < 3 || x.dtype() != DType::F32) {
        throw Error("rope: x must be f32 [..., seq, heads, head_dim], got " + std::string(to_string(x.dtype())) + " " + to_string(xs));
    }
    const std::int64_t dim = xs[xs.size() - 1], heads = xs[xs.size() - 2], seq = xs[xs.size() - 3];
    const Shape& ts = table.shape();
    if (table.dtype() != DType::F32 || ts.size() != 3 || ts[1] * 2 > dim || ts[2] != 2) {
        throw Error("rope: x " + to_string(xs) + " does not match the table " + to_string(ts) + " from rope_table");
    }
    if (start_pos < 0 || start_pos + seq > ts[0]) {
        throw Error("rope: positions " + std::to_string(start_pos) + " to " + std::to_string(start_pos + seq - 1) +
                    " are outside the table's " + std::to_string(ts[0]) + " positions");
    }
    Tensor out = like(x, xs, DType::F32);
    if (out.numel() == 0) return out;
    const std::int64_t rows = out.numel() / dim;
    const vkml_rope_params p{u32(rows * ts[1]), u32(ts[1]), u32(dim), u32(heads), u32(seq), u32(start_pos),
                             u32(rows * (dim - 2 * ts[1])), style == RopeStyle::Interleaved ? 0u : 1u};
    check(vkml_rope(&p, static_cast<const float*>(x.data()), static_cast<const float*>(table.data()), static_cast<float*>(out.data())), "rope");
    return out;
}

namespace detail {

// a [..., M, K] times b [K, N] (or [N, K] transposed), b shared when 2-D,
// batched otherwise; b_group as the reference (src/ops/matmul.cpp:124-195).
Tensor matmul(const char* name, const Tensor& a, const Tensor& b, bool transposed, std::int64_t b_group, std::int64_t b_rows,
              std::int64_t causal_offset) {
    const Shape& as = a.shape();
    Shape bs = b.shape();
    const std::string b_desc = (transposed ? "transposed " : "") + to_string(bs);
    if (b_rows >= 0) {
        if (bs.size() != 3 || b_rows > bs[1]) throw Error(std::string(name) + ": cannot use the first " + std::to_string(b_rows) + " rows of " + b_desc);
        bs[1] = b_rows;
    }
    if (as.size() < 2 || bs.size() < 2) {
        throw Error(std::string(name) + ": both operands need at least 2 dimensions, got " + to_string(as) + " and " + to_string(bs));
    }
    if (a.dtype() != DType::F32 || b.dtype() == DType::I32) {
        throw Error(std::string(name) + ": no kernel for " + std::string(to_string(a.dtype())) + " x " + std::string(to_string(b.dtype())) + " yet");
    }
    const std::size_t rank = bs.size();
    const std::int64_t b_batch_elements = b.shape()[rank - 2] * b.shape()[rank - 1];
    const std::int64_t k = as.back();
    const std::int64_t b_k = transposed ? bs[rank - 1] : bs[rank - 2];
    const std::int64_t n = transposed ? bs[rank - 2] : bs[rank - 1];
    if (k != b_k) throw Error(std::string(name) + ": cannot multiply " + to_string(as) + " by " + b_desc);
    std::int64_t m = product(as, as.size() - 1), batches = 1, b_stride = 0;
    if (b_group > 1) {
        if (as.size() != 3 || rank != 3 || as[0] != bs[0] * b_group) {
            throw Error(std::string(name) + ": " + to_string(as) + " does not have " + std::to_string(b_group) + " batches per batch of " + b_desc);
        }
        batches = as[0];
        m = as[1];
        b_stride = b_batch_elements;
    } else if (rank > 2) {
        if (as.size() != rank || !std::equal(as.begin(), as.end() - 2, bs.begin())) {
            throw Error(std::string(name) + ": batch dimensions of " + to_string(as) + " and " + b_desc + " differ");
        }
        batches = product(as, as.size() - 2);
        m = as[as.size() - 2];
        b_stride = b_batch_elements;
    }
    Shape out_shape = as;
    out_shape.back() = n;
    Tensor out = like(a, out_shape, DType::F32);
    if (out.numel() == 0) return out;
    if (k == 0) {
        check(vkml_fill_u32(out.data(), 0u, static_cast<std::uint64_t>(out.numel())), name);
        return out;
    }
    // gemv.comp for a few rows against a transposed b, matmul.comp
    // otherwise (matmul.cpp:96), each batch z against b's z / b_group.
    const std::uint32_t group = u32(std::max<std::int64_t>(b_group, 1));
    if (transposed && m <= kGemvMaxRows) {
        const vkml_gemv_params p{u32(m), u32(n), u32(k), detail::type_code(b.dtype()), VKML_F16, u32(b_stride), group, u32(batches)};
        check(vkml_gemv(&p, static_cast<const float*>(a.data()), b.data(), static_cast<float*>(out.data()), nullptr), name);
        return out;
    }
    const vkml_matmul_params p{u32(m), u32(n), u32(k), u32(b_stride), group, u32(batches), transposed ? 1u : 0u,
                               detail::type_code(b.dtype()), VKML_F32, causal_offset >= 0 ? 1u : 0u,
                               u32(std::max<std::int64_t>(causal_offset, 0))};
    check(vkml_matmul(&p, static_cast<const float*>(a.data()), b.data(), static_cast<float*>(out.data()), nullptr), name);
    return out;
}

}  // namespace detail

Tensor matmul(const Tensor& a, const Tensor& b) { return detail::matmul("matmul", a, b, false); }
Tensor matmul_transposed(const Tensor& a, const Tensor& b) { return detail::matmul("matmul_transposed", a, b, true); }

QuantizedMatrix quantize_q8(const Tensor& w) { return quantize("quantize_q8", w, QuantType::q8_0); }
QuantizedMatrix quantize_q4(const Tensor& w) { return quantize("quantize_q4", w, QuantType::q4_0); }
QuantizedMatrix quantize_q4_1(const Tensor& w) { return quantize("quantize_q4_1", w, QuantType::q4_1); }

Tensor dequantize(const QuantizedMatrix& q) {
    Tensor out = like(q.values, {q.rows, q.cols}, DType::F32);
    if (out.numel() == 0) return out;
    const vkml_dequantize_params p{u32(out.numel()), quant_code(q.type), scale_code(q), u32(q.cols)};
    check(vkml_dequantize(&p, q.values.data(), q.scales.data(), static_cast<float*>(out.data())), "dequantize");
    return out;
}

Tensor embedding(const QuantizedMatrix& table, const Tensor& ids) {
    if (ids.dtype() != DType::I32) throw Error("embedding: ids must be i32, got " + std::string(to_string(ids.dtype())));
    Shape out_shape = ids.shape();
    out_shape.push_back(table.cols);
    Tensor out = like(table.values, out_shape, DType::F32);
    if (out.numel() == 0) return out;
    const vkml_embedding_params p{u32(out.numel()), u32(table.cols), u32(table.rows), quant_code(table.type), scale_code(table)};
    check(vkml_embedding(&p, table.values.data(), table.scales.data(), static_cast<const std::int32_t*>(ids.data()),
                         static_cast<float*>(out.data())),
          "embedding");
    return out;
}

Tensor matmul_transposed(const Tensor& a, const QuantizedMatrix& b) {
    const Shape& as = a.shape();
    if (as.size() < 2 || a.dtype() != DType::F32 || as.back() != b.cols) {
        throw Error("matmul_transposed: cannot multiply " + std::string(to_string(a.dtype())) + " " + to_string(as) +
                    " by a quantized matrix of " + std::to_string(b.rows) + " rows and " + std::to_string(b.cols) + " columns");
    }
    Shape out_shape = as;
    out_shape.back() = b.rows;
    Tensor out = like(a, out_shape, DType::F32);
    if (out.numel() == 0) return out;
    const std::int64_t m = product(as, as.size() - 1);
    const std::uint32_t type = quant_code(b.type), st = scale_code(b);
    detail::Runtime& rt = TensorAccess::runtime(a);
    const bool dot_ok = b.cols % (b.type == QuantType::q4_K ? 256 : 32) == 0;  // every matrix the reference's int8 path takes
    float* c = static_cast<float*>(out.data());
    if (rt.integer_dot() && dot_ok && m == 1 && b.cols <= 4096) {
        // One row: the Q8_0 of a computed inside the GEMV (one launch).
        const vkml_gemv_fused_params p{u32(b.rows), u32(b.cols), type, st, 0, 2, 0.0f, 0};
        check(vkml_gemv_fused(&p, a.data(), nullptr, nullptr, b.values.data(), b.scales.data(), nullptr, nullptr, nullptr, c, nullptr,
                              nullptr),
              "matmul_transposed");
        return out;
    }
    if (rt.integer_dot() && dot_ok) {
        // Quantize a too and multiply int8 by int8 (matmul.cpp:225-259):
        // gemv_dot for up to 8 rows, matmul_dot on the matrix cores beyond.
        const QuantizedMatrix aq = detail::quantize_q8_f32(a.reshape({m, b.cols}));
        const vkml_gemv_dot_params p{u32(m), u32(b.rows), u32(b.cols), type, st};
        const auto* av = aq.values.data();
        const auto* as_ = static_cast<const float*>(aq.scales.data());
        if (m <= kGemvMaxRows) check(vkml_gemv_dot(&p, av, b.values.data(), c, b.scales.data(), as_), "matmul_transposed");
        else check(vkml_matmul_dot(&p, av, b.values.data(), c, b.scales.data(), as_), "matmul_transposed");
        return out;
    }
    // f32 a against the widened weights: gemv.comp for up to 8 rows,
    // matmul.comp beyond (matmul.cpp:96, 263-270).
    if (m <= kGemvMaxRows) {
        const vkml_gemv_params p{u32(m), u32(b.rows), u32(b.cols), type, st, 0, 1, 1};
        check(vkml_gemv(&p, static_cast<const float*>(a.data()), b.values.data(), c, b.scales.data()), "matmul_transposed");
    } else {
        const vkml_matmul_params p{u32(m), u32(b.rows), u32(b.cols), 0, 1, 1, 1, type, st, 0, 0};
        check(vkml_matmul(&p, static_cast<const float*>(a.data()), b.values.data(), c, b.scales.data()), "matmul_transposed");
    }
    return out;
}

namespace detail {

// Decode attention for one query per head (attention.cpp:40-84): the
// chunked kernel (128 keys a chunk, as the reference) and its merge.
Tensor attend_one_query(const Tensor& q, const Tensor& k_cache, const Tensor& v_cache, std::int64_t kv_start, std::int64_t kv_len,
                        float softcap) {
    const std::int64_t heads = q.shape()[0], hd = q.shape()[2], kv_heads = k_cache.shape()[0], capacity = k_cache.shape()[1];
    const std::int64_t chunks = (kv_len - kv_start + 127) / 128;
    Tensor partial = like(q, {heads, chunks, hd}, DType::F32);
    Tensor stats = like(q, {heads, chunks, 2}, DType::F32);
    Tensor out = like(q, {heads, 1, hd}, DType::F32);
    const vkml_attend_params p{u32(kv_start), u32(kv_len), u32(capacity), u32(heads), u32(kv_heads), u32(hd), type_code(k_cache.dtype()),
                               u32(chunks), 1.0f / std::sqrt(static_cast<float>(hd)), softcap};
    check(vkml_attend(&p, static_cast<const float*>(q.data()), k_cache.data(), v_cache.data(), static_cast<float*>(partial.data()),
                      static_cast<float*>(stats.data()), nullptr),
          "attention");
    check(vkml_attend_merge(&p, static_cast<const float*>(partial.data()), static_cast<const float*>(stats.data()),
                            static_cast<float*>(out.data()), nullptr, nullptr),
          "attention");
    return out;
}

// Rows start.. of every batch of src [B, *, width] into rows at.. of dst
// [B, *, width], 32-bit words (attention.cpp:103-122).
void copy_rows(const Tensor& src, std::int64_t start, const Tensor& dst, std::int64_t at, std::int64_t rows) {
    const std::int64_t batches = src.shape()[0], width = src.shape()[2] * std::int64_t(element_size(src.dtype())) / 4;
    const vkml_copy_rows_params p{u32(batches * rows * width), u32(rows * width), u32(src.shape()[1] * width), u32(start * width),
                                  u32(dst.shape()[1] * width), u32(at * width)};
    if (p.count == 0) return;
    check(vkml_copy_rows(&p, src.data(), const_cast<void*>(dst.data())), "attention");
}

// attention_block (attention.cpp:127-138): scores q k^T over keys 0..keys
// of the caches, the causal softmax with query i at key position keys -
// rows + i, then probs v.
Tensor attention_block(const Tensor& q, const Tensor& k_cache, const Tensor& v_cache, std::int64_t keys, bool causal,
                       std::int64_t window, float softcap) {
    const std::int64_t heads = q.shape()[0], rows = q.shape()[1], hd = q.shape()[2];
    const std::int64_t group = heads / k_cache.shape()[0];
    const Tensor scores = matmul("attention", q, k_cache, true, group, keys);
    Tensor probs = like(q, scores.shape(), DType::F32);
    if (probs.numel() > 0) {
        const vkml_softmax_params p{u32(heads * rows), u32(keys), 1.0f / std::sqrt(static_cast<float>(hd)), causal ? 1u : 0u,
                                    u32(rows), u32(keys - rows), u32(window), softcap, 0};
        check(vkml_softmax(&p, static_cast<const float*>(scores.data()), static_cast<float*>(probs.data())), "attention");
    }
    return matmul("attention", probs, v_cache, false, group, keys);
}

// detail::attention for more than one query (attention.cpp:205-226). The
// reference runs the queries in chunks whose scores [heads, rows, kv_len]
// f32 fit max_score_bytes (whole 64s of rows when at least 64), each
// against the keys its last query sees. What the chunks fix is only which
// queries' scores go through gemv.comp's order (a chunk of 8 rows or
// fewer); keys past a chunk's last query carry probability exactly 0 and
// add nothing. So the rows of chunks of more than 8 are run here in pieces
// of this build's own budget (HBM is large), with the work the causal mask
// makes moot skipped, and the rest as the reference's chunks. piece_bytes
// defaults to 1 GiB: the reference's 64 MiB budget is sized for integrated
// GPUs, and MI355X has 288 GB of HBM.
Tensor attention_prompt(const Tensor& q, const Tensor& k_cache, const Tensor& v_cache, std::int64_t kv_len, bool causal,
                        std::int64_t window, float softcap, std::int64_t max_score_bytes, std::int64_t piece_bytes) {
    const std::int64_t heads = q.shape()[0], q_len = q.shape()[1], hd = q.shape()[2];
    const std::int64_t row_bytes = heads * std::max<std::int64_t>(kv_len, 1) * 4;
    std::int64_t chunk = std::max<std::int64_t>(1, max_score_bytes / row_bytes);
    if (chunk >= 64) chunk -= chunk % 64;
    if (q_len <= chunk && (q_len <= kGemvMaxRows || !causal)) return attention_block(q, k_cache, v_cache, kv_len, causal, window, softcap);
    const std::int64_t first = kv_len - q_len;  // key position of query 0
    Tensor out = like(q, q.shape(), DType::F32);
    const auto reference_chunk = [&](std::int64_t q0, std::int64_t rows) {
        const std::int64_t keys = causal ? first + q0 + rows : kv_len;
        Tensor part = like(q, {heads, rows, hd}, DType::F32);
        copy_rows(q, q0, part, 0, rows);
        copy_rows(attention_block(part, k_cache, v_cache, keys, causal, window, softcap), 0, out, q0, rows);
    };
    if (chunk <= kGemvMaxRows || !causal) {
        for (std::int64_t q0 = 0; q0 < q_len; q0 += chunk) reference_chunk(q0, std::min(chunk, q_len - q0));
        return out;
    }
    const std::int64_t tail = q_len > chunk ? q_len % chunk : 0;
    const std::int64_t gemv_rows = tail <= kGemvMaxRows ? tail : 0;
    const std::int64_t rows_all = q_len - gemv_rows;
    const std::int64_t group = heads / k_cache.shape()[0];
    std::int64_t piece = std::max<std::int64_t>(64, piece_bytes / row_bytes);
    piece -= piece % 64;
    for (std::int64_t r0 = 0; r0 < rows_all;) {
        std::int64_t rows = std::min(piece, rows_all - r0);
        if (rows_all - r0 - rows <= kGemvMaxRows) rows = rows_all - r0;  // no piece of 8 rows or fewer
        const std::int64_t keys = first + r0 + rows;
        Tensor part = q;
        if (rows != q_len) {
            part = like(q, {heads, rows, hd}, DType::F32);
            copy_rows(q, r0, part, 0, rows);
        }
        const Tensor scores = matmul("attention", part, k_cache, true, group, keys, first + r0);
        Tensor probs = like(q, scores.shape(), DType::F32);
        const vkml_softmax_params sp{u32(heads * rows), u32(keys), 1.0f / std::sqrt(static_cast<float>(hd)), 1u, u32(rows),
                                     u32(first + r0), u32(window), softcap, 0};
        check(vkml_softmax(&sp, static_cast<const float*>(scores.data()), static_cast<float*>(probs.data())), "attention");
        const Tensor o = matmul("attention", probs, v_cache, false, group, keys, first + r0);
        if (rows == q_len) return o;
        copy_rows(o, 0, out, r0, rows);
        r0 += rows;
    }
    if (gemv_rows) reference_chunk(rows_all, gemv_rows);
    return out;
}

std::int64_t sliding_rows(std::int64_t heads, std::int64_t t, std::int64_t q0, std::int64_t start, std::int64_t ring, std::int64_t window,
                          std::int64_t max_score_bytes) {
    // Rows written for positions up to the piece's end overwrite those
    // before end - ring, which its first query no longer needs as long as
    // they are before its window, or no row wraps yet.
    const std::int64_t first = start + q0;
    std::int64_t rows = std::max(ring - window + 1, ring - first);
    const std::int64_t keys = std::min(first + rows, ring);
    rows = std::min(rows, std::max<std::int64_t>(1, max_score_bytes / (heads * keys * 4)));
    if (rows >= 64) rows -= rows % 64;  // whole blocks of the tiled matmul
    return std::min(rows, t - q0);
}

Tensor ring_attention(const Tensor& q, const Tensor& k_ring, const Tensor& v_ring, std::int64_t first, std::int64_t window, float softcap) {
    const std::int64_t heads = q.shape()[0], rows = q.shape()[1], hd = q.shape()[2], ring = k_ring.shape()[1];
    const std::int64_t end = first + rows;
    if (rows == 1) return attend_one_query(q, k_ring, v_ring, std::max<std::int64_t>(0, end - window), end, softcap);
    // attention_block with the ring mask (attention.cpp:127-138): every row
    // of the ring written so far, in column order
    const std::int64_t keys = std::min(end, ring), group = heads / k_ring.shape()[0];
    const Tensor scores = matmul("attention", q, k_ring, true, group, keys);
    Tensor probs = like(q, scores.shape(), DType::F32);
    const vkml_softmax_params p{u32(heads * rows), u32(keys), 1.0f / std::sqrt(static_cast<float>(hd)), 1u, u32(rows), u32(first),
                                u32(window), softcap, u32(ring)};
    check(vkml_softmax(&p, static_cast<const float*>(scores.data()), static_cast<float*>(probs.data())), "attention");
    return matmul("attention", probs, v_ring, false, group, keys);
}

Tensor sliding_attention(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& k_ring, const Tensor& v_ring, std::int64_t start,
                         std::int64_t window, std::int64_t max_score_bytes, float softcap) {
    const Shape& qs = q.shape();
    const Shape& ks = k_ring.shape();
    const bool shapes = qs.size() == 3 && ks.size() == 3 && k.shape().size() == 3 && v.shape() == k.shape() && v_ring.shape() == ks &&
                        k.shape()[0] == ks[0] && k.shape()[1] == qs[1] && k.shape()[2] == qs[2] && ks[2] == qs[2] && ks[0] > 0 &&
                        qs[0] % ks[0] == 0;
    if (!shapes || k.dtype() != k_ring.dtype() || v.dtype() != k_ring.dtype() || v_ring.dtype() != k_ring.dtype()) {
        throw Error("sliding_attention: cannot append " + std::string(to_string(k.dtype())) + " k " + to_string(k.shape()) + " and " +
                    std::string(to_string(v.dtype())) + " v " + to_string(v.shape()) + " to " + std::string(to_string(k_ring.dtype())) +
                    " and " + std::string(to_string(v_ring.dtype())) + " caches " + to_string(ks) + " for q " + to_string(qs));
    }
    const std::int64_t ring = ks[1], t = qs[1], heads = qs[0];
    if (window < 1 || window > ring || start < 0) {
        throw Error("sliding_attention: a window of " + std::to_string(window) + " keys must be positive and fit a ring of " +
                    std::to_string(ring) + " rows, from position " + std::to_string(start));
    }
    // positions from.. of rows row.. of src into the ring, in at most two
    // pieces where it wraps around
    const auto append = [&](const Tensor& src, const Tensor& cache, std::int64_t row, std::int64_t from, std::int64_t n) {
        const std::int64_t at = from % ring, head = std::min(n, ring - at);
        copy_rows(src, row, cache, at, head);
        copy_rows(src, row + head, cache, 0, n - head);
    };
    Tensor out = like(q, qs, DType::F32);
    for (std::int64_t q0 = 0; q0 < t;) {
        const std::int64_t rows = sliding_rows(heads, t, q0, start, ring, window, max_score_bytes);
        append(k, k_ring, q0, start + q0, rows);
        append(v, v_ring, q0, start + q0, rows);
        Tensor qc = q;
        if (rows != t) {
            qc = like(q, {heads, rows, qs[2]}, DType::F32);
            copy_rows(q, q0, qc, 0, rows);
        }
        const Tensor block = ring_attention(qc, k_ring, v_ring, start + q0, window, softcap);
        if (rows == t) return block;
        copy_rows(block, 0, out, q0, rows);
        q0 += rows;
    }
    return out;
}

}  // namespace detail

Tensor attention(const Tensor& q, const Tensor& k, const Tensor& v, bool causal, std::int64_t window, float softcap) {
    const Shape& qs = q.shape();
    const Shape& ks = k.shape();
    if (qs.size() != 3 || ks.size() != 3 || v.shape().size() != 3) {
        throw Error("attention: q, k and v must be [heads, seq, head_dim], got " + to_string(qs) + ", " + to_string(ks) + " and " +
                    to_string(v.shape()));
    }
    const std::int64_t heads = qs[0], q_len = qs[1], hd = qs[2], kv_heads = ks[0], kv_len = ks[1];
    if (ks[2] != hd || v.shape() != ks) {
        throw Error("attention: k " + to_string(ks) + " and v " + to_string(v.shape()) + " must match each other and q's head_dim in " + to_string(qs));
    }
    if (kv_heads == 0 || heads % kv_heads != 0) {
        throw Error("attention: q's " + std::to_string(heads) + " heads must be a multiple of k and v's " + std::to_string(kv_heads));
    }
    if (window < 0 || (window > 0 && !causal)) {
        throw Error("attention: a window of " + std::to_string(window) + " keys needs causal attention and must not be negative");
    }
    if (causal && q_len > kv_len) {
        throw Error("attention: " + std::to_string(q_len) + " queries is more queries than the " + std::to_string(kv_len) +
                    " keys a causal mask can place them among");
    }
    if (q.dtype() != DType::F32 || k.dtype() != v.dtype() || (k.dtype() != DType::F32 && k.dtype() != DType::F16)) {
        throw Error("attention: q must be f32 and k, v both f32 or both f16");
    }
    const std::int64_t group = heads / kv_heads;
    const bool fused = q_len == 1 && kv_len > 0 && (hd == 64 || hd == 128 || hd == 256) && (group == 1 || group == 2 || group == 4 || group == 8);
    if (fused) {
        const std::int64_t start = window > 0 && kv_len > window ? kv_len - window : 0;
        return detail::attend_one_query(q, k, v, start, kv_len, softcap);
    }
    return detail::attention_prompt(q, k, v, kv_len, causal, window, softcap, detail::kMaxScoreBytes);
}

}  // namespace vkml
