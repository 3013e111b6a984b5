#pragma once

#include <cstdint>
#include <optional>
#include <span>
#include <vector>

#include "vkml/context.hpp"
#include "vkml/tensor.hpp"

// vkml's ops (reference: include/vkml/ops.hpp:16-163), each one or a few HIP
// kernels of libvkml_hip.so. Semantics and error messages follow the reference.
namespace vkml {

// Elementwise a OP b over f32; b has a's shape or its trailing dimensions and
// repeats over the leading ones.
Tensor add(const Tensor& a, const Tensor& b);
Tensor sub(const Tensor& a, const Tensor& b);
Tensor mul(const Tensor& a, const Tensor& b);
Tensor div(const Tensor& a, const Tensor& b);

Tensor silu(const Tensor& x);
Tensor gelu(const Tensor& x);
Tensor softcap(const Tensor& x, float cap);

// Softmax over the last dimension, f32; -inf entries become 0.
Tensor softmax(const Tensor& x);

// Index of each row's largest entry (the first of equal ones, NaNs skipped), i32.
Tensor argmax(const Tensor& x);

Tensor rms_norm(const Tensor& x, const Tensor& weight, float eps);

// f32 <-> f16/bf16 conversions (narrowing rounds to nearest even), f32 copy.
Tensor cast(const Tensor& x, DType dtype);

Tensor permute(const Tensor& x, std::vector<int> dims);
Tensor transpose(const Tensor& x, int dim0, int dim1);

// Rows of a [vocab, dim] f32/f16/bf16 table for i32 ids; out-of-range ids give zeros.
Tensor embedding(const Tensor& table, const Tensor& ids);

enum class RopeStyle : std::uint8_t {
    Interleaved,  // (2i, 2i + 1): Meta's LLaMA checkpoints and GGUF files
    RotateHalf,   // (i, i + dim / 2): HF transformers and GPT-NeoX
};

struct RopeScaling {
    float factor;
    float low_freq_factor;
    float high_freq_factor;
    std::int64_t original_max_positions;
};

// cos and sin of position * theta^(-2i / head_dim) (llama3 scaling and
// frequency divisors applied), f32 [max_positions, head_dim / 2, 2], computed
// on the host in double precision.
Tensor rope_table(Context& context, std::int64_t max_positions, std::int64_t head_dim, float theta,
                  std::optional<RopeScaling> scaling = std::nullopt, std::span<const float> freq_factors = {},
                  float magnitude = 1.0f);

// Rotary embedding of x [..., seq, heads, head_dim], f32, sequence index s at start_pos + s.
Tensor rope(const Tensor& x, const Tensor& table, std::int64_t start_pos, RopeStyle style);

// a [..., M, K] times b [K, N] (f32/f16/bf16) in f32, batched as the reference.
Tensor matmul(const Tensor& a, const Tensor& b);
// As matmul with b stored transposed, [N, K].
Tensor matmul_transposed(const Tensor& a, const Tensor& b);

// Quantized formats. q8_0, q4_0 and q4_1 are the reference's (32-value
// blocks, f16 scales; see the reference's ops.hpp:106-126 for the packing).
// q4_K is llama.cpp's q4_K kept in its 256-value super-blocks: values holds
// each super-block's 128 code bytes, scales its 16-byte header (f16 d, f16
// dmin, 12 bytes of 6-bit scales and mins). Its values are exactly those of
// the q4_1 matrix the reference repacks q4_K into (scale f16(d * sc), offset
// f16(-(dmin * m))), at 0.5625 bytes per weight instead of 0.625.
enum class QuantType : std::uint8_t { q8_0, q4_0, q4_1, q4_K };

struct QuantizedMatrix {
    Tensor values;  // i32 [rows, cols / 4] (q8_0) or [rows, cols / 8] (q4_0, q4_1, q4_K)
    Tensor scales;  // f16 or f32 [rows, cols / 32] ([.., 2] for q4_1); q4_K: i32 [rows, cols / 256, 4]
    std::int64_t rows = 0;
    std::int64_t cols = 0;
    QuantType type = QuantType::q8_0;
};

QuantizedMatrix quantize_q8(const Tensor& w);
QuantizedMatrix quantize_q4(const Tensor& w);
QuantizedMatrix quantize_q4_1(const Tensor& w);

Tensor dequantize(const QuantizedMatrix& q);

// Rows of a quantized table, decoded as dequantize would.
Tensor embedding(const QuantizedMatrix& table, const Tensor& ids);

// a [..., M, cols] times b transposed: [..., M, rows].
Tensor matmul_transposed(const Tensor& a, const QuantizedMatrix& b);

// softmax(q k^T / sqrt(head_dim)) v per head; q [heads, q_len, hd], k and v
// [kv_heads, kv_len, hd] (f32, or f16 for the decode kernel); grouped-query
// heads, causal masking, windows and soft caps as in the reference.
Tensor attention(const Tensor& q, const Tensor& k, const Tensor& v, bool causal, std::int64_t window = 0,
                 float softcap = 0.0f);

}  // namespace vkml
