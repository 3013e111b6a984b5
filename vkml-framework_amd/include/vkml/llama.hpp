#pragma once

#include <cstdint>
#include <filesystem>
#include <memory>
#include <optional>
#include <span>
#include <variant>
#include <vector>

#include "vkml/context.hpp"
#include "vkml/ops.hpp"
#include "vkml/tensor.hpp"

namespace vkml {

enum class Activation : std::uint8_t { silu, gelu_tanh };

// A LLaMA-architecture model's hyperparameters (reference: include/vkml/
// llama.hpp:29-116). This build runs the GGUF "llama" architecture (LLaMA,
// Mistral, TinyLlama, SmolLM); the fields for other families are kept so the
// struct matches, and a config that sets them is refused with an Error
// rather than run wrongly.
struct LlamaConfig {
    std::int64_t vocab_size = 0;
    std::int64_t hidden_size = 0;
    std::int64_t intermediate_size = 0;
    std::int64_t num_layers = 0;
    std::int64_t num_heads = 0;
    std::int64_t num_kv_heads = 0;
    std::int64_t head_dim = 0;
    std::int64_t max_positions = 0;
    float rms_norm_eps = 1e-5f;
    float rope_theta = 10000.0f;
    bool tie_word_embeddings = false;
    Activation activation = Activation::silu;
    bool qkv_bias = false;
    bool o_bias = false;
    bool qk_norm = false;
    std::vector<std::int32_t> eos_token_ids;
    std::optional<RopeScaling> rope_scaling;
    float rope_linear_factor = 1.0f;
    RopeStyle rope_style = RopeStyle::RotateHalf;
    std::vector<float> rope_freq_factors;
    std::optional<std::int64_t> sliding_window;
    std::vector<bool> sliding_layers;
    std::vector<bool> rope_layers;
    std::int64_t rotary_dim = 0;
    float embedding_scale = 1.0f;
    float norm_weight_offset = 0.0f;
    bool sandwich_norms = false;
    bool pre_norms = true;
    bool qk_norm_whole = false;
    std::optional<float> query_pre_attn_scalar;
    float attn_logit_softcap = 0.0f;
    float final_logit_softcap = 0.0f;
    float residual_scale = 1.0f;
    float logit_divisor = 1.0f;

    // From a GGUF file's metadata (reference: src/models/config.cpp:14-140).
    static LlamaConfig from_gguf(const std::filesystem::path& path);
};

struct LlamaOptions {
    // Quantize float weight matrices while loading (matrices whose width is a
    // multiple of 32; the output projection gets q8_0 unless q8_0 is asked).
    std::optional<QuantType> quantize;
    // The KV cache's element type: f32 (the reference's default) or f16.
    DType kv_cache = DType::F32;
    // A sliding window's caches are rings of window + this many rows (at
    // most the context), so that a prompt's keys append in large pieces and
    // rewinding that far keeps the window (reference: llama.hpp:133).
    std::int64_t sliding_extra_rows = 1024;
    // Replay each decode step as a captured HIP graph.
    bool use_graphs = true;
    // int8 activations for this model's quantized weights, when the Context
    // allows them too (ContextOptions::integer_dot_product).
    bool integer_dot_product = true;
    // The f32 scores one piece of a prompt's attention may hold ([heads,
    // queries, keys]); longer prompts run in pieces of whole 64s of queries.
    // The results do not depend on it (the reference's own 64 MiB chunks
    // decide which queries take gemv's order).
    std::int64_t prompt_score_bytes = std::int64_t{1} << 30;
    // Decode attention on the matrix cores: f32 attention to within f32
    // rounding, not the reference's order of f32 operations (so logits are
    // no longer its bits). f16 caches, head_dim 64 or 128, no sliding
    // window; other models keep the exact kernels. Off by default.
    bool fast_attention = false;
    // A sliding window over every layer and the attention / final logit
    // soft caps (0: none). The reference takes these from Gemma files only
    // (config.cpp:114-133) and ignores them in a llama file, as from_gguf
    // does here; a llama model gets them from these options.
    std::int64_t sliding_window = 0;
    float attn_logit_softcap = 0.0f;
    float final_logit_softcap = 0.0f;
};

class Llama {
public:
    // Loads a GGUF file: its metadata and tensors (f32, f16, bf16, q8_0,
    // q4_0, q4_1 and q4_K kept as they are; q6_K and the other k-quants
    // requantized to q8_0 on the host, as the reference does).
    static Llama load(Context& context, const std::filesystem::path& path, std::int64_t context_length,
                      LlamaOptions options = {});

    Llama(Llama&&) noexcept;
    Llama& operator=(Llama&&) noexcept;
    ~Llama();

    const LlamaConfig& config() const noexcept;
    std::int64_t context_length() const noexcept;
    std::int64_t position() const noexcept;

    // Runs tokens after those already processed; logits of the last, [vocab_size].
    Tensor forward(std::span<const std::int32_t> tokens);
    // Logits of every token, [tokens, vocab_size].
    Tensor forward_all(std::span<const std::int32_t> tokens);

    // Greedy decoding on the device: feeds `first` and then each argmax back
    // for `count` steps without waiting on the host between them, and returns
    // the `count` tokens chosen (each step's argmax). Same result as calling
    // argmax(forward({&next, 1})) count times.
    std::vector<std::int32_t> generate_greedy(std::int32_t first, std::int64_t count);

    void reset() noexcept;
    std::int64_t rewind(std::int64_t position);
    // Moves the sequence forward to position (at most the context length)
    // without running the tokens in between: the KV-cache rows of those
    // positions keep what they hold (zeros in a fresh model, or an earlier
    // sequence's keys and values). No counterpart in the reference: for
    // benchmarks and tests that time decode steps at a given position.
    std::int64_t advance(std::int64_t position);
    std::int64_t kv_cache_bytes() const noexcept;

    // The layer-l KV caches [kv_heads, context_length, head_dim], for tests.
    const Tensor& k_cache(std::int64_t layer) const;
    const Tensor& v_cache(std::int64_t layer) const;

    struct Impl;

private:
    explicit Llama(std::unique_ptr<Impl> impl);
    std::unique_ptr<Impl> impl_;
};

}  // namespace vkml
