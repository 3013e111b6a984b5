// llama.cpp -- the Llama model on the MI355X: GGUF loading and the token
// loop (the reference's src/models/llama.cpp:140-406, weights.cpp:26-159 and
// config.cpp:14-140).
//
// The reference records ~29 dispatches per layer, each separated by a full
// barrier. Here one decode step (t = 1) is six kernels per layer on the int8
// path, all reading the step's token and position from a small device-side
// state:
//   q|k|v GEMV (one fused matrix; rms_norm + Q8_0 of x in its prologue) ->
//   attention chunks (rope of q and k, f16 cast and KV append inside) ->
//   merge + Q8_0 -> o GEMV + residual -> gate|up GEMV (rms_norm + Q8_0
//   prologue, SwiGLU + Q8_0 epilogue) -> down GEMV + residual,
// then the final norm, the lm_head GEMV and (greedy) an argmax that writes
// the next token into the state. The step is captured once as a HIP graph
// and replayed, so a greedy generation is a stream of graph launches with no
// host round trip between tokens. A prompt of several tokens runs at once,
// as the reference's Llama::run does (prefill below).
#include <algorithm>
#include <map>
#include <cmath>
#include <cstring>
#include <numeric>

#include "gguf.hpp"
#include "runtime.hpp"
#include "vkml/llama.hpp"

namespace vkml {

using detail::check;
using detail::Gguf;
using detail::TensorAccess;

namespace {

std::uint32_t u32(std::int64_t v) { return static_cast<std::uint32_t>(v); }

// A loaded weight matrix: float as stored, or quantized.
struct Weight {
    bool quantized = false;
    Tensor t;           // float: f32, f16 or bf16 [rows, cols]
    QuantizedMatrix q;  // quantized
    std::int64_t rows = 0, cols = 0;

    std::uint32_t type_code() const {
        if (!quantized) return detail::type_code(t.dtype());
        switch (q.type) {
            case QuantType::q8_0: return VKML_Q8_0;
            case QuantType::q4_0: return VKML_Q4_0;
            case QuantType::q4_1: return VKML_Q4_1;
            case QuantType::q4_K: return VKML_Q4_K;
        }
        return VKML_Q8_0;
    }
    std::uint32_t scale_code() const { return q.type == QuantType::q4_K ? std::uint32_t(VKML_F16) : detail::type_code(q.scales.dtype()); }
    const void* values() const { return quantized ? q.values.data() : t.data(); }
    const void* scales() const { return quantized ? q.scales.data() : nullptr; }
    // The int8 path takes K a multiple of 32 (q4_K: 256), as the reference's
    // (matmul.cpp:226-259); above VKML_GEMV_STAGED_MAX_K only gemv_dot and
    // gemv_dot_add, whose rows kernel reads the activation from memory.
    bool int_dot_ok() const { return quantized && cols % (q.type == QuantType::q4_K ? 256 : 32) == 0; }
    bool staged_ok() const { return int_dot_ok() && cols <= VKML_GEMV_STAGED_MAX_K; }
};

// Host-side form of a matrix before upload: bytes of values and scales.
struct HostMatrix {
    bool quantized = false;
    QuantType type = QuantType::q8_0;
    DType dtype = DType::F32;  // float matrices
    std::vector<std::uint8_t> values, scales;
    std::int64_t rows = 0, cols = 0;
};

// gguf.cpp:525-638 (load_quantized) and 503-523 (load_q8): a file's matrix
// in QuantizedMatrix's layout. q4_K keeps its super-blocks, split into code
// bytes and 16-byte headers.
HostMatrix host_matrix(const Gguf& file, const std::string& name, std::int64_t rows, std::int64_t cols) {
    const Gguf::Entry& e = file.entry(name);
    if (e.shape != Shape{rows, cols}) {
        throw Error("Llama: weight " + name + " is " + to_string(e.shape) + ", but the config needs " + to_string(Shape{rows, cols}));
    }
    const std::span<const std::uint8_t> data = file.bytes(name);
    HostMatrix m;
    m.rows = rows;
    m.cols = cols;
    const std::size_t count = std::size_t(rows * cols);
    if (e.type == detail::kGgmlF32 || e.type == detail::kGgmlF16 || e.type == detail::kGgmlBF16) {
        m.dtype = e.type == detail::kGgmlF32 ? DType::F32 : e.type == detail::kGgmlF16 ? DType::F16 : DType::BF16;
        m.values.assign(data.begin(), data.end());
        return m;
    }
    m.quantized = true;
    const std::size_t groups = count / 32;
    const auto pack = [](std::uint8_t* out, const std::uint8_t codes[32]) {
        for (int w = 0; w < 4; ++w)
            for (int k = 0; k < 4; ++k) out[4 * w + k] = std::uint8_t(codes[8 * w + k] | (codes[8 * w + k + 4] << 4));
    };
    switch (e.type) {
        case detail::kGgmlQ8_0:
        case detail::kGgmlQ4_0:
        case detail::kGgmlQ4_1: {
            if (cols % 32) throw Error("gguf: tensor \"" + name + "\" of shape " + to_string(e.shape) + " is not a matrix of whole blocks");
            const bool q8 = e.type == detail::kGgmlQ8_0, offset = e.type == detail::kGgmlQ4_1;
            const std::size_t bsize = q8 ? 34 : offset ? 20 : 18;
            m.type = q8 ? QuantType::q8_0 : offset ? QuantType::q4_1 : QuantType::q4_0;
            m.values.resize(groups * (q8 ? 32 : 16));
            m.scales.resize(groups * 2 * (offset ? 2 : 1));
            auto* halves = reinterpret_cast<std::uint16_t*>(m.scales.data());
            detail::parallel_for(groups, [&](std::size_t begin, std::size_t end) {
                for (std::size_t b = begin; b < end; ++b) {
                    const std::uint8_t* block = data.data() + b * bsize;
                    if (offset) {
                        std::memcpy(&halves[2 * b], block, 4);
                    } else {
                        std::memcpy(&halves[b], block, 2);
                    }
                    if (q8) {
                        std::memcpy(&m.values[b * 32], block + 2, 32);
                    } else {
                        const std::uint8_t* qs = block + (offset ? 4 : 2);
                        std::uint8_t codes[32];
                        for (int j = 0; j < 16; ++j) {
                            codes[j] = qs[j] & 0x0F;
                            codes[j + 16] = qs[j] >> 4;
                        }
                        pack(&m.values[b * 16], codes);
                    }
                }
            });
            return m;
        }
        case detail::kGgmlQ4_K: {
            if (cols % 256) throw Error("gguf: tensor \"" + name + "\" of shape " + to_string(e.shape) + " is not a matrix of whole blocks");
            m.type = QuantType::q4_K;
            const std::size_t blocks = count / 256;
            m.values.resize(blocks * 128);
            m.scales.resize(blocks * 16);
            detail::parallel_for(blocks, [&](std::size_t begin, std::size_t end) {
                for (std::size_t b = begin; b < end; ++b) {
                    std::memcpy(&m.scales[b * 16], data.data() + b * 144, 16);
                    std::memcpy(&m.values[b * 128], data.data() + b * 144 + 16, 128);
                }
            });
            return m;
        }
        default: {
            // q6_K and the other k-quants: decoded and requantized to Q8_0
            // on the host, finer than any of them (weights.cpp:146-148).
            if (cols % 32) throw Error("gguf: tensor \"" + name + "\" of shape " + to_string(e.shape) + " is not a matrix of whole Q8_0 blocks");
            m.type = QuantType::q8_0;
            m.values.resize(count);
            m.scales.resize(groups * 2);
            detail::requantize_q8(e.type, data.data(), rows, cols, reinterpret_cast<std::uint32_t*>(m.values.data()),
                                  reinterpret_cast<std::uint16_t*>(m.scales.data()));
            return m;
        }
    }
}

Weight upload(Context& context, const HostMatrix& h) {
    Weight w;
    w.rows = h.rows;
    w.cols = h.cols;
    w.quantized = h.quantized;
    if (!h.quantized) {
        w.t = Tensor::from_bytes(context, std::as_bytes(std::span{h.values}), {h.rows, h.cols}, h.dtype);
        return w;
    }
    const std::int64_t per_word = h.type == QuantType::q8_0 ? 4 : 8;
    w.q.rows = h.rows;
    w.q.cols = h.cols;
    w.q.type = h.type;
    w.q.values = Tensor::from_bytes(context, std::as_bytes(std::span{h.values}), {h.rows, h.cols / per_word}, DType::I32);
    if (h.type == QuantType::q4_K) {
        w.q.scales = Tensor::from_bytes(context, std::as_bytes(std::span{h.scales}), {h.rows, h.cols / 256, 4}, DType::I32);
    } else {
        const Shape ss = h.type == QuantType::q4_1 ? Shape{h.rows, h.cols / 32, 2} : Shape{h.rows, h.cols / 32};
        w.q.scales = Tensor::from_bytes(context, std::as_bytes(std::span{h.scales}), ss, DType::F16);
    }
    return w;
}

// Rows of a, then rows of b (same format): one matrix for one launch.
HostMatrix stack_rows(std::vector<HostMatrix> parts) {
    HostMatrix out = std::move(parts[0]);
    for (std::size_t i = 1; i < parts.size(); ++i) {
        out.values.insert(out.values.end(), parts[i].values.begin(), parts[i].values.end());
        out.scales.insert(out.scales.end(), parts[i].scales.begin(), parts[i].scales.end());
        out.rows += parts[i].rows;
    }
    return out;
}

bool same_format(const HostMatrix& a, const HostMatrix& b) {
    return a.quantized == b.quantized && a.cols == b.cols && (a.quantized ? a.type == b.type : a.dtype == b.dtype);
}

std::vector<float> read_vector(const Gguf& file, const std::string& name, std::int64_t size) {
    const Gguf::Entry& e = file.entry(name);
    if (e.shape != Shape{size}) {
        throw Error("Llama: weight " + name + " is " + to_string(e.shape) + ", but the config needs " + to_string(Shape{size}));
    }
    const std::span<const std::uint8_t> data = file.bytes(name);
    std::vector<float> out(static_cast<std::size_t>(size));
    for (std::size_t i = 0; i < out.size(); ++i) {
        if (e.type == detail::kGgmlF32) {
            std::memcpy(&out[i], &data[4 * i], 4);
        } else if (e.type == detail::kGgmlF16 || e.type == detail::kGgmlBF16) {
            std::uint16_t h;
            std::memcpy(&h, &data[2 * i], 2);
            if (e.type == detail::kGgmlF16) {
                out[i] = detail::f16_to_float(h);
            } else {
                const std::uint32_t bits = std::uint32_t(h) << 16;
                std::memcpy(&out[i], &bits, 4);
            }
        } else {
            throw Error("Llama: vector " + name + " is " + file.type_name(name) + ", not a float type");
        }
    }
    return out;
}

const LlamaConfig& validated(const LlamaConfig& c, std::int64_t context_length) {
    const bool positive = c.vocab_size > 0 && c.hidden_size > 0 && c.intermediate_size > 0 && c.num_layers > 0 && c.num_heads > 0 &&
                          c.num_kv_heads > 0 && c.head_dim > 0 && c.max_positions > 0;
    if (!positive || c.num_heads % c.num_kv_heads != 0 || c.head_dim % 2 != 0) {
        throw Error("Llama: config needs positive sizes, num_heads a multiple of num_kv_heads, and an even head_dim");
    }
    if (context_length < 1 || context_length > c.max_positions) {
        throw Error("Llama: context length " + std::to_string(context_length) + " must be between 1 and max_position_embeddings (" +
                    std::to_string(c.max_positions) + ")");
    }
    if (c.head_dim != 64 && c.head_dim != 128 && c.head_dim != 256) {
        throw Error("Llama: head_dim " + std::to_string(c.head_dim) + " is not implemented (64, 128 and 256 are)");
    }
    if (c.sliding_window && (*c.sliding_window < 1 || !c.sliding_layers.empty())) {
        throw Error("Llama: a sliding window must be positive and cover every layer in this build");
    }
    if (c.qkv_bias || c.o_bias || c.qk_norm || c.sandwich_norms || !c.pre_norms || c.embedding_scale != 1.0f ||
        c.residual_scale != 1.0f || c.logit_divisor != 1.0f || c.attn_logit_softcap < 0.0f || c.final_logit_softcap < 0.0f ||
        c.activation != Activation::silu || c.rotary_dim != 0 || c.norm_weight_offset != 0.0f || !c.rope_layers.empty() ||
        c.query_pre_attn_scalar) {
        throw Error("Llama: this config uses features of another model family, which this build does not implement");
    }
    return c;
}

}  // namespace

// config.cpp:14-140, for the architectures this build runs.
LlamaConfig LlamaConfig::from_gguf(const std::filesystem::path& path) {
    const Gguf file{path};
    const std::string where = "Llama: " + path.string();
    const std::string arch = file.string("general.architecture", "?");
    if (arch != "llama") {
        throw Error(where + " is a " + arch + " model, which vkml does not implement in this build (llama is)");
    }
    const auto key = [&](const std::string& k) { return arch + "." + k; };
    const auto need = [&](const std::string& k) -> std::int64_t {
        if (!file.has(key(k))) throw Error(where + " has no " + key(k));
        return static_cast<std::int64_t>(file.number(key(k), 0));
    };
    LlamaConfig c;
    const std::string scaling = file.string(key("rope.scaling.type"), "none");
    if (scaling == "linear") {
        c.rope_linear_factor = static_cast<float>(file.number(key("rope.scaling.factor"), 1.0));
    } else if (scaling != "none") {
        throw Error(where + " scales rope (" + scaling + "), which vkml does not implement for GGUF files (linear it does)");
    }
    c.hidden_size = need("embedding_length");
    c.intermediate_size = need("feed_forward_length");
    c.num_layers = need("block_count");
    c.num_heads = need("attention.head_count");
    c.num_kv_heads = static_cast<std::int64_t>(file.number(key("attention.head_count_kv"), double(c.num_heads)));
    c.head_dim = static_cast<std::int64_t>(file.number(key("attention.key_length"), c.num_heads > 0 ? double(c.hidden_size / c.num_heads) : 0.0));
    c.max_positions = need("context_length");
    c.rms_norm_eps = static_cast<float>(file.number(key("attention.layer_norm_rms_epsilon"), c.rms_norm_eps));
    c.rope_theta = static_cast<float>(file.number(key("rope.freq_base"), c.rope_theta));
    // A llama file's attention.sliding_window and soft-capping keys are
    // ignored, as the reference ignores them (it reads them for Gemma only,
    // config.cpp:114-133): LlamaOptions sets a window or soft caps.
    if (!file.contains("token_embd.weight")) throw Error(where + " has no token_embd.weight");
    c.vocab_size = file.shape("token_embd.weight").at(0);
    c.tie_word_embeddings = !file.contains("output.weight");
    c.rope_style = RopeStyle::Interleaved;  // llama.cpp's converter reorders q and k rows for it
    c.qkv_bias = file.contains("blk.0.attn_q.bias");
    c.qk_norm = file.contains("blk.0.attn_q_norm.weight");
    if (file.contains("rope_freqs.weight")) {
        const Gguf::Entry& e = file.entry("rope_freqs.weight");
        c.rope_freq_factors = read_vector(file, "rope_freqs.weight", e.shape.empty() ? 0 : e.shape[0]);
    }
    if (file.has("tokenizer.ggml.eos_token_id")) c.eos_token_ids = {static_cast<std::int32_t>(file.number("tokenizer.ggml.eos_token_id", 0))};
    return c;
}

struct Llama::Impl {
    Context* context = nullptr;
    LlamaConfig config;
    std::int64_t context_length = 0;
    LlamaOptions options;
    std::int64_t position = 0;
    bool int_dot = true;

    struct Layer {
        Tensor attn_norm, ffn_norm;
        std::vector<std::pair<Weight, std::int64_t>> qkv;  // fused q|k|v, or parts at row offsets
        Weight o, gate, up, down;
        Tensor k_cache, v_cache;
        // A sliding layer's caches are rings of `rows` rows (position p at
        // row p % rows); else rows = context_length.
        bool slides = false;
        std::int64_t rows = 0;
        // The keys a query sees: the window (at most the ring), or 0 for all.
        std::int64_t window = 0;
        // Decode attention's 128-key chunks: over the window, or the cache.
        std::int64_t chunks() const { return ((slides ? window : rows) + 127) / 128; }
        // The decode step's attention: in one launch with the o GEMV
        // (vkml_attend_step_fused's, or with fast, vkml_attend_step_fast's),
        // as decided at load for every chunk count up to chunks().
        bool one_launch = false, fast = false;
    };
    // With a sliding window: the window (at most the rings' rows), the
    // rings' rows, and the first position they still hold (llama.cpp:
    // 236-241,273-285,361).
    std::int64_t window = 0, ring_rows = 0, oldest_kept = 0;
    Weight embed;
    std::shared_ptr<Weight> lm_head_own;  // when not tied to embed
    bool tied = false;
    Tensor final_norm, rope;
    std::vector<Layer> layers;

    // Decode buffers.
    Tensor x, xn, xq, xs, qkv, q, attn, aq, as, partial, stats, h, hq, hs, gate_tmp, up_tmp, ytmp, logits, state, log;
    Tensor o_sync;      // vkml_attend_step_o: the merge + o launch's sync words
    Tensor fused_sync;  // vkml_attend_step_fused: a block per layer (empty: not used)
    std::int64_t chunks = 1;  // decode attention's 128-key chunks over the whole cache
    // With the one-launch attention on every layer, a step launches the
    // chunks its position needs, in powers of two from kMinTier (each tier
    // its own captured graph); 0: every chunk of the cache.
    static constexpr std::int64_t kMinTier = 8;
    bool tiered = false;
    // Set once a device-side wait gave up: the attention no longer takes
    // launches whose workgroups wait for others (fall_back).
    bool no_waits = false;
    std::int64_t step_tier = 0;
    std::map<std::pair<bool, std::int64_t>, std::uint64_t> graphs;  // (greedy, tier) -> captured step

    const Weight& lm_head() const { return tied ? embed : *lm_head_own; }

    ~Impl() {
        for (const auto& [key, g] : graphs) (void)vkml_graph_destroy(g);
    }

    // The chunk tier of a step at position pos: 128-key chunks covering its
    // pos + 1 keys, rounded up to a power of two (0 when not tiered).
    std::int64_t tier_for(std::int64_t pos) const {
        if (!tiered) return 0;
        const std::int64_t need = (pos + 1 + 127) / 128;
        std::int64_t t = kMinTier;
        while (t < need) t *= 2;
        return t;
    }

    void tag(const char* t) const { (void)vkml_set_profile_tag(t); }

    // The final soft cap of the logits (llama.cpp:405), when the model has one.
    void final_softcap(float* logits_p, std::int64_t count) const {
        if (config.final_logit_softcap <= 0.0f) return;
        tag("softcap");
        check(vkml_unary(2, u32(count), config.final_logit_softcap, logits_p, logits_p), "softcap");
    }

    // Notes that positions up to end have run: a sliding layer's rings keep
    // only the last ring_rows of them.
    void ran_to(std::int64_t end) {
        if (ring_rows) oldest_kept = std::max(oldest_kept, end - ring_rows);
    }

    // y = w . in (+ residual), in given as f32 (xn-like) and, for the int8
    // path, Q8_0 (values, scales).
    void project(const Weight& w, const Tensor& in_f32, const Tensor* in_values, const Tensor* in_scales, float* out, const float* residual,
                 const char* t) const {
        tag(t);
        if (int_dot && w.int_dot_ok() && in_values) {
            const vkml_gemv_dot_params p{1, u32(w.rows), u32(w.cols), w.type_code(), w.scale_code()};
            if (residual) {
                check(vkml_gemv_dot_add(&p, in_values->data(), w.values(), out, w.scales(), static_cast<const float*>(in_scales->data()), residual), t);
            } else {
                check(vkml_gemv_dot(&p, in_values->data(), w.values(), out, w.scales(), static_cast<const float*>(in_scales->data())), t);
            }
            return;
        }
        const vkml_gemv_params p{1, u32(w.rows), u32(w.cols), w.type_code(), w.scale_code(), 0, 1, 1};
        float* y = residual ? static_cast<float*>(ytmp.data()) : out;  // out may be the residual itself
        check(vkml_gemv(&p, static_cast<const float*>(in_f32.data()), w.values(), y, w.scales()), t);
        if (residual) check(vkml_binary(0, u32(w.rows), u32(w.rows), residual, y, out), t);
    }

    bool quantized_input(const Weight& w) const { return int_dot && w.int_dot_ok(); }

    // Whether a device-side wait of the steps since the last check gave up
    // (an o GEMV waiting for its merges: another process holding the GPU's
    // compute units, say). Those steps' KV rows and logits are then invalid.
    // A position past the launched chunks is a fault of the tiers and throws.
    bool waits_failed() const {
        if (!int_dot) return false;
        std::uint32_t flag = 0;
        check(vkml_attend_o_status(static_cast<std::uint32_t*>(const_cast<void*>(o_sync.data())), &flag), "Llama: decode step");
        bool failed = flag != 0;
        if (fused_sync.numel()) {
            std::uint32_t f = 0;
            check(vkml_attend_fused_status(static_cast<std::uint32_t*>(const_cast<void*>(fused_sync.data())), u32(layers.size()), &f),
                  "Llama: decode step");
            if (f == 2) throw Error("Llama: decode step: a position lay past the keys of the launched chunks; the step's results are invalid");
            failed = failed || f != 0;
        }
        return failed;
    }

    // From now on the attention takes the launches that never wait (the
    // chunk pass, the merge and the o GEMV apart, over every chunk of the
    // cache), and the captured steps that waited are dropped.
    void fall_back() {
        no_waits = true;
        tiered = false;
        for (const auto& [key, g] : graphs) (void)vkml_graph_destroy(g);
        graphs.clear();
    }

    // count decode steps from token first at the current position (greedy:
    // each step's argmax feeds the next, on the device). If a device-side
    // wait gave up in them, they run again through the launches that never
    // wait, which the model keeps using: their results replace the invalid
    // ones (the KV rows of those positions and the token log are rewritten).
    void decode_steps(bool greedy, std::int32_t first, std::int64_t count) {
        for (int attempt = 0;; ++attempt) {
            set_state(first, position);
            for (std::int64_t i = 0; i < count; ++i) run_step(greedy, position + i);
            if (!waits_failed()) return;
            if (attempt > 0) throw Error("Llama: decode step: a device-side wait gave up without waiting launches");
            fall_back();
        }
    }

    // One token: the state's token at the state's position.
    void step(bool greedy) {
        const LlamaConfig& c = config;
        const std::int64_t d = c.hidden_size, hd = c.head_dim, ff = c.intermediate_size;
        auto* xp = static_cast<float*>(x.data());
        const auto* st = static_cast<const vkml_decode_state*>(state.data());
        tag("embed");
        const vkml_embedding_params ep{u32(d), u32(d), u32(c.vocab_size), embed.type_code(), embed.quantized ? embed.scale_code() : std::uint32_t(VKML_F16)};
        check(vkml_embedding_state(&ep, embed.values(), embed.scales(), st, xp), "embedding");
        const vkml_rms_norm_params np{1, u32(d), c.rms_norm_eps};
        const bool quant_d = d % 32 == 0;
        const auto norm = [&](const Tensor& w, const char* t) {
            tag(t);
            if (quant_d) {
                check(vkml_rms_norm_quantize(&np, xp, static_cast<const float*>(w.data()), static_cast<float*>(xn.data()), xq.data(),
                                             static_cast<float*>(xs.data())),
                      "rms_norm");
            } else {
                check(vkml_rms_norm(&np, xp, static_cast<const float*>(w.data()), static_cast<float*>(xn.data())), "rms_norm");
            }
        };
        // A norm whose consumers all take the int8 path is folded into their
        // GEMV (rms_norm + Q8_0 in the kernel's prologue, vkml_gemv_fused);
        // not the lm_head's, whose thousands of workgroups would each redo it.
        const bool fold = quant_d && d <= 4096;
        const auto fused = [&](const Weight& w, const Tensor& nw, float* out, const char* t) {
            tag(t);
            const vkml_gemv_fused_params fp{u32(w.rows), u32(w.cols), w.type_code(), w.scale_code(), 0, 1, c.rms_norm_eps, 0};
            check(vkml_gemv_fused(&fp, xp, nullptr, static_cast<const float*>(nw.data()), w.values(), w.scales(), nullptr, nullptr, nullptr,
                                  out, nullptr, nullptr),
                  t);
        };
        auto* fsync = fused_sync.numel() ? static_cast<std::uint32_t*>(fused_sync.data()) : nullptr;
        const auto blocks = u32(layers.size());
        for (std::size_t li = 0; li < layers.size(); ++li) {
            const Layer& L = layers[li];
            const bool fold_qkv =
                fold && std::all_of(L.qkv.begin(), L.qkv.end(), [&](const auto& wr) { return quantized_input(wr.first); });
            // With interleaved RoPE the q|k|v GEMV also rotates q and k and
            // appends the new key and value (vkml_gemv_rope): the attention
            // then starts from q and the caches as they are.
            const bool prepared = fold_qkv && c.rope_style == RopeStyle::Interleaved;
            const uint32_t kv_code = detail::type_code(L.k_cache.dtype());
            if (prepared) {
                for (const auto& [w, row] : L.qkv) {
                    tag("qkv");
                    const vkml_gemv_rope_params rp{u32(w.rows), u32(w.cols), w.type_code(), w.scale_code(), c.rms_norm_eps, u32(row),
                                                   u32(c.num_heads), u32(c.num_kv_heads), u32(hd), u32(L.rows), kv_code, 1};
                    check(vkml_gemv_rope(&rp, xp, static_cast<const float*>(L.attn_norm.data()), w.values(), w.scales(),
                                         static_cast<float*>(qkv.data()), static_cast<const float*>(rope.data()), st, L.k_cache.data(),
                                         L.v_cache.data()),
                          "qkv");
                }
            } else if (fold_qkv) {
                for (const auto& [w, row] : L.qkv) fused(w, L.attn_norm, static_cast<float*>(qkv.data()) + row, "qkv");
            } else {
                norm(L.attn_norm, "attn_norm");
                for (const auto& [w, row] : L.qkv)
                    project(w, xn, quant_d ? &xq : nullptr, &xs, static_cast<float*>(qkv.data()) + row, nullptr, "qkv");
            }
            const bool o_q = quantized_input(L.o);
            // rope, append and attention in one launch, then the merge
            tag("attention");
            const bool merge_o = int_dot && o_q && L.o.int_dot_ok() && !no_waits;
            const std::int64_t launched = merge_o && fsync && step_tier ? std::min(L.chunks(), step_tier) : L.chunks();
            // A tier above the smallest serves positions whose keys fill at
            // least half its chunks: those chunks' items may load before
            // reading the position.
            const std::int64_t ready = step_tier > kMinTier ? std::min(step_tier / 2, launched) : 0;
            const vkml_attend_step_params sp{u32(c.num_heads), u32(c.num_kv_heads), u32(hd), u32(L.rows), 0, 0, kv_code, u32(launched),
                                             c.rope_style == RopeStyle::Interleaved ? 0u : 1u, 1,
                                             1.0f / std::sqrt(static_cast<float>(hd)), c.attn_logit_softcap, u32(L.window),
                                             prepared ? 1u : 0u, u32(ready)};
            if (merge_o && fsync && L.fast) {
                // ... on the matrix cores (the fast_attention option)
                const vkml_gemv_dot_params op{1, u32(L.o.rows), u32(L.o.cols), L.o.type_code(), L.o.scale_code()};
                check(vkml_attend_step_fast(&sp, static_cast<const float*>(qkv.data()), L.k_cache.data(), L.v_cache.data(),
                                            static_cast<float*>(partial.data()), static_cast<float*>(stats.data()),
                                            static_cast<float*>(attn.data()), aq.data(), static_cast<float*>(as.data()), st, &op,
                                            L.o.values(), L.o.scales(), xp, fsync, u32(li), blocks),
                      "attention");
            } else if (merge_o && fsync) {
                // ... and the merge and the o projection + residual too (block
                // li of the fused sync words, whose next block it zeroes)
                const vkml_gemv_dot_params op{1, u32(L.o.rows), u32(L.o.cols), L.o.type_code(), L.o.scale_code()};
                check(vkml_attend_step_fused(&sp, static_cast<const float*>(qkv.data()), static_cast<const float*>(rope.data()),
                                             L.k_cache.data(), L.v_cache.data(), static_cast<float*>(partial.data()),
                                             static_cast<float*>(stats.data()), static_cast<float*>(attn.data()), aq.data(),
                                             static_cast<float*>(as.data()), st, &op, L.o.values(), L.o.scales(), xp, fsync, u32(li), blocks),
                      "attention");
            } else if (merge_o) {
                // ... and the merge shares a launch with the o projection + residual
                const vkml_gemv_dot_params op{1, u32(L.o.rows), u32(L.o.cols), L.o.type_code(), L.o.scale_code()};
                check(vkml_attend_step_o(&sp, static_cast<const float*>(qkv.data()), static_cast<const float*>(rope.data()),
                                         L.k_cache.data(), L.v_cache.data(), static_cast<float*>(partial.data()),
                                         static_cast<float*>(stats.data()), static_cast<float*>(attn.data()), aq.data(),
                                         static_cast<float*>(as.data()), st, &op, L.o.values(), L.o.scales(), xp,
                                         static_cast<std::uint32_t*>(o_sync.data())),
                      "attention");
            } else {
                check(vkml_attend_step(&sp, static_cast<const float*>(qkv.data()), static_cast<const float*>(rope.data()), L.k_cache.data(),
                                       L.v_cache.data(), static_cast<float*>(partial.data()), static_cast<float*>(stats.data()),
                                       static_cast<float*>(attn.data()), o_q ? aq.data() : nullptr,
                                       o_q ? static_cast<float*>(as.data()) : nullptr, st),
                      "attention");
                project(L.o, attn, o_q ? &aq : nullptr, &as, xp, xp, "o");
            }
            auto* hp = static_cast<float*>(h.data());
            const bool down_q = quantized_input(L.down) && ff % 32 == 0;
            bool h_quantized = false;
            if (quantized_input(L.gate) && quantized_input(L.up) && L.gate.staged_ok() && L.up.staged_ok() &&
                L.gate.type_code() == L.up.type_code() && quant_d) {
                // gate|up GEMV + SwiGLU (+ the ffn norm before, + Q8_0 of h after)
                if (!fold) norm(L.ffn_norm, "ffn_norm");
                tag("gate_up");
                const vkml_gemv_fused_params fp{u32(ff), u32(d), L.gate.type_code(), L.gate.scale_code(), 2, fold ? 1u : 0u,
                                                c.rms_norm_eps, down_q ? 1u : 0u};
                check(vkml_gemv_fused(&fp, fold ? static_cast<const void*>(xp) : xq.data(), fold ? nullptr : static_cast<const float*>(xs.data()),
                                      static_cast<const float*>(L.ffn_norm.data()), L.gate.values(), L.gate.scales(), L.up.values(),
                                      L.up.scales(), nullptr, hp, down_q ? hq.data() : nullptr, down_q ? static_cast<float*>(hs.data()) : nullptr),
                      "gate_up");
                h_quantized = down_q;
            } else {
                norm(L.ffn_norm, "ffn_norm");
                project(L.gate, xn, quant_d ? &xq : nullptr, &xs, static_cast<float*>(gate_tmp.data()), nullptr, "gate");
                project(L.up, xn, quant_d ? &xq : nullptr, &xs, static_cast<float*>(up_tmp.data()), nullptr, "up");
                tag("swiglu");
                check(vkml_unary(0, u32(ff), 0.0f, static_cast<const float*>(gate_tmp.data()), static_cast<float*>(gate_tmp.data())), "silu");
                check(vkml_binary(2, u32(ff), u32(ff), static_cast<const float*>(gate_tmp.data()), static_cast<const float*>(up_tmp.data()), hp),
                      "mul");
            }
            if (down_q && !h_quantized) {
                tag("down_quantize");
                const vkml_quantize_params qp{u32(ff / 32), VKML_F32, VKML_Q8_0, VKML_F32};
                check(vkml_quantize(&qp, hp, hq.data(), hs.data()), "quantize");
            }
            project(L.down, h, down_q ? &hq : nullptr, &hs, xp, xp, "down");
        }
        norm(final_norm, "final_norm");
        project(lm_head(), xn, quant_d ? &xq : nullptr, &xs, static_cast<float*>(logits.data()), nullptr, "lm_head");
        final_softcap(static_cast<float*>(logits.data()), c.vocab_size);
        tag("finish");
        check(vkml_step_finish(u32(c.vocab_size), greedy ? static_cast<const float*>(logits.data()) : nullptr,
                               static_cast<vkml_decode_state*>(state.data()), static_cast<std::int32_t*>(log.data()), u32(context_length)),
              "step");
        tag("");
    }

    // The Q8_0 form of a shared input (detail::SharedInput, matmul.cpp:
    // 225-229): made once, for every projection of that input.
    struct Rows {
        Tensor f;         // f32 [t, k]
        Tensor values;    // Q8_0 codes, t * k bytes
        Tensor scales;    // f32, one per 32 values
        bool quantized = false;
    };

    Rows rows_of(const Tensor& f, std::int64_t t, std::int64_t k, bool quantize) const {
        Rows r{f, {}, {}, false};
        if (!quantize) return r;
        r.values = Tensor::empty(*context, {t * k / 4}, DType::I32);
        r.scales = Tensor::empty(*context, {t * k / 32}, DType::F32);
        const vkml_quantize_params qp{u32(t * k / 32), VKML_F32, VKML_Q8_0, VKML_F32};
        check(vkml_quantize(&qp, f.data(), r.values.data(), r.scales.data()), "quantize");
        r.quantized = true;
        return r;
    }

    // The rows of x normalized (and their Q8_0 form when a consumer takes it).
    Rows norm_rows(const Tensor& x, const Tensor& w, std::int64_t t, bool quantize) const {
        const std::int64_t d = config.hidden_size;
        const vkml_rms_norm_params np{u32(t), u32(d), config.rms_norm_eps};
        Rows r{Tensor::empty(*context, {t, d}, DType::F32), {}, {}, false};
        if (quantize && d % 32 == 0) {
            r.values = Tensor::empty(*context, {t * d / 4}, DType::I32);
            r.scales = Tensor::empty(*context, {t * d / 32}, DType::F32);
            check(vkml_rms_norm_quantize(&np, static_cast<const float*>(x.data()), static_cast<const float*>(w.data()),
                                         static_cast<float*>(r.f.data()), r.values.data(), static_cast<float*>(r.scales.data())),
                  "rms_norm");
            r.quantized = true;
        } else {
            check(vkml_rms_norm(&np, static_cast<const float*>(x.data()), static_cast<const float*>(w.data()), static_cast<float*>(r.f.data())),
                  "rms_norm");
        }
        return r;
    }

    // out [t, w.rows] = in . w^T (SharedInput::times_transposed, matmul.cpp:
    // 207-272): the int8 product (gemv_dot for up to 8 rows, matmul_dot on
    // the matrix cores beyond) when in has its Q8_0 form and w takes it,
    // else f32 rows against the widened weights (gemv, or matmul.comp).
    void project_rows(const Weight& w, const Rows& in, std::int64_t t, float* out, const char* what) const {
        tag(what);
        if (in.quantized && quantized_input(w)) {
            const vkml_gemv_dot_params p{u32(t), u32(w.rows), u32(w.cols), w.type_code(), w.scale_code()};
            const auto* as = static_cast<const float*>(in.scales.data());
            if (t <= 8) check(vkml_gemv_dot(&p, in.values.data(), w.values(), out, w.scales(), as), what);
            else check(vkml_matmul_dot(&p, in.values.data(), w.values(), out, w.scales(), as), what);
            return;
        }
        const auto* a = static_cast<const float*>(in.f.data());
        if (t <= 8) {
            const vkml_gemv_params p{u32(t), u32(w.rows), u32(w.cols), w.type_code(), w.scale_code(), 0, 1, 1};
            check(vkml_gemv(&p, a, w.values(), out, w.scales()), what);
        } else {
            const vkml_matmul_params p{u32(t), u32(w.rows), u32(w.cols), 0, 1, 1, 1, w.type_code(), w.scale_code(), 0, 0};
            check(vkml_matmul(&p, a, w.values(), out, w.scales()), what);
        }
    }

    // x [t, w.rows] += in . w^T, the o and down projections with the
    // residual add after them (llama.cpp:374,386): the add in matmul_dot's
    // store on the matrix-core path, else the product into tmp and a binary
    // add (the same f32 sum either way).
    void project_add(const Weight& w, const Rows& in, std::int64_t t, float* x, float* tmp, const char* what) const {
        if (t > 8 && in.quantized && quantized_input(w)) {
            tag(what);
            const vkml_gemv_dot_params p{u32(t), u32(w.rows), u32(w.cols), w.type_code(), w.scale_code()};
            check(vkml_matmul_dot_add(&p, in.values.data(), w.values(), x, w.scales(), static_cast<const float*>(in.scales.data()), x),
                  what);
            return;
        }
        project_rows(w, in, t, tmp, what);
        check(vkml_binary(0, u32(t * w.rows), u32(t * w.rows), x, tmp, x), "add");
    }

    bool any_quantized(const std::vector<std::pair<Weight, std::int64_t>>& ws) const {
        return std::any_of(ws.begin(), ws.end(), [&](const auto& wr) { return quantized_input(wr.first); });
    }

    // t > 1 tokens at once, as the reference's Llama::run (llama.cpp:
    // 299-406): every projection over all t rows, rope + the KV append for
    // all of them in one launch, attention as scores + causal softmax +
    // probs v in the reference's query chunks. The last row's logits go to
    // `logits`, or with all every row's to *all [t, vocab].
    void prefill(std::span<const std::int32_t> tokens, Tensor* all) {
        ran_to(position + static_cast<std::int64_t>(tokens.size()));
        const LlamaConfig& c = config;
        Context& ctx = *context;
        const auto t = static_cast<std::int64_t>(tokens.size());
        const std::int64_t d = c.hidden_size, hd = c.head_dim, ff = c.intermediate_size;
        const std::int64_t heads = c.num_heads, qd = heads * hd, kvd = c.num_kv_heads * hd, width = qd + 2 * kvd;
        const std::int64_t end = position + t;
        const auto f32 = [&](Shape shape) { return Tensor::empty(ctx, std::move(shape), DType::F32); };
        const Tensor ids = Tensor::from_data<std::int32_t>(ctx, tokens, {t});
        Tensor x = f32({t, d});
        tag("embed");
        const vkml_embedding_params ep{u32(t * d), u32(d), u32(c.vocab_size), embed.type_code(),
                                       embed.quantized ? embed.scale_code() : std::uint32_t(VKML_F16)};
        check(vkml_embedding(&ep, embed.values(), embed.scales(), static_cast<const std::int32_t*>(ids.data()), static_cast<float*>(x.data())),
              "embedding");
        auto* xp = static_cast<float*>(x.data());
        Tensor qkv_rows = f32({t, width}), y = f32({t, d}), gate = f32({t, ff}), up = f32({t, ff});
        auto* yp = static_cast<float*>(y.data());
        for (const Layer& L : layers) {
            tag("attn_norm");
            const Rows h = norm_rows(x, L.attn_norm, t, int_dot && any_quantized(L.qkv));
            auto* qkv_p = static_cast<float*>(qkv_rows.data());
            if (L.qkv.size() == 1) {
                project_rows(L.qkv[0].first, h, t, qkv_p, "qkv");
            } else {
                for (const auto& [w, at] : L.qkv) {
                    Tensor part = f32({t, w.rows});
                    project_rows(w, h, t, static_cast<float*>(part.data()), "qkv");
                    const vkml_copy_rows_params cp{u32(t * w.rows), u32(w.rows), u32(w.rows), 0, u32(width), u32(at)};
                    check(vkml_copy_rows(&cp, part.data(), qkv_p), "qkv");
                }
            }
            // heads_first + rope of q and k, k and v to the caches' type at
            // rows position.. (llama.cpp:320-355)
            const auto rope_kv = [&](std::int64_t t0, std::int64_t rows, Tensor& q_rows) {
                tag("rope_kv");
                const vkml_rope_kv_params rp{u32(heads), u32(c.num_kv_heads), u32(hd), u32(L.rows), u32(position + t0),
                                             c.rope_style == RopeStyle::Interleaved ? 0u : 1u, detail::type_code(L.k_cache.dtype()), 1};
                check(vkml_rope_kv_prompt(&rp, u32(rows), u32(width), qkv_p + t0 * width, static_cast<const float*>(rope.data()),
                                          static_cast<float*>(q_rows.data()), const_cast<void*>(L.k_cache.data()),
                                          const_cast<void*>(L.v_cache.data())),
                      "rope_kv");
                tag("attention");
            };
            Tensor attn, merged;
            // With fast_attention, the prompt's attention on the matrix cores
            // (vkml_attend_prompt_fast), written in the o projection's rows.
            const vkml_attend_prompt_params pp{u32(heads), u32(c.num_kv_heads), u32(hd), u32(L.rows), u32(t), u32(position),
                                               detail::type_code(L.k_cache.dtype()), 1.0f / std::sqrt(static_cast<float>(hd)),
                                               c.attn_logit_softcap};
            if (!L.slides && options.fast_attention && vkml_attend_prompt_fast_supported(&pp) == 1) {
                Tensor q = f32({heads, t, hd});
                rope_kv(0, t, q);
                merged = f32({t, qd});
                check(vkml_attend_prompt_fast(&pp, static_cast<const float*>(q.data()), L.k_cache.data(), L.v_cache.data(),
                                              static_cast<float*>(merged.data())),
                      "attention");
            } else if (!L.slides) {
                Tensor q = f32({heads, t, hd});
                rope_kv(0, t, q);
                attn = detail::attention_prompt(q, L.k_cache, L.v_cache, end, true, 0, c.attn_logit_softcap, detail::kMaxScoreBytes,
                                                options.prompt_score_bytes);
            } else {
                // detail::sliding_attention (llama.cpp:356-364): each piece's
                // keys join the rings just before its queries see them
                attn = f32({heads, t, hd});
                for (std::int64_t q0 = 0; q0 < t;) {
                    const std::int64_t rows = detail::sliding_rows(heads, t, q0, position, L.rows, L.window, detail::kMaxScoreBytes);
                    Tensor q = f32({heads, rows, hd});
                    rope_kv(q0, rows, q);
                    detail::copy_rows(detail::ring_attention(q, L.k_cache, L.v_cache, position + q0, L.window, c.attn_logit_softcap), 0,
                                      attn, q0, rows);
                    q0 += rows;
                }
            }
            if (!merged.numel()) merged = permute(attn, {1, 0, 2}).reshape({t, qd});
            const Rows m_in = rows_of(merged, t, qd, int_dot && quantized_input(L.o) && qd % 32 == 0);
            project_add(L.o, m_in, t, xp, yp, "o");
            tag("ffn_norm");
            const Rows h2 = norm_rows(x, L.ffn_norm, t, int_dot && (quantized_input(L.gate) || quantized_input(L.up)));
            auto* gp = static_cast<float*>(gate.data());
            auto* up_p = static_cast<float*>(up.data());
            project_rows(L.gate, h2, t, gp, "gate");
            project_rows(L.up, h2, t, up_p, "up");
            tag("swiglu");
            Rows g_in;
            if (int_dot && quantized_input(L.down) && ff % 32 == 0) {
                // silu, mul and the down projection's Q8_0 input in one pass
                g_in.values = Tensor::empty(ctx, {t * ff / 4}, DType::I32);
                g_in.scales = Tensor::empty(ctx, {t * ff / 32}, DType::F32);
                g_in.quantized = true;
                check(vkml_swiglu_quantize(u32(t * ff), gp, up_p, g_in.values.data(), static_cast<float*>(g_in.scales.data())),
                      "swiglu");
            } else {
                check(vkml_unary(0, u32(t * ff), 0.0f, gp, gp), "silu");
                check(vkml_binary(2, u32(t * ff), u32(t * ff), gp, up_p, gp), "mul");
                g_in = rows_of(gate, t, ff, false);
            }
            project_add(L.down, g_in, t, xp, yp, "down");
        }
        position = end;
        // The final norm; every row through the output projection, or the
        // last row alone (llama.cpp:392-405).
        tag("final_norm");
        const bool q_head = int_dot && quantized_input(lm_head());
        if (all) {
            const Rows hn = norm_rows(x, final_norm, t, q_head);
            project_rows(lm_head(), hn, t, static_cast<float*>(all->data()), "lm_head");
            final_softcap(static_cast<float*>(all->data()), t * c.vocab_size);
        } else {
            Tensor row = f32({1, d});
            check(vkml_memcpy_d2d(row.data(), xp + (t - 1) * d, static_cast<std::uint64_t>(d) * 4), "final_norm");
            const Rows hn = norm_rows(row, final_norm, 1, q_head);
            project_rows(lm_head(), hn, 1, static_cast<float*>(logits.data()), "lm_head");
            final_softcap(static_cast<float*>(logits.data()), c.vocab_size);
        }
        tag("");
    }

    // The decode step at position pos (the state's position).
    void run_step(bool greedy, std::int64_t pos) {
        step_tier = tier_for(pos);
        const bool use_graphs = options.use_graphs && !vkml_get_profiling();
        if (!use_graphs) {
            step(greedy);
            return;
        }
        std::uint64_t& g = graphs[{greedy, step_tier}];
        if (!g) {
            check(vkml_graph_begin(), "Llama: graph capture");
            try {
                step(greedy);
            } catch (...) {
                std::uint64_t dropped = 0;
                (void)vkml_graph_end(&dropped);
                if (dropped) (void)vkml_graph_destroy(dropped);
                throw;
            }
            check(vkml_graph_end(&g), "Llama: graph capture");
        }
        check(vkml_graph_launch(g), "Llama: graph launch");
    }

    void set_state(std::int32_t token, std::int64_t pos) {
        check(vkml_state_set(static_cast<vkml_decode_state*>(state.data()), token, static_cast<std::int32_t>(pos), 0), "Llama: state");
    }

    void check_room(std::int64_t t) const {
        if (t == 0) throw Error("Llama::forward: no tokens");
        if (position + t > context_length) {
            throw Error("Llama::forward: " + std::to_string(position + t) + " tokens exceed the context length of " +
                        std::to_string(context_length));
        }
    }
};

Llama::Llama(std::unique_ptr<Impl> impl) : impl_(std::move(impl)) {}
Llama::Llama(Llama&&) noexcept = default;
Llama& Llama::operator=(Llama&&) noexcept = default;
Llama::~Llama() = default;

Llama Llama::load(Context& context, const std::filesystem::path& path, std::int64_t context_length, LlamaOptions options) {
    if (!std::filesystem::exists(path)) {
        throw Error("Llama::load: no model at " + path.string() + ": give a .gguf file");
    }
    if (path.extension() != ".gguf") throw Error("Llama::load: " + path.string() + " is not a .gguf file (this build reads GGUF)");
    if (options.prompt_score_bytes <= 0) throw Error("Llama: prompt_score_bytes must be positive");
    if (options.kv_cache != DType::F32 && options.kv_cache != DType::F16) {
        throw Error("Llama: a KV cache of " + std::string(to_string(options.kv_cache)) + " is not implemented (f32 and f16 are)");
    }
    auto impl = std::make_unique<Impl>();
    Impl& m = *impl;
    m.context = &context;
    m.config = LlamaConfig::from_gguf(path);
    if (options.sliding_window < 0 || options.attn_logit_softcap < 0.0f || options.final_logit_softcap < 0.0f) {
        throw Error("Llama: sliding_window and the logit soft caps must not be negative (0: none)");
    }
    if (options.sliding_window > 0) m.config.sliding_window = options.sliding_window;
    m.config.attn_logit_softcap = options.attn_logit_softcap;
    m.config.final_logit_softcap = options.final_logit_softcap;
    validated(m.config, context_length);
    m.context_length = context_length;
    m.options = options;
    m.int_dot = context.runtime().integer_dot() && options.integer_dot_product;
    const LlamaConfig& c = m.config;
    const Gguf file{path};
    const std::int64_t d = c.hidden_size, ff = c.intermediate_size, hd = c.head_dim;
    const std::int64_t qd = c.num_heads * hd, kvd = c.num_kv_heads * hd;

    // A float matrix quantized on request (llama.cpp:24-34); the output
    // projection keeps q8_0 unless q8_0 was asked (llama.cpp:95-99).
    const auto finish = [&](Weight w, bool head) {
        if (!options.quantize || w.quantized || w.cols % 32 != 0) return w;
        QuantType qt = *options.quantize;
        if (head && qt != QuantType::q8_0) qt = QuantType::q8_0;
        Weight out;
        out.rows = w.rows;
        out.cols = w.cols;
        out.quantized = true;
        switch (qt) {
            case QuantType::q4_0: out.q = quantize_q4(w.t); break;
            case QuantType::q4_1: out.q = quantize_q4_1(w.t); break;
            case QuantType::q8_0: out.q = quantize_q8(w.t); break;
            case QuantType::q4_K: throw Error("Llama: quantizing to q4_K on load is not implemented (q8_0, q4_0 and q4_1 are)");
        }
        return out;
    };
    const auto matrix = [&](const std::string& name, std::int64_t rows, std::int64_t cols, bool head = false) {
        return finish(upload(context, host_matrix(file, name, rows, cols)), head);
    };
    const auto vec = [&](const std::string& name) {
        return Tensor::from_data<float>(context, read_vector(file, name, d), {d});
    };

    m.embed = upload(context, host_matrix(file, "token_embd.weight", c.vocab_size, d));
    m.tied = c.tie_word_embeddings && (m.embed.quantized || !options.quantize);
    if (!m.tied) {
        m.lm_head_own = std::make_shared<Weight>(c.tie_word_embeddings ? finish(m.embed, true) : matrix("output.weight", c.vocab_size, d, true));
    }
    m.final_norm = vec("output_norm.weight");
    std::vector<float> divisors = c.rope_freq_factors;
    if (c.rope_linear_factor != 1.0f) {
        if (divisors.empty()) divisors.assign(std::size_t(hd / 2), 1.0f);
        for (float& f : divisors) f *= c.rope_linear_factor;
    }
    m.rope = rope_table(context, context_length, hd, c.rope_theta, c.rope_scaling, divisors);
    if (c.sliding_window) {
        if (options.sliding_extra_rows < 0) throw Error("Llama: sliding_extra_rows must not be negative");
        m.ring_rows = std::min(context_length, *c.sliding_window + options.sliding_extra_rows);
        m.window = std::min(*c.sliding_window, m.ring_rows);
    }
    // Decode attention merges at most 1024 chunks of 128 keys per head.
    if ((c.sliding_window ? m.window : context_length) > 131072) {
        throw Error("Llama: a step attends to at most 131072 keys; a context of " + std::to_string(context_length) +
                    " needs a sliding window of at most that");
    }
    for (std::int64_t l = 0; l < c.num_layers; ++l) {
        const std::string p = "blk." + std::to_string(l) + ".";
        Impl::Layer L;
        L.attn_norm = vec(p + "attn_norm.weight");
        L.ffn_norm = vec(p + "ffn_norm.weight");
        HostMatrix hq = host_matrix(file, p + "attn_q.weight", qd, d);
        HostMatrix hk = host_matrix(file, p + "attn_k.weight", kvd, d);
        HostMatrix hv = host_matrix(file, p + "attn_v.weight", kvd, d);
        if (!options.quantize && same_format(hq, hk) && same_format(hq, hv)) {
            L.qkv.emplace_back(upload(context, stack_rows({std::move(hq), std::move(hk), std::move(hv)})), 0);
        } else {
            L.qkv.emplace_back(finish(upload(context, hq), false), 0);
            L.qkv.emplace_back(finish(upload(context, hk), false), qd);
            L.qkv.emplace_back(finish(upload(context, hv), false), qd + kvd);
        }
        L.o = matrix(p + "attn_output.weight", d, qd);
        L.gate = matrix(p + "ffn_gate.weight", ff, d);
        L.up = matrix(p + "ffn_up.weight", ff, d);
        L.down = matrix(p + "ffn_down.weight", d, ff);
        L.slides = c.sliding_window.has_value();
        L.rows = L.slides ? m.ring_rows : context_length;
        L.window = L.slides ? m.window : 0;
        L.k_cache = Tensor::zeros(context, {c.num_kv_heads, L.rows, hd}, options.kv_cache);
        L.v_cache = Tensor::zeros(context, {c.num_kv_heads, L.rows, hd}, options.kv_cache);
        m.layers.push_back(std::move(L));
    }

    // Decode buffers.
    const auto f32 = [&](std::int64_t n) { return Tensor::zeros(context, {n}, DType::F32); };
    m.x = f32(d);
    m.xn = f32(d);
    m.xq = Tensor::zeros(context, {std::max<std::int64_t>(d / 4, 1)}, DType::I32);
    m.xs = f32(std::max<std::int64_t>(d / 32, 1));
    m.qkv = f32(qd + 2 * kvd);
    m.q = f32(qd);
    m.attn = f32(qd);
    m.aq = Tensor::zeros(context, {qd / 4}, DType::I32);
    m.as = f32(qd / 32);
    m.h = f32(ff);
    m.hq = Tensor::zeros(context, {std::max<std::int64_t>(ff / 4, 1)}, DType::I32);
    m.hs = f32(std::max<std::int64_t>(ff / 32, 1));
    m.gate_tmp = f32(ff);
    m.up_tmp = f32(ff);
    m.ytmp = f32(d);
    m.logits = f32(c.vocab_size);
    m.state = Tensor::zeros(context, {4}, DType::I32);
    m.o_sync = Tensor::zeros(context, {static_cast<std::int64_t>(vkml_attend_o_sync_bytes() / 4)}, DType::I32);
    // Every layer's attention in one launch each (vkml_attend_step_fused)
    // when every layer can take it: layer L uses block L and clears block L + 1.
    if (m.layers.size() >= 2 && std::all_of(m.layers.begin(), m.layers.end(), [&](const auto& L) { return m.quantized_input(L.o); }))
        m.fused_sync = Tensor::zeros(context, {static_cast<std::int64_t>(vkml_attend_fused_sync_bytes(u32(m.layers.size())) / 4)}, DType::I32);
    // Which layers take the one launch: the library's own plan for the
    // shapes (the o format, LDS, occupancy, the merge's sets) at the
    // layer's largest chunk count, the one a step may launch. Launches sized
    // by position need it on every layer (the separate launches need
    // chunks covering the cache).
    if (m.fused_sync.numel()) {
        const bool fold = d % 32 == 0 && d <= 4096;
        for (auto& L : m.layers) {
            const bool prepared = fold && c.rope_style == RopeStyle::Interleaved &&
                                  std::all_of(L.qkv.begin(), L.qkv.end(), [&](const auto& wr) { return m.quantized_input(wr.first); });
            const vkml_attend_step_params sp{u32(c.num_heads), u32(c.num_kv_heads), u32(hd), u32(L.rows), 0, 0,
                                             detail::type_code(L.k_cache.dtype()), u32(L.chunks()), 0, 1,
                                             1.0f / std::sqrt(static_cast<float>(hd)), c.attn_logit_softcap, u32(L.window),
                                             prepared ? 1u : 0u, 0};
            const vkml_gemv_dot_params op{1, u32(L.o.rows), u32(L.o.cols), L.o.type_code(), L.o.scale_code()};
            const bool o_ok = m.int_dot && L.o.int_dot_ok();
            L.fast = o_ok && options.fast_attention && vkml_attend_step_fast_supported(&sp, &op) == 1;
            L.one_launch = L.fast || (o_ok && vkml_attend_step_fused_supported(&sp, &op) == 1);
        }
    }
    m.tiered = m.fused_sync.numel() && std::all_of(m.layers.begin(), m.layers.end(), [](const auto& L) { return L.one_launch; });
    m.log = Tensor::zeros(context, {context_length}, DType::I32);
    m.chunks = (context_length + 127) / 128;
    m.partial = f32(c.num_heads * m.chunks * hd);
    m.stats = f32(c.num_heads * m.chunks * 2);
    context.synchronize();
    return Llama(std::move(impl));
}

const LlamaConfig& Llama::config() const noexcept { return impl_->config; }
std::int64_t Llama::context_length() const noexcept { return impl_->context_length; }
std::int64_t Llama::position() const noexcept { return impl_->position; }

Tensor Llama::forward(std::span<const std::int32_t> tokens) {
    Impl& m = *impl_;
    const auto t = static_cast<std::int64_t>(tokens.size());
    m.check_room(t);
    if (t == 1) {
        // One token: the decode step (fused decode attention, llama.cpp:
        // 366 with attention.cpp:199-203).
        m.decode_steps(false, tokens[0], 1);
        m.ran_to(++m.position);
    } else {
        m.prefill(tokens, nullptr);
    }
    Tensor out = Tensor::empty(*m.context, {m.config.vocab_size}, DType::F32);
    check(vkml_memcpy_d2d(out.data(), m.logits.data(), out.nbytes()), "Llama::forward");
    return out;
}

Tensor Llama::forward_all(std::span<const std::int32_t> tokens) {
    Impl& m = *impl_;
    const auto t = static_cast<std::int64_t>(tokens.size());
    m.check_room(t);
    Tensor out = Tensor::empty(*m.context, {t, m.config.vocab_size}, DType::F32);
    if (t == 1) {
        m.decode_steps(false, tokens[0], 1);
        m.ran_to(++m.position);
        check(vkml_memcpy_d2d(out.data(), m.logits.data(), out.nbytes()), "Llama::forward_all");
    } else {
        m.prefill(tokens, &out);
    }
    return out;
}

std::vector<std::int32_t> Llama::generate_greedy(std::int32_t first, std::int64_t count) {
    Impl& m = *impl_;
    if (count <= 0) return {};
    m.check_room(count);
    m.decode_steps(true, first, count);
    std::vector<std::int32_t> out(static_cast<std::size_t>(count));
    check(vkml_memcpy_d2h(out.data(), m.log.data(), out.size() * 4), "Llama::generate_greedy");
    m.position += count;
    m.ran_to(m.position);
    return out;
}

void Llama::reset() noexcept {
    impl_->position = 0;
    impl_->oldest_kept = 0;
}

std::int64_t Llama::rewind(std::int64_t position) {
    Impl& m = *impl_;
    if (position < 0 || position > m.position) {
        throw Error("Llama::rewind: cannot rewind to position " + std::to_string(position) + " of a sequence at " + std::to_string(m.position));
    }
    // Later cache rows are overwritten when those positions come again; a
    // sliding window's rings must still hold the window of position's
    // query, or the model starts over (llama.cpp:273-285).
    const std::int64_t window = m.window ? m.window : 1;
    if (std::max<std::int64_t>(0, position - window + 1) < m.oldest_kept) position = 0;
    if (position == 0) m.oldest_kept = 0;
    m.position = position;
    return position;
}

std::int64_t Llama::advance(std::int64_t position) {
    Impl& m = *impl_;
    if (position < m.position || position > m.context_length) {
        throw Error("Llama::advance: cannot advance to position " + std::to_string(position) + " from " + std::to_string(m.position) +
                    " in a context of " + std::to_string(m.context_length));
    }
    m.position = position;
    m.ran_to(position);
    return position;
}

std::int64_t Llama::kv_cache_bytes() const noexcept {
    std::int64_t bytes = 0;
    for (const auto& L : impl_->layers) bytes += std::int64_t(L.k_cache.nbytes() + L.v_cache.nbytes());
    return bytes;
}

const Tensor& Llama::k_cache(std::int64_t layer) const { return impl_->layers.at(static_cast<std::size_t>(layer)).k_cache; }
const Tensor& Llama::v_cache(std::int64_t layer) const { return impl_->layers.at(static_cast<std::size_t>(layer)).v_cache; }

}  // namespace vkml
