// capi.cpp -- the C entry points of include/vkml_llama.h over vkml::Llama.
#include <cstring>
#include <limits>
#include <memory>
#include <string>

#include "runtime.hpp"
#include "vkml/generation.hpp"
#include "vkml/llama.hpp"
#include "vkml/sampling.hpp"
#include "vkml_llama.h"

struct vkml_llama {
    vkml::Llama model;
};

struct vkml_sampler {
    vkml::Sampler sampler;
};

struct vkml_session {
    vkml::Session session;
};

namespace {

thread_local std::string g_error;
std::unique_ptr<vkml::Context> g_context;
int g_models = 0;

template <class F>
int guarded(F&& f) {
    try {
        f();
        return 0;
    } catch (const std::exception& e) {
        g_error = e.what();
        return 1;
    }
}

vkml::Context& context(const vkml_llama_options& o) {
    if (!g_context) {
        vkml::ContextOptions co;
        co.device_name = o.device_name ? o.device_name : "";
        g_context = std::make_unique<vkml::Context>(co);
    }
    return *g_context;
}

vkml_llama_config c_config(const vkml::LlamaConfig& c) {
    return vkml_llama_config{c.vocab_size, c.hidden_size, c.intermediate_size, c.num_layers, c.num_heads, c.num_kv_heads, c.head_dim,
                             c.max_positions, c.rms_norm_eps, c.rope_theta, c.tie_word_embeddings ? 1 : 0,
                             c.rope_style == vkml::RopeStyle::Interleaved ? 1 : 0};
}

// Copies rows of TokenLogprobs out: logprob[i], and top_ids / top_logprobs
// [i * top + j] (-1 and NaN past a row's alternatives).
void copy_logprobs(const std::vector<vkml::TokenLogprobs>& rows, int32_t top, float* logprobs, int32_t* top_ids, float* top_logprobs) {
    for (std::size_t i = 0; i < rows.size(); ++i) {
        if (logprobs) logprobs[i] = rows[i].logprob;
        for (int32_t j = 0; j < top; ++j) {
            const bool has = std::size_t(j) < rows[i].top.size();
            if (top_ids) top_ids[i * std::size_t(top) + std::size_t(j)] = has ? rows[i].top[std::size_t(j)].first : -1;
            if (top_logprobs)
                top_logprobs[i * std::size_t(top) + std::size_t(j)] =
                    has ? rows[i].top[std::size_t(j)].second : std::numeric_limits<float>::quiet_NaN();
        }
    }
}

}  // namespace

extern "C" {

const char* vkml_llama_last_error(void) { return g_error.c_str(); }

void vkml_llama_default_options(vkml_llama_options* out) {
    if (!out) return;
    *out = vkml_llama_options{0, -1, 1, 1, nullptr, std::int64_t{1} << 30, 1024, 0, 0, 0.0f, 0.0f};
}

int vkml_llama_load(const char* path, int64_t context_length, const vkml_llama_options* options, vkml_llama** out) {
    return guarded([&] {
        if (!path || !out) throw vkml::Error("vkml_llama_load: null argument");
        vkml_llama_options o;
        vkml_llama_default_options(&o);
        if (options) o = *options;
        vkml::LlamaOptions lo;
        lo.kv_cache = o.kv_cache_f16 ? vkml::DType::F16 : vkml::DType::F32;
        if (o.quantize >= 0) {
            if (o.quantize > 2) throw vkml::Error("vkml_llama_load: quantize must be -1, 0 (q8_0), 1 (q4_0) or 2 (q4_1)");
            lo.quantize = static_cast<vkml::QuantType>(o.quantize);
        }
        lo.use_graphs = o.use_graphs != 0;
        lo.integer_dot_product = o.integer_dot != 0;
        if (o.prompt_score_bytes <= 0) throw vkml::Error("vkml_llama_load: prompt_score_bytes must be positive");
        lo.prompt_score_bytes = o.prompt_score_bytes;
        lo.sliding_extra_rows = o.sliding_extra_rows;
        lo.fast_attention = o.fast_attention != 0;
        lo.sliding_window = o.sliding_window;
        lo.attn_logit_softcap = o.attn_logit_softcap;
        lo.final_logit_softcap = o.final_logit_softcap;
        vkml::Context& ctx = context(o);
        *out = new vkml_llama{vkml::Llama::load(ctx, path, context_length, lo)};
        ++g_models;
    });
}

void vkml_llama_free(vkml_llama* model) {
    if (!model) return;
    delete model;
    --g_models;
}

int vkml_llama_shutdown(void) {
    return guarded([] {
        if (g_models > 0) throw vkml::Error("vkml_llama_shutdown: " + std::to_string(g_models) + " models are still alive");
        g_context.reset();
    });
}

int vkml_llama_read_config(const char* path, vkml_llama_config* out) {
    return guarded([&] {
        if (!path || !out) throw vkml::Error("vkml_llama_read_config: null argument");
        *out = c_config(vkml::LlamaConfig::from_gguf(path));
    });
}

int vkml_llama_get_config(const vkml_llama* m, vkml_llama_config* out) {
    return guarded([&] {
        if (!m || !out) throw vkml::Error("vkml_llama_get_config: null argument");
        *out = c_config(m->model.config());
    });
}

int64_t vkml_llama_context_length(const vkml_llama* m) { return m ? m->model.context_length() : -1; }
int64_t vkml_llama_position(const vkml_llama* m) { return m ? m->model.position() : -1; }
int64_t vkml_llama_kv_cache_bytes(const vkml_llama* m) { return m ? m->model.kv_cache_bytes() : -1; }

int vkml_llama_forward(vkml_llama* m, const int32_t* tokens, int64_t count, float* logits) {
    return guarded([&] {
        if (!m || (!tokens && count) || !logits) throw vkml::Error("vkml_llama_forward: null argument");
        const std::vector<float> v = m->model.forward({tokens, static_cast<std::size_t>(count)}).to_vector<float>();
        std::memcpy(logits, v.data(), v.size() * 4);
    });
}

int vkml_llama_forward_all(vkml_llama* m, const int32_t* tokens, int64_t count, float* logits) {
    return guarded([&] {
        if (!m || (!tokens && count) || !logits) throw vkml::Error("vkml_llama_forward_all: null argument");
        const std::vector<float> v = m->model.forward_all({tokens, static_cast<std::size_t>(count)}).to_vector<float>();
        std::memcpy(logits, v.data(), v.size() * 4);
    });
}

int vkml_llama_generate_greedy(vkml_llama* m, int32_t first, int64_t count, int32_t* tokens_out) {
    return guarded([&] {
        if (!m || (!tokens_out && count > 0)) throw vkml::Error("vkml_llama_generate_greedy: null argument");
        const std::vector<int32_t> t = m->model.generate_greedy(first, count);
        std::memcpy(tokens_out, t.data(), t.size() * 4);
    });
}

int vkml_llama_reset(vkml_llama* m) {
    return guarded([&] {
        if (!m) throw vkml::Error("vkml_llama_reset: null model");
        m->model.reset();
    });
}

int vkml_llama_rewind(vkml_llama* m, int64_t position, int64_t* out) {
    return guarded([&] {
        if (!m) throw vkml::Error("vkml_llama_rewind: null model");
        const int64_t p = m->model.rewind(position);
        if (out) *out = p;
    });
}

int vkml_llama_advance(vkml_llama* m, int64_t position) {
    return guarded([&] {
        if (!m) throw vkml::Error("vkml_llama_advance: null model");
        (void)m->model.advance(position);
    });
}

int vkml_llama_read_kv_cache(const vkml_llama* m, int64_t layer, void* k_out, void* v_out, uint64_t bytes) {
    return guarded([&] {
        if (!m) throw vkml::Error("vkml_llama_read_kv_cache: null model");
        const vkml::Tensor& k = m->model.k_cache(layer);
        const vkml::Tensor& v = m->model.v_cache(layer);
        if (bytes != k.nbytes()) throw vkml::Error("vkml_llama_read_kv_cache: the caches hold " + std::to_string(k.nbytes()) + " bytes each");
        const auto kb = k.to_bytes(), vb = v.to_bytes();
        if (k_out) std::memcpy(k_out, kb.data(), kb.size());
        if (v_out) std::memcpy(v_out, vb.data(), vb.size());
    });
}

void vkml_sampling_default_options(vkml_sampling_options* out) {
    if (!out) return;
    const vkml::SamplingOptions d;
    *out = vkml_sampling_options{d.temperature, d.top_k, d.top_p, d.repetition_penalty, d.min_p, d.frequency_penalty, d.presence_penalty,
                                 d.seed};
}

int vkml_sampler_create(const vkml_sampling_options* o, vkml_sampler** out) {
    return guarded([&] {
        if (!o || !out) throw vkml::Error("vkml_sampler_create: null argument");
        vkml::SamplingOptions s;
        s.temperature = o->temperature;
        s.top_k = o->top_k;
        s.top_p = o->top_p;
        s.repetition_penalty = o->repetition_penalty;
        s.min_p = o->min_p;
        s.frequency_penalty = o->frequency_penalty;
        s.presence_penalty = o->presence_penalty;
        s.seed = o->seed;
        *out = new vkml_sampler{vkml::Sampler(s)};
    });
}

void vkml_sampler_free(vkml_sampler* s) { delete s; }

int vkml_sampler_sample(vkml_sampler* s, const float* logits, int64_t vocab, const int32_t* previous, int64_t n_previous,
                        int32_t* token_out) {
    return guarded([&] {
        if (!s || !logits || vocab < 0 || !token_out || n_previous < 0 || (n_previous && !previous))
            throw vkml::Error("vkml_sampler_sample: null or negative argument");
        *token_out = s->sampler.sample({logits, std::size_t(vocab)}, {previous, std::size_t(n_previous)});
    });
}

int vkml_session_create(vkml_llama* m, const int32_t* stop, int64_t n_stop, vkml_session** out) {
    return guarded([&] {
        if (!m || !out || n_stop < 0 || (n_stop && !stop)) throw vkml::Error("vkml_session_create: null or negative argument");
        *out = new vkml_session{vkml::Session(m->model, std::vector<std::int32_t>(stop, stop + n_stop))};
    });
}

void vkml_session_free(vkml_session* s) { delete s; }


int vkml_session_generate(vkml_session* s, const int32_t* prompt, int64_t n_prompt, vkml_sampler* sampler, int64_t max_tokens,
                          int32_t* reply, int64_t capacity, int64_t* reply_len, int32_t* finish) {
    return vkml_session_generate_logprobs(s, prompt, n_prompt, sampler, max_tokens, 0, reply, capacity, reply_len, finish, nullptr,
                                          nullptr, nullptr);
}

int vkml_session_generate_logprobs(vkml_session* s, const int32_t* prompt, int64_t n_prompt, vkml_sampler* sampler,
                                   int64_t max_tokens, int32_t top, int32_t* reply, int64_t capacity, int64_t* reply_len,
                                   int32_t* finish, float* logprobs, int32_t* top_ids, float* top_logprobs) {
    return guarded([&] {
        if (!s || !prompt || n_prompt <= 0 || !sampler || capacity < 0 || (!reply && capacity) || !reply_len || top < 0)
            throw vkml::Error("vkml_session_generate: null or negative argument, or an empty prompt");
        // The reply never outgrows the caller's buffer: at most capacity tokens.
        const std::int64_t limit = max_tokens < 0 ? capacity : std::min(max_tokens, capacity);
        const bool want = logprobs || top_ids || top_logprobs;
        std::vector<std::int32_t> out;
        std::vector<vkml::TokenLogprobs> lp;
        const auto f = s->session.generate({prompt, std::size_t(n_prompt)}, sampler->sampler, limit, out, want ? &lp : nullptr, top);
        std::copy(out.begin(), out.end(), reply);
        *reply_len = std::int64_t(out.size());
        if (finish) *finish = f == vkml::Session::Finish::stop ? 0 : 1;
        if (want) copy_logprobs(lp, top, logprobs, top_ids, top_logprobs);
    });
}

int vkml_session_score(vkml_session* s, const int32_t* prompt, int64_t n_prompt, int32_t top, float* logprobs, int32_t* top_ids,
                       float* top_logprobs) {
    return guarded([&] {
        if (!s || !prompt || n_prompt <= 0 || top < 0) throw vkml::Error("vkml_session_score: null or negative argument, or an empty prompt");
        copy_logprobs(s->session.score({prompt, std::size_t(n_prompt)}, top), top, logprobs, top_ids, top_logprobs);
    });
}

int vkml_token_logprobs(const float* logits, int64_t vocab, int32_t token, int32_t top, float* logprob, int32_t* top_ids,
                        float* top_logprobs) {
    return guarded([&] {
        if (!logits || vocab <= 0 || top < 0) throw vkml::Error("vkml_token_logprobs: null or empty logits, or a negative top");
        copy_logprobs({vkml::token_logprobs({logits, std::size_t(vocab)}, token, top)}, top, logprob, top_ids, top_logprobs);
    });
}

int64_t vkml_session_cached(const vkml_session* s, int32_t* out, int64_t capacity) {
    if (!s) return -1;
    const auto& c = s->session.cached();
    for (std::int64_t i = 0; out && i < capacity && i < std::int64_t(c.size()); ++i) out[i] = c[std::size_t(i)];
    return std::int64_t(c.size());
}

int vkml_llama_set_profiling(int32_t enabled) {
    return guarded([&] {
        if (!g_context) throw vkml::Error("vkml_llama_set_profiling: no context (load a model first)");
        g_context->set_profiling(enabled != 0);
    });
}

int vkml_llama_profile(char* names, uint32_t stride, uint64_t* calls, double* ms, uint32_t capacity, uint32_t* count) {
    return guarded([&] {
        if (!g_context) throw vkml::Error("vkml_llama_profile: no context (load a model first)");
        const auto rows = g_context->profile();
        if (count) *count = static_cast<uint32_t>(rows.size());
        for (uint32_t i = 0; i < capacity && i < rows.size(); ++i) {
            if (names && stride) {
                std::strncpy(names + std::size_t(i) * stride, rows[i].name.c_str(), stride - 1);
                names[std::size_t(i) * stride + stride - 1] = 0;
            }
            if (calls) calls[i] = rows[i].calls;
            if (ms) ms[i] = rows[i].milliseconds;
        }
    });
}

int vkml_llama_reset_profile(void) {
    return guarded([] {
        if (g_context) g_context->reset_profile();
    });
}

int vkml_llama_synchronize(void) {
    return guarded([] {
        if (g_context) g_context->synchronize();
    });
}

}  // extern "C"
