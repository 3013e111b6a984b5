/*
 * vkml_llama.h -- C entry points over vkml::Llama (libvkml.so), for callers
 * that bind a C ABI (ctypes, cgo, JNI, N-API) rather than C++.
 *
 * Each function stands for a member of the reference's public C++ API
 * (include/vkml/llama.hpp:143-223 and context.hpp:104-134 there), with the
 * same meaning and error behaviour: a non-zero status and a message from
 * vkml_llama_last_error() where the C++ API throws vkml::Error (the
 * messages are the reference's, e.g. "Llama::forward: ... exceed the context
 * length of ..." and "Llama::rewind: cannot rewind to position ...").
 *
 * One process holds one device context (created by the first
 * vkml_llama_load, destroyed by vkml_llama_shutdown after the last model is
 * freed). Not thread-safe: serialize calls, as the reference's server does
 * (apps/server.hpp:257 there).
 */
#ifndef VKML_LLAMA_H
#define VKML_LLAMA_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct vkml_llama vkml_llama;

/* LlamaOptions (llama.hpp:118-139) plus ContextOptions::integer_dot_product
 * (context.hpp:80-97) and this build's decode settings. */
typedef struct vkml_llama_options {
    int32_t kv_cache_f16;       /* 0: f32 KV cache (the reference's default), 1: f16 */
    int32_t quantize;           /* -1 none; 0 q8_0, 1 q4_0, 2 q4_1: float weights on load */
    int32_t integer_dot;        /* 1: int8 activations for quantized weights (default) */
    int32_t use_graphs;         /* 1: replay the decode step as a HIP graph (default) */
    const char* device_name;    /* NULL or "": VKML_DEVICE, then device 0 */
    int64_t prompt_score_bytes; /* scores one piece of a prompt's attention may hold (default 1 GiB); no effect on results */
    int64_t sliding_extra_rows; /* a sliding window's rings hold window + this many rows (default 1024) */
    /* 1: decode attention on the matrix cores (vkml_attend_step_fast in
     * vkml_hip.h), f32 attention within f32 rounding instead of the
     * reference's order of f32 operations; 0 (default): bit-exact. */
    int32_t fast_attention;
    /* A sliding window over every layer and logit soft caps (0: none). The
     * reference reads these only from Gemma files (config.cpp:114-133 there)
     * and ignores them in a llama file, as here; they are set explicitly. */
    int64_t sliding_window;
    float attn_logit_softcap;
    float final_logit_softcap;
} vkml_llama_options;

/* LlamaConfig (llama.hpp:29-116), the fields of the llama architecture. */
typedef struct vkml_llama_config {
    int64_t vocab_size, hidden_size, intermediate_size, num_layers, num_heads, num_kv_heads, head_dim, max_positions;
    float rms_norm_eps, rope_theta;
    int32_t tie_word_embeddings;
    int32_t rope_interleaved;
} vkml_llama_config;

const char* vkml_llama_last_error(void);
void vkml_llama_default_options(vkml_llama_options* out);

/* Llama::load(Context&, path, context_length, options) (llama.hpp:149-150). */
int vkml_llama_load(const char* gguf_path, int64_t context_length, const vkml_llama_options* options, vkml_llama** out);
void vkml_llama_free(vkml_llama* model);
/* Destroys the process's device context; fails while models are alive. */
int vkml_llama_shutdown(void);

/* LlamaConfig::from_gguf (llama.hpp:115, config.cpp:14-140 there): a GGUF
 * file's model config, read from its header alone (no device needed). */
int vkml_llama_read_config(const char* gguf_path, vkml_llama_config* out);

/* Llama::config, context_length, position, kv_cache_bytes (llama.hpp:155-180). */
int vkml_llama_get_config(const vkml_llama* model, vkml_llama_config* out);
int64_t vkml_llama_context_length(const vkml_llama* model);
int64_t vkml_llama_position(const vkml_llama* model);
int64_t vkml_llama_kv_cache_bytes(const vkml_llama* model);

/* Llama::forward: the last token's logits into logits[vocab_size]. */
int vkml_llama_forward(vkml_llama* model, const int32_t* tokens, int64_t count, float* logits);
/* Llama::forward_all: every token's logits into logits[count * vocab_size]. */
int vkml_llama_forward_all(vkml_llama* model, const int32_t* tokens, int64_t count, float* logits);
/* vkml::argmax(model.forward({&token, 1})) for count steps, on the device:
 * tokens_out[i] is step i's argmax (the decode loop of apps/vkml_run.cpp:
 * 282-298 there), with no host round trip between steps. */
int vkml_llama_generate_greedy(vkml_llama* model, int32_t first, int64_t count, int32_t* tokens_out);
/* Llama::reset and rewind (llama.hpp:171-177). *out gets the position. */
int vkml_llama_reset(vkml_llama* model);
int vkml_llama_rewind(vkml_llama* model, int64_t position, int64_t* out);
/* Llama::advance: moves the sequence forward to position without running
 * the tokens between (their KV rows keep what they hold). No reference
 * counterpart: for benchmarks and tests that time steps at a position. */
int vkml_llama_advance(vkml_llama* model, int64_t position);
/* Layer l's KV caches [kv_heads, context_length, head_dim] copied to the
 * host (element size 2 for an f16 cache, 4 for f32). */
int vkml_llama_read_kv_cache(const vkml_llama* model, int64_t layer, void* k_out, void* v_out, uint64_t bytes);

/* ---- Sampling and serving (include/vkml/sampling.hpp:14-31 and
 * src/io/sampling.cpp:17-139 there; apps/generation.hpp:139-202 there). ---- */

/* SamplingOptions: temperature 0 (or top_k 1) is greedy; top_k 0 keeps all;
 * top_p 1 and min_p 0 are off; penalties 1 (repetition) and 0 are off. */
typedef struct vkml_sampling_options {
    float temperature;
    int32_t top_k;
    float top_p;
    float repetition_penalty;
    float min_p;
    float frequency_penalty;
    float presence_penalty;
    uint64_t seed;
} vkml_sampling_options;
void vkml_sampling_default_options(vkml_sampling_options* out);

/* Sampler: host code, no device needed. sample() is Sampler::sample over
 * logits[vocab] with previous[n_previous] (the tokens so far) for the
 * repetition penalty; each call advances the sampler's generator. */
typedef struct vkml_sampler vkml_sampler;
int vkml_sampler_create(const vkml_sampling_options* options, vkml_sampler** out);
void vkml_sampler_free(vkml_sampler* sampler);
int vkml_sampler_sample(vkml_sampler* sampler, const float* logits, int64_t vocab, const int32_t* previous,
                        int64_t n_previous, int32_t* token_out);

/* A model with the tokens its KV cache holds, for one request after another
 * (ChatModel::generate): each prompt reuses the cache of its longest common
 * prefix with the last; the reply (without the stop token) goes to
 * reply[capacity], its length to *reply_len, and *finish is 0 for a stop
 * token, 1 for max_tokens (negative: none), capacity or the context's end:
 * the reply stops at capacity tokens, so it always fits. The model must
 * outlive the session; one thread at a time. */
typedef struct vkml_session vkml_session;
int vkml_session_create(vkml_llama* model, const int32_t* stop, int64_t n_stop, vkml_session** out);
void vkml_session_free(vkml_session* session);
int vkml_session_generate(vkml_session* session, const int32_t* prompt, int64_t n_prompt, vkml_sampler* sampler,
                          int64_t max_tokens, int32_t* reply, int64_t capacity, int64_t* reply_len, int32_t* finish);
/* vkml_session_generate with each reply token's log probability under the
 * model's logits (before any sampling setting) in logprobs[i] and its top
 * likeliest tokens and theirs in top_ids / top_logprobs[i * top + j]
 * (ChatModel::generate with logprobs, apps/generation.hpp:139-142,176-190
 * there; -1 / NaN past a row's alternatives). Any of the three may be NULL;
 * every step's logits are read back when one is not. */
int vkml_session_generate_logprobs(vkml_session* session, const int32_t* prompt, int64_t n_prompt, vkml_sampler* sampler,
                                   int64_t max_tokens, int32_t top, int32_t* reply, int64_t capacity, int64_t* reply_len,
                                   int32_t* finish, float* logprobs, int32_t* top_ids, float* top_logprobs);
/* ChatModel::score (apps/generation.hpp:104-131 there): each prompt token's
 * log probability given the ones before (logprobs[0] is NaN) and the top
 * alternatives at its position (top_ids / top_logprobs [n_prompt * top]),
 * from forward_all; the model starts over and ends holding the prompt. */
int vkml_session_score(vkml_session* session, const int32_t* prompt, int64_t n_prompt, int32_t top, float* logprobs,
                       int32_t* top_ids, float* top_logprobs);
/* token_logprobs (include/vkml/sampling.hpp there): token's log-softmax
 * probability under logits[vocab] and the top likeliest tokens with theirs.
 * Host code, no device needed. */
int vkml_token_logprobs(const float* logits, int64_t vocab, int32_t token, int32_t top, float* logprob, int32_t* top_ids,
                        float* top_logprobs);

/* The tokens the cache holds: writes up to capacity, returns how many. */
int64_t vkml_session_cached(const vkml_session* session, int32_t* out, int64_t capacity);

/* Context::set_profiling / profile / reset_profile (context.hpp:120-126):
 * up to capacity labels, slowest first; *count gets how many exist. */
int vkml_llama_set_profiling(int32_t enabled);
int vkml_llama_profile(char* names, uint32_t name_stride, uint64_t* calls, double* milliseconds, uint32_t capacity, uint32_t* count);
int vkml_llama_reset_profile(void);
/* Context::synchronize: waits for queued work. */
int vkml_llama_synchronize(void);

#ifdef __cplusplus
}
#endif
#endif
