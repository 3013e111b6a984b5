/*
 * vkml_oracle.h -- CPU restatement of vkml's batch-1 decode arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and
 * never as the thing measured or shipped. The product (libvkml_hip.so,
 * libvkml.so) neither links nor calls it.
 *
 * Every function restates one piece of the reference
 * (danielkwan-dev/vkml-framework, read-only at /root/reference) and cites the
 * file:line it follows. Floating-point expressions keep the reference's
 * operation order and are compiled with -ffp-contract=off, so no multiply-add
 * is fused here that the reference writes as two operations.
 *
 * Pinning (what checks each function against something other than itself) is
 * listed in tests/test_oracle.py; functions no check pins are marked
 * "parity unpinned" below.
 */
#ifndef VKML_ORACLE_H
#define VKML_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Quantized formats, numbered as vkml::QuantType (include/vkml/ops.hpp:119). */
enum { ORC_Q8_0 = 0, ORC_Q4_0 = 1, ORC_Q4_1 = 2 };

/* ggml tensor type numbers (src/io/gguf.cpp:30-40). */
enum {
    ORC_GGML_F32 = 0, ORC_GGML_F16 = 1, ORC_GGML_Q4_0 = 2, ORC_GGML_Q4_1 = 3,
    ORC_GGML_Q8_0 = 8, ORC_GGML_Q4_K = 12, ORC_GGML_Q6_K = 14, ORC_GGML_BF16 = 30
};

/* Weight element types of the float matrix-vector path (shaders/include/halves.glsl:5-24). */
enum { ORC_T_F32 = 0, ORC_T_F16 = 1, ORC_T_BF16 = 2, ORC_T_Q8 = 3, ORC_T_Q4 = 4, ORC_T_Q4_1 = 5 };

const char* orc_last_error(void);
void orc_set_threads(int threads); /* worker threads for model-level work (default 1) */
int orc_get_threads(void);

/* ---- 16-bit floats: src/io/host_quant.cpp:74-114, shaders/include/halves.glsl:61-93 ---- */
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);
float orc_bf16_to_f32(uint16_t h);
void orc_cast_f32_to_f16(const float* x, uint16_t* y, int64_t n);
void orc_cast_f16_to_f32(const uint16_t* x, float* y, int64_t n);

/* ---- ggml block decoders: src/io/gguf.cpp:117-228 ----
 * Returns the number of values written, or -1 for a type not on the path. */
int64_t orc_dequantize_ggml(int ggml_type, const uint8_t* blocks, int64_t nbytes, float* out);
int64_t orc_ggml_row_bytes(int ggml_type, int64_t cols); /* -1 if not whole blocks */

/* ---- load-time repacking into QuantizedMatrix's layout ----
 * orc_load_quantized: q8_0/q4_0/q4_1/q4_K file data (src/io/gguf.cpp:525-638);
 * returns the ORC_Q* type, or -1. words: rows*cols/4 (q8_0) or /8 words;
 * halves: rows*cols/32 f16 scales, or twice that (scale, offset) for q4_1.
 * orc_load_q8: any decodable type requantized to Q8_0 with f16 scales
 * (src/io/gguf.cpp:503-523, src/io/host_quant.cpp:116-159). */
int orc_load_quantized(int ggml_type, const uint8_t* data, int64_t rows, int64_t cols,
                       uint32_t* words, uint16_t* halves);
int orc_load_q8(int ggml_type, const uint8_t* data, int64_t rows, int64_t cols, uint32_t* words,
                uint16_t* halves);

/* ---- quantize.comp / dequantize.comp ----
 * scale_f16 = 1: f16 scales (weights), packed as uint16; 0: f32 scales (activations). */
void orc_quantize(int quant, int scale_f16, const float* x, int64_t rows, int64_t cols,
                  uint32_t* words, void* scales);
void orc_dequantize(int quant, int scale_f16, const uint32_t* words, const void* scales,
                    int64_t rows, int64_t cols, float* out);

/* ---- int8 matrix-vector / matrix products ----
 * a: Q8_0 activations (f32 scales), M rows; b: [N, K] quantized weights.
 * orc_gemv_dot follows shaders/gemv_dot.comp (M <= 8); orc_matmul_dot follows
 * shaders/matmul_dot.comp (M > 8). out: [M, N]. */
void orc_gemv_dot(int quant, int scale_f16, const uint32_t* a_words, const float* a_scales,
                  int64_t M, const uint32_t* b_words, const void* b_scales, int64_t N, int64_t K,
                  float* out);
void orc_matmul_dot(int quant, int scale_f16, const uint32_t* a_words, const float* a_scales,
                    int64_t M, const uint32_t* b_words, const void* b_scales, int64_t N,
                    int64_t K, float* out);

/* ---- float matrix-vector path: shaders/gemv.comp:101-212 ----
 * a f32 [M, K]; b [N, K] of b_type (ORC_T_*); b_scales for quantized b. */
void orc_gemv_float(int b_type, int scale_f16, const float* a, int64_t M, const void* b,
                    const void* b_scales, int64_t N, int64_t K, float* out);
/* ---- float matrix product: shaders/matmul.comp, b transposed [N, K] ----
 * the path for M > 8 rows (matmul.cpp:96); sums in k order. */
void orc_matmul_float(int b_type, int scale_f16, const float* a, int64_t M, const void* b,
                      const void* b_scales, int64_t N, int64_t K, float* out);

/* ---- norms, rope, activations ---- */
void orc_rms_norm(const float* x, const float* w, int64_t rows, int64_t cols, float eps,
                  float* out);                                        /* rms_norm.comp */
void orc_rope_table(int64_t positions, int64_t head_dim, float theta, float* table); /* rope.cpp:32-86 */
void orc_rope(const float* x, const float* table, int64_t rows, int64_t heads, int64_t seq,
              int64_t dim, int64_t half_dim, int64_t start_pos, int style, float* out); /* rope.comp */
float orc_expf(float x);   /* the exp shared with the GPU kernels; exp of unary.comp:22 and attend.comp:129 */
void orc_expf_array(const float* x, float* y, int64_t n);
void orc_silu(const float* x, float* y, int64_t n);                  /* unary.comp:21-24 */
void orc_binary(int op, const float* a, const float* b, int64_t n, int64_t b_count,
                float* out);                                          /* binary.comp */
int32_t orc_argmax(const float* x, int64_t n);                        /* argmax.comp */

/* ---- embeddings ---- */
void orc_embedding_quantized(int quant, const uint32_t* words, const uint16_t* halves,
                             int64_t vocab, int64_t dim, const int32_t* ids, int64_t n,
                             float* out);                             /* embedding_quantized.comp */

/* ---- attention over a KV cache [kv_heads, capacity, hd] (f32, or f16 bits) ----
 * orc_attend_decode: one query per head, attend.comp + attend_merge.comp
 * (chunks of 128 keys, merged). orc_attention_prefill: q [heads, q_len, hd],
 * query i at position kv_len - q_len + i, in the reference's chunks of
 * queries (attention.cpp:205-226), each attention_block's matmul + softmax +
 * matmul (src/ops/attention.cpp:127-138, shaders/softmax.comp). */
void orc_attend_decode(const float* q, int64_t heads, const void* k, const void* v, int kv_f16,
                       int64_t kv_heads, int64_t capacity, int64_t hd, int64_t kv_start,
                       int64_t kv_len, float softcap, float* out);
void orc_attention_prefill(const float* q, int64_t heads, int64_t q_len, const void* k,
                           const void* v, int kv_f16, int64_t kv_heads, int64_t capacity,
                           int64_t hd, int64_t kv_len, int64_t max_score_bytes, float softcap, float* out);
/* detail::sliding_attention (attention.cpp:229-294): queries q [heads, t, hd]
 * at positions start.., their keys and values k, v [kv_heads, t, hd] (in the
 * caches' type) appended chunk by chunk to rings [kv_heads, ring, hd]
 * (position p in row p % ring), each query seeing the last `window`
 * positions up to its own; out [heads, t, hd]. */
void orc_attention_sliding(const float* q, int64_t heads, int64_t t, const void* k, const void* v, void* k_ring,
                           void* v_ring, int f16, int64_t kv_heads, int64_t ring, int64_t hd, int64_t start,
                           int64_t window, int64_t max_score_bytes, float softcap, float* out);
/* The reference's score budget per attention call (ops/internal.hpp:92). */
#define ORC_MAX_SCORE_BYTES ((int64_t)64 << 20)

/* ---- whole model: src/models/llama.cpp:170-406 (GGUF llama architecture) ----
 * int_dot: 1 quantizes activations for quantized weights (gemv_dot /
 * matmul_dot), 0 multiplies them in f32 (gemv.comp). */
typedef struct orc_model orc_model;
orc_model* orc_model_load(const char* gguf_path, int64_t context_length, int kv_f16, int int_dot);
/* The same with LlamaOptions::sliding_extra_rows (llama.hpp:133 there): a
 * sliding window's rings hold window + that many rows (at most the context). */
orc_model* orc_model_load_ex(const char* gguf_path, int64_t context_length, int kv_f16, int int_dot,
                             int64_t sliding_extra_rows);
/* As orc_model_load_ex with a sliding window over every layer and the
 * attention / final logit soft caps given (0: none). */
orc_model* orc_model_load_opts(const char* gguf_path, int64_t context_length, int kv_f16, int int_dot, int64_t sliding_extra_rows,
                               int64_t window, float attn_softcap, float final_softcap);
/* Test instrumentation: decode steps move each attention output by up to
 * ulps units in the last place (pseudo-random, fixed by layer and
 * position) before it is quantized; 0 turns it off. Not the reference's
 * arithmetic: it measures how far last-bit changes carry. */
void orc_model_set_attention_noise(orc_model* m, int ulps);
/* Rows of each layer's caches (the ring's with a sliding window). */
int64_t orc_model_ring(const orc_model* m);
void orc_model_free(orc_model* m);
/* Runs t tokens after those processed; logits of the last token -> logits[vocab].
 * Returns 0, or -1 with orc_last_error set (llama.cpp:300-305 errors). */
int orc_model_forward(orc_model* m, const int32_t* tokens, int64_t t, float* logits);
/* As orc_model_forward with every row's logits -> logits[t * vocab]
 * (Llama::forward_all, llama.cpp:393-396). */
int orc_model_forward_all(orc_model* m, const int32_t* tokens, int64_t t, float* logits);
/* Sets the score budget of the model's attention calls (a test hook that
 * makes short prompts take the chunked path). */
void orc_model_set_max_score_bytes(orc_model* m, int64_t bytes);
int64_t orc_model_position(const orc_model* m);
int orc_model_set_position(orc_model* m, int64_t position); /* timing samples only */
int64_t orc_model_rewind(orc_model* m, int64_t position); /* -1 on error */
void orc_model_reset(orc_model* m);
int64_t orc_model_vocab(const orc_model* m);
/* vocab, hidden, ffn, layers, heads, kv_heads, head_dim, context. */
void orc_model_dims(const orc_model* m, int64_t out[8]);
/* The layer-0 k cache as the model holds it (f32 or f16 bits), for cache tests. */
const void* orc_model_k_cache(const orc_model* m, int layer);
const void* orc_model_v_cache(const orc_model* m, int layer);
/* Copies layer l's caches [kv_heads, context, hd] in (f16 bits or f32, as the
 * model holds them), so that a cache computed elsewhere -- the GPU's prefill
 * of a long prompt -- is continued here with orc_model_set_position. */
int orc_model_set_kv(orc_model* m, int layer, const void* k, const void* v);

/* ---- the sampler: src/io/sampling.cpp:17-139 (oracle_sampling.c) ---- */
typedef struct orc_sampler orc_sampler;
orc_sampler* orc_sampler_new(float temperature, int top_k, float top_p, uint64_t seed, float repetition_penalty,
                             float min_p, float frequency_penalty, float presence_penalty);
void orc_sampler_free(orc_sampler* s);
int32_t orc_sampler_sample(orc_sampler* s, const float* logits, int64_t n, const int32_t* previous,
                           int64_t n_previous);
/* token_logprobs (src/io/sampling.cpp:141-164); writes min(top, n) entries. */
float orc_token_logprobs(const float* logits, int64_t n, int32_t token, int top, int32_t* top_ids, float* top_logprobs);
/* The generator alone, for its pins: the next 64-bit output, and a
 * uniform_real_distribution<double>(0, total) draw. */
uint64_t orc_sampler_draw_u64(orc_sampler* s);
double orc_sampler_draw_uniform(orc_sampler* s, double total);

/* Double-precision forward of the dequantized weights from scratch, no
 * activation quantization (tests/test_llama.cpp:585-755): logits of the last
 * token. Returns 0 or -1. */
int orc_model_reference_f64(const char* gguf_path, const int32_t* tokens, int64_t t,
                            double* logits);

#ifdef __cplusplus
}
#endif
#endif
