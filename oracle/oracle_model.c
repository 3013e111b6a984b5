/*
 * oracle_model.c -- CPU restatement of vkml's Llama token loop for GGUF
 * "llama"-architecture files (src/models/llama.cpp:170-406,
 * src/models/weights.cpp:26-159, src/models/config.cpp:14-140).
 *
 * TEST INFRASTRUCTURE ONLY (see vkml_oracle.h).
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "vkml_oracle.h"

void orc_error(const char* fmt, const char* a, long long b, long long c);

/* ------------------------------------------------------------------------ */
/* GGUF reading (format per src/io/gguf.cpp:310-387)                         */
/* ------------------------------------------------------------------------ */

typedef struct { char* key; int type; double num; char* str; } gkv;
typedef struct { char* name; int dims; int64_t shape[4]; int type; uint64_t offset; } gtensor;
typedef struct {
    uint8_t* file; size_t size;
    gkv* kvs; int64_t n_kv;
    gtensor* tensors; int64_t n_tensors;
    uint64_t data_start;
} gguf;

typedef struct { const uint8_t* p; const uint8_t* end; int bad; } rd;
static int rd_bytes(rd* r, void* out, size_t n) {
    if (r->bad || (size_t)(r->end - r->p) < n) { r->bad = 1; return 0; }
    memcpy(out, r->p, n);
    r->p += n;
    return 1;
}
static uint64_t rd_u64(rd* r) { uint64_t v = 0; rd_bytes(r, &v, 8); return v; }
static uint32_t rd_u32(rd* r) { uint32_t v = 0; rd_bytes(r, &v, 4); return v; }
static char* rd_str(rd* r) {
    const uint64_t n = rd_u64(r);
    if (r->bad || n > (uint64_t)(r->end - r->p)) { r->bad = 1; return NULL; }
    char* s = (char*)malloc(n + 1);
    rd_bytes(r, s, n);
    s[n] = 0;
    return s;
}
/* Reads a value of type t; scalars land in *num, strings in *str. */
static void rd_value(rd* r, int t, double* num, char** str, int depth) {
    union { uint8_t u8; int8_t i8; uint16_t u16; int16_t i16; uint32_t u32; int32_t i32; float f; uint64_t u64; int64_t i64; double d; } v = {0};
    *num = 0;
    switch (t) {
        case 0: rd_bytes(r, &v.u8, 1); *num = v.u8; break;
        case 1: rd_bytes(r, &v.i8, 1); *num = v.i8; break;
        case 2: rd_bytes(r, &v.u16, 2); *num = v.u16; break;
        case 3: rd_bytes(r, &v.i16, 2); *num = v.i16; break;
        case 4: rd_bytes(r, &v.u32, 4); *num = v.u32; break;
        case 5: rd_bytes(r, &v.i32, 4); *num = v.i32; break;
        case 6: rd_bytes(r, &v.f, 4); *num = v.f; break;
        case 7: rd_bytes(r, &v.u8, 1); *num = v.u8 != 0; break;
        case 8: { char* s = rd_str(r); if (str) *str = s; else free(s); break; }
        case 9: {
            if (depth > 4) { r->bad = 1; break; }
            const uint32_t et = rd_u32(r);
            const uint64_t count = rd_u64(r);
            if (count > ((uint64_t)1 << 28)) { r->bad = 1; break; }
            for (uint64_t i = 0; i < count && !r->bad; ++i) { double d; rd_value(r, (int)et, &d, NULL, depth + 1); }
            break;
        }
        case 10: rd_bytes(r, &v.u64, 8); *num = (double)v.u64; break;
        case 11: rd_bytes(r, &v.i64, 8); *num = (double)v.i64; break;
        case 12: rd_bytes(r, &v.d, 8); *num = v.d; break;
        default: r->bad = 1;
    }
}

static void gguf_free(gguf* g) {
    if (!g) return;
    for (int64_t i = 0; i < g->n_kv; ++i) { free(g->kvs[i].key); free(g->kvs[i].str); }
    for (int64_t i = 0; i < g->n_tensors; ++i) free(g->tensors[i].name);
    free(g->kvs); free(g->tensors); free(g->file); free(g);
}

static gguf* gguf_open(const char* path) {
    FILE* f = fopen(path, "rb");
    if (!f) { orc_error("gguf: %s: cannot open file", path, 0, 0); return NULL; }
    fseek(f, 0, SEEK_END);
    const long size = ftell(f);
    fseek(f, 0, SEEK_SET);
    gguf* g = (gguf*)calloc(1, sizeof(gguf));
    g->file = (uint8_t*)malloc((size_t)size);
    g->size = (size_t)size;
    if (fread(g->file, 1, (size_t)size, f) != (size_t)size) { fclose(f); gguf_free(g); orc_error("gguf: %s: read failed", path, 0, 0); return NULL; }
    fclose(f);
    rd r = {g->file, g->file + size, 0};
    char magic[4];
    rd_bytes(&r, magic, 4);
    const uint32_t version = rd_u32(&r);
    if (r.bad || memcmp(magic, "GGUF", 4) != 0 || version < 2 || version > 3) {
        gguf_free(g); orc_error("gguf: %s: not a GGUF v2/v3 file", path, 0, 0); return NULL;
    }
    g->n_tensors = (int64_t)rd_u64(&r);
    g->n_kv = (int64_t)rd_u64(&r);
    if (g->n_tensors > (1 << 24) || g->n_kv > (1 << 24)) { gguf_free(g); orc_error("gguf: %s: malformed counts", path, 0, 0); return NULL; }
    g->kvs = (gkv*)calloc((size_t)g->n_kv + 1, sizeof(gkv));
    g->tensors = (gtensor*)calloc((size_t)g->n_tensors + 1, sizeof(gtensor));
    uint64_t alignment = 32;
    for (int64_t i = 0; i < g->n_kv && !r.bad; ++i) {
        g->kvs[i].key = rd_str(&r);
        g->kvs[i].type = (int)rd_u32(&r);
        rd_value(&r, g->kvs[i].type, &g->kvs[i].num, &g->kvs[i].str, 0);
        if (g->kvs[i].key && strcmp(g->kvs[i].key, "general.alignment") == 0) alignment = (uint64_t)g->kvs[i].num;
    }
    for (int64_t i = 0; i < g->n_tensors && !r.bad; ++i) {
        gtensor* t = &g->tensors[i];
        t->name = rd_str(&r);
        t->dims = (int)rd_u32(&r);
        if (t->dims > 4) { r.bad = 1; break; }
        for (int d = 0; d < t->dims; ++d) t->shape[t->dims - 1 - d] = (int64_t)rd_u64(&r);
        t->type = (int)rd_u32(&r);
        t->offset = rd_u64(&r);
    }
    if (r.bad || alignment == 0) { gguf_free(g); orc_error("gguf: %s: malformed header", path, 0, 0); return NULL; }
    const uint64_t pos = (uint64_t)(r.p - g->file);
    g->data_start = (pos + alignment - 1) / alignment * alignment;
    return g;
}

static const gkv* gguf_kv(const gguf* g, const char* key) {
    for (int64_t i = 0; i < g->n_kv; ++i) if (g->kvs[i].key && strcmp(g->kvs[i].key, key) == 0) return &g->kvs[i];
    return NULL;
}
static const gtensor* gguf_tensor(const gguf* g, const char* name) {
    for (int64_t i = 0; i < g->n_tensors; ++i) if (strcmp(g->tensors[i].name, name) == 0) return &g->tensors[i];
    return NULL;
}
static const uint8_t* gguf_data(const gguf* g, const gtensor* t) { return g->file + g->data_start + t->offset; }

/* ------------------------------------------------------------------------ */
/* Model                                                                     */
/* ------------------------------------------------------------------------ */

enum { W_FLOAT = 0, W_QUANT = 1 };
typedef struct {
    int kind;   /* W_FLOAT: elem ORC_T_F32/F16/BF16; W_QUANT: quant ORC_Q* with f16 scales */
    int elem;
    int quant;
    void* data;      /* floats, 16-bit values, or quantized words */
    uint16_t* scales;
    int64_t rows, cols;
} weight;

typedef struct {
    float* attn_norm; float* ffn_norm;
    weight q, k, v, o, gate, up, down;
    void* k_cache; void* v_cache;
} layer;

struct orc_model {
    int64_t vocab, d, ff, n_layers, heads, kv_heads, hd, max_pos, context;
    float eps, theta;
    int tied, kv_f16, int_dot;
    weight embed, lm_head;
    float* final_norm;
    float* rope;
    layer* layers;
    int64_t position;
    int attention_noise; /* test instrumentation (orc_model_set_attention_noise); 0: none */
    int64_t max_score_bytes; /* attention's score budget (ORC_MAX_SCORE_BYTES) */
    /* Sliding window (every layer, 0: none): the caches are rings of
     * min(context, window + extra rows) rows; oldest_kept is the first
     * position the rings still hold (llama.cpp:236-241,273-285,356-364). */
    int64_t window, ring, oldest_kept;
    float attn_softcap, final_softcap;
};

static void weight_free(weight* w) { free(w->data); free(w->scales); }

static float clamp10(float v) { return v < -10.0f ? -10.0f : (10.0f < v ? 10.0f : v); }

/* weights.cpp:136-149 (quantized_named) and 128-134 (tensor_named): matrices
 * the file quantizes load quantized (q8_0/q4_0/q4_1/q4_K as they are or
 * repacked, others requantized to Q8_0); float matrices stay as stored. */
static int load_matrix(const gguf* g, const char* name, int64_t rows, int64_t cols, weight* w) {
    const gtensor* t = gguf_tensor(g, name);
    if (!t) { orc_error("Llama: the GGUF file has no tensor %s", name, 0, 0); return -1; }
    if (t->dims != 2 || t->shape[0] != rows || t->shape[1] != cols) {
        orc_error("Llama: weight %s is not [%lld, %lld]", name, (long long)rows, (long long)cols);
        return -1;
    }
    memset(w, 0, sizeof *w);
    w->rows = rows; w->cols = cols;
    const uint8_t* src = gguf_data(g, t);
    const int64_t count = rows * cols;
    if (t->type == ORC_GGML_F32 || t->type == ORC_GGML_F16 || t->type == ORC_GGML_BF16) {
        w->kind = W_FLOAT;
        w->elem = t->type == ORC_GGML_F32 ? ORC_T_F32 : t->type == ORC_GGML_F16 ? ORC_T_F16 : ORC_T_BF16;
        const size_t bytes = (size_t)count * (w->elem == ORC_T_F32 ? 4 : 2);
        w->data = malloc(bytes);
        memcpy(w->data, src, bytes);
        return 0;
    }
    w->kind = W_QUANT;
    const int direct = t->type == ORC_GGML_Q8_0 || t->type == ORC_GGML_Q4_0 ||
                       t->type == ORC_GGML_Q4_1 || t->type == ORC_GGML_Q4_K;
    const int q8 = !direct || t->type == ORC_GGML_Q8_0;
    w->data = malloc((size_t)(count / (q8 ? 4 : 8)) * 4);
    const int pairs = direct && (t->type == ORC_GGML_Q4_1 || t->type == ORC_GGML_Q4_K);
    w->scales = (uint16_t*)malloc((size_t)(count / 32) * 2 * (pairs ? 2 : 1));
    w->quant = direct ? orc_load_quantized(t->type, src, rows, cols, (uint32_t*)w->data, w->scales)
                      : orc_load_q8(t->type, src, rows, cols, (uint32_t*)w->data, w->scales);
    if (w->quant < 0) { orc_error("Llama: weight %s has a type the oracle cannot load", name, 0, 0); return -1; }
    return 0;
}

/* A vector weight widened to f32 (weights.cpp:20-23). */
static float* load_vector(const gguf* g, const char* name, int64_t n) {
    const gtensor* t = gguf_tensor(g, name);
    if (!t || t->dims != 1 || t->shape[0] != n) { orc_error("Llama: bad vector %s", name, 0, 0); return NULL; }
    float* v = (float*)malloc((size_t)n * 4);
    const uint8_t* src = gguf_data(g, t);
    for (int64_t i = 0; i < n; ++i) {
        if (t->type == ORC_GGML_F32) memcpy(&v[i], src + 4 * i, 4);
        else { uint16_t h; memcpy(&h, src + 2 * i, 2); v[i] = t->type == ORC_GGML_F16 ? orc_f16_to_f32(h) : orc_bf16_to_f32(h); }
    }
    return v;
}

static double kv_num(const gguf* g, const char* key, double fallback, int* found) {
    const gkv* kv = gguf_kv(g, key);
    if (found) *found = kv != NULL;
    return kv ? kv->num : fallback;
}

void orc_model_free(orc_model* m) {
    if (!m) return;
    weight_free(&m->embed);
    if (!m->tied) weight_free(&m->lm_head);
    free(m->final_norm); free(m->rope);
    for (int64_t l = 0; l < m->n_layers; ++l) {
        layer* L = &m->layers[l];
        free(L->attn_norm); free(L->ffn_norm);
        weight_free(&L->q); weight_free(&L->k); weight_free(&L->v); weight_free(&L->o);
        weight_free(&L->gate); weight_free(&L->up); weight_free(&L->down);
        free(L->k_cache); free(L->v_cache);
    }
    free(m->layers);
    free(m);
}

/* Test instrumentation, not the reference's arithmetic: moves each of
 * x[0 .. n) by a pseudo-random whole number of ulps in [-ulps, ulps] (a
 * linear congruential sequence seeded by seed; zeros stay), to measure how
 * far a change of an f32 result's last bits carries through the model. */
static void add_ulp_noise(float* x, int64_t n, int ulps, uint32_t seed) {
    uint32_t s = 12345u + seed;
    for (int64_t i = 0; i < n; ++i) {
        s = s * 1103515245u + 12345u;
        const int32_t d = (int32_t)((s >> 16) % (uint32_t)(2 * ulps + 1)) - ulps;
        if (x[i] == 0.0f) continue;
        uint32_t b;
        memcpy(&b, &x[i], 4);
        b = (uint32_t)((int32_t)b + d);
        memcpy(&x[i], &b, 4);
    }
}

void orc_model_set_attention_noise(orc_model* m, int ulps) { m->attention_noise = ulps; }

/* config.cpp:14-140 for arch "llama", then llama.cpp:170-271. The
 * reference reads a sliding window and soft caps from Gemma files only
 * (config.cpp:114-133) and ignores those keys in a llama file, as here: a
 * window over every layer (as the reference's HF Mistral configs apply it)
 * and the soft caps come from the caller (0: none). */
orc_model* orc_model_load(const char* path, int64_t context_length, int kv_f16, int int_dot) {
    return orc_model_load_opts(path, context_length, kv_f16, int_dot, 1024, 0, 0.0f, 0.0f);
}

orc_model* orc_model_load_ex(const char* path, int64_t context_length, int kv_f16, int int_dot, int64_t sliding_extra_rows) {
    return orc_model_load_opts(path, context_length, kv_f16, int_dot, sliding_extra_rows, 0, 0.0f, 0.0f);
}

orc_model* orc_model_load_opts(const char* path, int64_t context_length, int kv_f16, int int_dot, int64_t sliding_extra_rows,
                               int64_t window, float attn_softcap, float final_softcap) {
    gguf* g = gguf_open(path);
    if (!g) return NULL;
    const gkv* arch = gguf_kv(g, "general.architecture");
    if (!arch || !arch->str || strcmp(arch->str, "llama") != 0) {
        orc_error("Llama: %s is not a llama-architecture GGUF file", path, 0, 0);
        gguf_free(g);
        return NULL;
    }
    orc_model* m = (orc_model*)calloc(1, sizeof(orc_model));
    m->max_score_bytes = ORC_MAX_SCORE_BYTES;
    int ok = 1, f;
    m->d = (int64_t)kv_num(g, "llama.embedding_length", 0, &f); ok &= f;
    m->ff = (int64_t)kv_num(g, "llama.feed_forward_length", 0, &f); ok &= f;
    m->n_layers = (int64_t)kv_num(g, "llama.block_count", 0, &f); ok &= f;
    m->heads = (int64_t)kv_num(g, "llama.attention.head_count", 0, &f); ok &= f;
    m->kv_heads = (int64_t)kv_num(g, "llama.attention.head_count_kv", (double)m->heads, NULL);
    m->hd = (int64_t)kv_num(g, "llama.attention.key_length", m->heads ? (double)(m->d / m->heads) : 0, NULL);
    m->max_pos = (int64_t)kv_num(g, "llama.context_length", 0, &f); ok &= f;
    m->eps = (float)kv_num(g, "llama.attention.layer_norm_rms_epsilon", 1e-5f, NULL);
    m->theta = (float)kv_num(g, "llama.rope.freq_base", 10000.0f, NULL);
    m->window = window > 0 ? window : 0;
    m->attn_softcap = attn_softcap > 0.0f ? attn_softcap : 0.0f;
    m->final_softcap = final_softcap > 0.0f ? final_softcap : 0.0f;
    const gtensor* te = gguf_tensor(g, "token_embd.weight");
    if (!ok || !te) { orc_error("Llama: %s lacks config keys", path, 0, 0); gguf_free(g); free(m); return NULL; }
    m->vocab = te->shape[0];
    m->tied = gguf_tensor(g, "output.weight") == NULL;
    m->kv_f16 = kv_f16;
    m->int_dot = int_dot;
    m->context = context_length;
    if (context_length < 1 || context_length > m->max_pos || m->heads % m->kv_heads || m->hd % 2) {
        orc_error("Llama: context length %s%lld outside 1..%lld", "", (long long)context_length, (long long)m->max_pos);
        gguf_free(g); free(m); return NULL;
    }
    const int64_t d = m->d, qd = m->heads * m->hd, kvd = m->kv_heads * m->hd;
    m->ring = m->window ? (context_length < m->window + sliding_extra_rows ? context_length : m->window + sliding_extra_rows)
                        : context_length;
    m->layers = (layer*)calloc((size_t)m->n_layers, sizeof(layer));
    int err = load_matrix(g, "token_embd.weight", m->vocab, d, &m->embed);
    if (!err) {
        if (m->tied) m->lm_head = m->embed;
        else err = load_matrix(g, "output.weight", m->vocab, d, &m->lm_head);
    }
    m->final_norm = load_vector(g, "output_norm.weight", d);
    err |= m->final_norm == NULL;
    char name[128];
    const size_t esz = kv_f16 ? 2 : 4;
    for (int64_t l = 0; l < m->n_layers && !err; ++l) {
        layer* L = &m->layers[l];
#define MAT(field, suffix, r, c) snprintf(name, sizeof name, "blk.%lld." suffix, (long long)l); err |= load_matrix(g, name, r, c, &L->field);
        snprintf(name, sizeof name, "blk.%lld.attn_norm.weight", (long long)l);
        L->attn_norm = load_vector(g, name, d);
        snprintf(name, sizeof name, "blk.%lld.ffn_norm.weight", (long long)l);
        L->ffn_norm = load_vector(g, name, d);
        err |= !L->attn_norm || !L->ffn_norm;
        MAT(q, "attn_q.weight", qd, d)
        MAT(k, "attn_k.weight", kvd, d)
        MAT(v, "attn_v.weight", kvd, d)
        MAT(o, "attn_output.weight", d, qd)
        MAT(gate, "ffn_gate.weight", m->ff, d)
        MAT(up, "ffn_up.weight", m->ff, d)
        MAT(down, "ffn_down.weight", d, m->ff)
#undef MAT
        L->k_cache = calloc((size_t)(m->kv_heads * m->ring * m->hd), esz);
        L->v_cache = calloc((size_t)(m->kv_heads * m->ring * m->hd), esz);
    }
    gguf_free(g);
    if (err) { m->n_layers = 0; orc_model_free(m); return NULL; }
    m->rope = (float*)malloc((size_t)(context_length * m->hd) * 4);
    orc_rope_table(context_length, m->hd, m->theta, m->rope);
    return m;
}

int64_t orc_model_position(const orc_model* m) { return m->position; }
/* Moves the sequence to position without computing it: for timing a decode
 * step at a long context, whatever the (zero) cache rows hold. */
int orc_model_set_position(orc_model* m, int64_t position) {
    if (position < 0 || position >= m->context) return -1;
    m->position = position;
    return 0;
}
int64_t orc_model_vocab(const orc_model* m) { return m->vocab; }
void orc_model_dims(const orc_model* m, int64_t out[8]) {
    const int64_t d[8] = {m->vocab, m->d, m->ff, m->n_layers, m->heads, m->kv_heads, m->hd, m->context};
    memcpy(out, d, sizeof d);
}
void orc_model_reset(orc_model* m) { m->position = 0; m->oldest_kept = 0; }
int64_t orc_model_rewind(orc_model* m, int64_t position) {
    if (position < 0 || position > m->position) {
        orc_error("Llama::rewind: cannot rewind to position %s%lld of a sequence at %lld", "",
                  (long long)position, (long long)m->position);
        return -1;
    }
    /* the window of position's query must still be in the rings */
    const int64_t window = m->window ? m->window : 1;
    if ((position - window + 1 > 0 ? position - window + 1 : 0) < m->oldest_kept) position = 0;
    if (position == 0) m->oldest_kept = 0;
    m->position = position;
    return position;
}
int64_t orc_model_ring(const orc_model* m) { return m->ring; }
const void* orc_model_k_cache(const orc_model* m, int l) { return m->layers[l].k_cache; }
int orc_model_set_kv(orc_model* m, int l, const void* k, const void* v) {
    if (l < 0 || l >= m->n_layers || !k || !v) return -1;
    const size_t bytes = (size_t)(m->kv_heads * m->ring * m->hd) * (m->kv_f16 ? 2 : 4);
    memcpy(m->layers[l].k_cache, k, bytes);
    memcpy(m->layers[l].v_cache, v, bytes);
    return 0;
}
const void* orc_model_v_cache(const orc_model* m, int l) { return m->layers[l].v_cache; }

/* SharedInput::times_transposed (matmul.cpp:207-272): x [t, K] times w^T. The
 * quantized activation is computed once per shared input (aq). */
typedef struct { uint32_t* words; float* scales; } act_q;

static void project(const orc_model* m, const float* x, int64_t t, act_q* aq, const weight* w, float* y) {
    if (w->kind == W_QUANT && m->int_dot) {
        if (!aq->words) {
            aq->words = (uint32_t*)malloc((size_t)(t * w->cols));
            aq->scales = (float*)malloc((size_t)(t * w->cols / 32) * 4);
            orc_quantize(ORC_Q8_0, 0, x, t, w->cols, aq->words, aq->scales);
        }
        if (t <= 8) orc_gemv_dot(w->quant, 1, aq->words, aq->scales, t, (const uint32_t*)w->data, w->scales, w->rows, w->cols, y);
        else orc_matmul_dot(w->quant, 1, aq->words, aq->scales, t, (const uint32_t*)w->data, w->scales, w->rows, w->cols, y);
        return;
    }
    const int elem = w->kind == W_QUANT ? (w->quant == ORC_Q8_0 ? ORC_T_Q8 : w->quant == ORC_Q4_0 ? ORC_T_Q4 : ORC_T_Q4_1)
                                        : w->elem;
    if (t <= 8) orc_gemv_float(elem, 1, x, t, w->data, w->scales, w->rows, w->cols, y);
    else orc_matmul_float(elem, 1, x, t, w->data, w->scales, w->rows, w->cols, y);
}

static void act_free(act_q* a) { free(a->words); free(a->scales); a->words = NULL; a->scales = NULL; }

/* embedding of ids from the model's table (embedding.cpp:27-91). */
static void embed_rows(const orc_model* m, const int32_t* ids, int64_t t, float* x) {
    const weight* e = &m->embed;
    if (e->kind == W_QUANT) {
        orc_embedding_quantized(e->quant, (const uint32_t*)e->data, e->scales, m->vocab, m->d, ids, t, x);
        return;
    }
    for (int64_t i = 0; i < t; ++i) {
        for (int64_t c = 0; c < m->d; ++c) {
            float v = 0.0f;
            if (ids[i] >= 0 && ids[i] < m->vocab) {
                const int64_t at = (int64_t)ids[i] * m->d + c;
                v = e->elem == ORC_T_F32 ? ((const float*)e->data)[at]
                    : e->elem == ORC_T_F16 ? orc_f16_to_f32(((const uint16_t*)e->data)[at])
                                           : orc_bf16_to_f32(((const uint16_t*)e->data)[at]);
            }
            x[i * m->d + c] = v;
        }
    }
}

/* llama.cpp:299-406 for the llama architecture (no biases, q/k norms,
 * sandwich norms, soft caps or sliding windows). all: every row's logits
 * [t, vocab] (forward_all), else the last row's. */
static int model_run(orc_model* m, const int32_t* tokens, int64_t t, int all, float* logits) {
    if (t == 0) { orc_error("Llama::forward: no tokens%s", "", 0, 0); return -1; }
    if (m->position + t > m->context) {
        orc_error("Llama::forward: %s%lld tokens exceed the context length of %lld", "",
                  (long long)(m->position + t), (long long)m->context);
        return -1;
    }
    const int64_t d = m->d, hd = m->hd, H = m->heads, KVH = m->kv_heads, ff = m->ff;
    const int64_t qd = H * hd, kvd = KVH * hd, end = m->position + t;
    float* x = (float*)malloc((size_t)(t * d) * 4);
    float* h = (float*)malloc((size_t)(t * d) * 4);
    float* q = (float*)malloc((size_t)(t * qd) * 4);
    float* k = (float*)malloc((size_t)(t * kvd) * 4);
    float* v = (float*)malloc((size_t)(t * kvd) * 4);
    float* tmp = (float*)malloc((size_t)(t * (qd > kvd ? qd : kvd)) * 4);
    float* qh = (float*)malloc((size_t)(t * qd) * 4);
    float* att = (float*)malloc((size_t)(t * qd) * 4);
    float* merged = (float*)malloc((size_t)(t * qd) * 4);
    float* y = (float*)malloc((size_t)(t * (d > ff ? d : ff)) * 4);
    float* gate = (float*)malloc((size_t)(t * ff) * 4);
    float* up = (float*)malloc((size_t)(t * ff) * 4);
    embed_rows(m, tokens, t, x);
    for (int64_t l = 0; l < m->n_layers; ++l) {
        layer* L = &m->layers[l];
        orc_rms_norm(x, L->attn_norm, t, d, m->eps, h);
        act_q aq = {0};
        project(m, h, t, &aq, &L->q, q);
        project(m, h, t, &aq, &L->k, k);
        project(m, h, t, &aq, &L->v, v);
        act_free(&aq);
        /* heads_first (llama.cpp:320-327): rope on [t, heads, hd], then permute. */
        orc_rope(q, m->rope, t * H, H, t, hd, hd / 2, m->position, 0, tmp);
        for (int64_t i = 0; i < t; ++i)
            for (int64_t hh = 0; hh < H; ++hh)
                memcpy(qh + (hh * t + i) * hd, tmp + (i * H + hh) * hd, (size_t)hd * 4);
        orc_rope(k, m->rope, t * KVH, KVH, t, hd, hd / 2, m->position, 0, tmp);
        if (m->window) {
            /* heads-first k and v in the cache type, appended to the rings
             * chunk by chunk by sliding_attention (llama.cpp:356-364). */
            const size_t esz = m->kv_f16 ? 2 : 4;
            char* kh_rows = (char*)malloc((size_t)(t * kvd) * esz);
            char* vh_rows = (char*)malloc((size_t)(t * kvd) * esz);
            for (int64_t i = 0; i < t; ++i)
                for (int64_t kh = 0; kh < KVH; ++kh)
                    for (int64_t c = 0; c < hd; ++c) {
                        const float kv_k = tmp[(i * KVH + kh) * hd + c], kv_v = v[(i * KVH + kh) * hd + c];
                        const int64_t at = (kh * t + i) * hd + c;
                        if (m->kv_f16) {
                            ((uint16_t*)kh_rows)[at] = orc_f32_to_f16(kv_k);
                            ((uint16_t*)vh_rows)[at] = orc_f32_to_f16(kv_v);
                        } else {
                            ((float*)kh_rows)[at] = kv_k;
                            ((float*)vh_rows)[at] = kv_v;
                        }
                    }
            if (end - m->ring > m->oldest_kept) m->oldest_kept = end - m->ring;
            orc_attention_sliding(qh, H, t, kh_rows, vh_rows, L->k_cache, L->v_cache, m->kv_f16, KVH, m->ring, hd,
                                  m->position, m->window < m->ring ? m->window : m->ring, m->max_score_bytes,
                                  m->attn_softcap, att);
            free(kh_rows);
            free(vh_rows);
            goto attended;
        }
        /* cast to the cache type and write_rows at position (llama.cpp:344-355). */
        for (int64_t i = 0; i < t; ++i) {
            for (int64_t kh = 0; kh < KVH; ++kh) {
                const int64_t row = (kh * m->context + m->position + i) * hd;
                for (int64_t c = 0; c < hd; ++c) {
                    const float kv_k = tmp[(i * KVH + kh) * hd + c], kv_v = v[(i * KVH + kh) * hd + c];
                    if (m->kv_f16) {
                        ((uint16_t*)L->k_cache)[row + c] = orc_f32_to_f16(kv_k);
                        ((uint16_t*)L->v_cache)[row + c] = orc_f32_to_f16(kv_v);
                    } else {
                        ((float*)L->k_cache)[row + c] = kv_k;
                        ((float*)L->v_cache)[row + c] = kv_v;
                    }
                }
            }
        }
        /* detail::attention (attention.cpp:167-227): the fused decode kernel
         * for one query, attention_block otherwise. */
        if (t == 1) {
            orc_attend_decode(qh, H, L->k_cache, L->v_cache, m->kv_f16, KVH, m->context, hd, 0, end, m->attn_softcap, att);
            if (m->attention_noise > 0) add_ulp_noise(att, H * hd, m->attention_noise, (uint32_t)(l * 7919 + m->position * 31));
        }
        else orc_attention_prefill(qh, H, t, L->k_cache, L->v_cache, m->kv_f16, KVH, m->context, hd, end,
                                   m->max_score_bytes, m->attn_softcap, att);
    attended:
        for (int64_t i = 0; i < t; ++i)
            for (int64_t hh = 0; hh < H; ++hh)
                memcpy(merged + (i * H + hh) * hd, att + (hh * t + i) * hd, (size_t)hd * 4);
        act_q ao = {0};
        project(m, merged, t, &ao, &L->o, y);
        act_free(&ao);
        orc_binary(0, x, y, t * d, t * d, x);
        orc_rms_norm(x, L->ffn_norm, t, d, m->eps, h);
        act_q a2 = {0};
        project(m, h, t, &a2, &L->gate, gate);
        orc_silu(gate, gate, t * ff);
        project(m, h, t, &a2, &L->up, up);
        act_free(&a2);
        orc_binary(2, gate, up, t * ff, t * ff, gate);
        act_q a3 = {0};
        project(m, gate, t, &a3, &L->down, y);
        act_free(&a3);
        orc_binary(0, x, y, t * d, t * d, x);
    }
    m->position = end;
    /* llama.cpp:392-405: the final norm of every row; all rows through the
     * output projection, or the last row alone. */
    act_q al = {0};
    if (all) {
        orc_rms_norm(x, m->final_norm, t, d, m->eps, h);
        project(m, h, t, &al, &m->lm_head, logits);
    } else {
        orc_rms_norm(x + (t - 1) * d, m->final_norm, 1, d, m->eps, h);
        project(m, h, 1, &al, &m->lm_head, logits);
    }
    act_free(&al);
    /* the final soft cap (llama.cpp:405, unary.comp:35) */
    if (m->final_softcap > 0.0f) {
        const float cap = m->final_softcap;
        for (int64_t i = 0; i < (all ? t : 1) * m->vocab; ++i) logits[i] = cap * tanhf(clamp10(logits[i] / cap));
    }
    free(x); free(h); free(q); free(k); free(v); free(tmp); free(qh); free(att); free(merged);
    free(y); free(gate); free(up);
    return 0;
}

int orc_model_forward(orc_model* m, const int32_t* tokens, int64_t t, float* logits) {
    return model_run(m, tokens, t, 0, logits);
}

int orc_model_forward_all(orc_model* m, const int32_t* tokens, int64_t t, float* logits) {
    return model_run(m, tokens, t, 1, logits);
}

void orc_model_set_max_score_bytes(orc_model* m, int64_t bytes) { m->max_score_bytes = bytes; }

/* ------------------------------------------------------------------------ */
/* Double-precision reference: tests/test_llama.cpp:585-755                  */
/* ------------------------------------------------------------------------ */

/* The f32 values a loaded weight stands for (vkml's dequantized weights). */
static double* weight_values(const weight* w) {
    const int64_t n = w->rows * w->cols;
    double* out = (double*)malloc((size_t)n * 8);
    float* tmp = (float*)malloc((size_t)n * 4);
    if (w->kind == W_QUANT) {
        orc_dequantize(w->quant, 1, (const uint32_t*)w->data, w->scales, w->rows, w->cols, tmp);
    } else {
        for (int64_t i = 0; i < n; ++i)
            tmp[i] = w->elem == ORC_T_F32 ? ((const float*)w->data)[i]
                     : w->elem == ORC_T_F16 ? orc_f16_to_f32(((const uint16_t*)w->data)[i])
                                            : orc_bf16_to_f32(((const uint16_t*)w->data)[i]);
    }
    for (int64_t i = 0; i < n; ++i) out[i] = tmp[i];
    free(tmp);
    return out;
}

static void matvec_d(const double* mtx, const double* x, int64_t in, int64_t out_n, double* y) {
    for (int64_t o = 0; o < out_n; ++o) {
        double s = 0.0;
        for (int64_t i = 0; i < in; ++i) s += mtx[o * in + i] * x[i];
        y[o] = s;
    }
}
static void rms_d(const double* x, const float* w, int64_t n, double eps, double* y) {
    double ss = 0.0;
    for (int64_t i = 0; i < n; ++i) ss += x[i] * x[i];
    const double scale = 1.0 / sqrt(ss / (double)n + eps);
    for (int64_t i = 0; i < n; ++i) y[i] = x[i] * scale * (double)w[i];
}
/* Interleaved pairs, as the GGUF llama architecture rotates them. */
static void rope_d(double* v, int64_t n_heads, int64_t hd, int64_t pos, double theta) {
    for (int64_t h = 0; h < n_heads; ++h) {
        for (int64_t i = 0; i < hd / 2; ++i) {
            const double inv = pow(theta, -2.0 * (double)i / (double)hd);
            const double angle = (double)pos * inv;
            double* a = &v[h * hd + 2 * i];
            double* b = &v[h * hd + 2 * i + 1];
            const double a0 = *a, b0 = *b;
            *a = a0 * cos(angle) - b0 * sin(angle);
            *b = a0 * sin(angle) + b0 * cos(angle);
        }
    }
}

int orc_model_reference_f64(const char* path, const int32_t* tokens, int64_t t, double* logits) {
    orc_model* m = orc_model_load(path, t, 0, 0);
    if (!m) return -1;
    const int64_t d = m->d, hd = m->hd, H = m->heads, KVH = m->kv_heads, ff = m->ff;
    const int64_t qd = H * hd, kvd = KVH * hd;
    double* x = (double*)calloc((size_t)(t * d), 8);
    double* emb = weight_values(&m->embed);
    for (int64_t i = 0; i < t; ++i)
        for (int64_t c = 0; c < d; ++c) x[i * d + c] = tokens[i] >= 0 && tokens[i] < m->vocab ? emb[(int64_t)tokens[i] * d + c] : 0.0;
    double* q = (double*)malloc((size_t)(t * qd) * 8);
    double* k = (double*)malloc((size_t)(t * kvd) * 8);
    double* v = (double*)malloc((size_t)(t * kvd) * 8);
    double* h = (double*)malloc((size_t)d * 8);
    double* attn = (double*)malloc((size_t)qd * 8);
    double* o = (double*)malloc((size_t)d * 8);
    double* g = (double*)malloc((size_t)ff * 8);
    double* u = (double*)malloc((size_t)ff * 8);
    double* s = (double*)malloc((size_t)t * 8);
    for (int64_t l = 0; l < m->n_layers; ++l) {
        layer* L = &m->layers[l];
        double* wq = weight_values(&L->q); double* wk = weight_values(&L->k); double* wv = weight_values(&L->v);
        double* wo = weight_values(&L->o); double* wg = weight_values(&L->gate); double* wu = weight_values(&L->up);
        double* wd = weight_values(&L->down);
        for (int64_t i = 0; i < t; ++i) {
            rms_d(x + i * d, L->attn_norm, d, m->eps, h);
            matvec_d(wq, h, d, qd, q + i * qd);
            matvec_d(wk, h, d, kvd, k + i * kvd);
            matvec_d(wv, h, d, kvd, v + i * kvd);
            rope_d(q + i * qd, H, hd, i, m->theta);
            rope_d(k + i * kvd, KVH, hd, i, m->theta);
        }
        for (int64_t i = 0; i < t; ++i) {
            for (int64_t hh = 0; hh < H; ++hh) {
                const int64_t kh = hh / (H / KVH);
                double mx = -1e300, sum = 0.0;
                for (int64_t j = 0; j <= i; ++j) {
                    double acc = 0.0;
                    for (int64_t c = 0; c < hd; ++c) acc += q[i * qd + hh * hd + c] * k[j * kvd + kh * hd + c];
                    s[j] = acc / sqrt((double)hd);
                    if (s[j] > mx) mx = s[j];
                }
                for (int64_t j = 0; j <= i; ++j) sum += (s[j] = exp(s[j] - mx));
                for (int64_t c = 0; c < hd; ++c) {
                    double acc = 0.0;
                    for (int64_t j = 0; j <= i; ++j) acc += s[j] / sum * v[j * kvd + kh * hd + c];
                    attn[hh * hd + c] = acc;
                }
            }
            matvec_d(wo, attn, qd, d, o);
            for (int64_t c = 0; c < d; ++c) x[i * d + c] += o[c];
            rms_d(x + i * d, L->ffn_norm, d, m->eps, h);
            matvec_d(wg, h, d, ff, g);
            matvec_d(wu, h, d, ff, u);
            for (int64_t c = 0; c < ff; ++c) g[c] = g[c] / (1.0 + exp(-g[c])) * u[c];
            matvec_d(wd, g, ff, d, o);
            for (int64_t c = 0; c < d; ++c) x[i * d + c] += o[c];
        }
        free(wq); free(wk); free(wv); free(wo); free(wg); free(wu); free(wd);
    }
    rms_d(x + (t - 1) * d, m->final_norm, d, m->eps, h);
    double* head = weight_values(&m->lm_head);
    matvec_d(head, h, d, m->vocab, logits);
    free(head); free(emb); free(x); free(q); free(k); free(v); free(h); free(attn); free(o);
    free(g); free(u); free(s);
    orc_model_free(m);
    return 0;
}
