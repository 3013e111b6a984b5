/*
 * vkml_oracle.c -- CPU restatement of vkml's decode-path kernels.
 *
 * TEST INFRASTRUCTURE ONLY (see vkml_oracle.h): the checker for the HIP
 * product, never part of it. Built with -ffp-contract=off by oracle/Makefile.
 */
#include "vkml_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static __thread char g_error[512];
static int g_threads = 1;

const char* orc_last_error(void) { return g_error; }
void orc_set_threads(int threads) { g_threads = threads < 1 ? 1 : (threads > 256 ? 256 : threads); }
int orc_get_threads(void) { return g_threads; }

/* Runs fn(ctx, begin, end) over [0, n) split across g_threads threads. Each
 * output of the products below is computed by one call on its own, so the
 * results do not depend on the thread count. */
typedef void (*range_fn)(void* ctx, int64_t begin, int64_t end);
typedef struct { range_fn fn; void* ctx; int64_t begin, end; } range_job;
/* Set on the threads of a parallel_for while they run its ranges: a
 * parallel_for inside one runs serially there. */
static __thread int t_in_parallel;

static void* range_thread(void* p) {
    range_job* j = (range_job*)p;
    t_in_parallel = 1;
    j->fn(j->ctx, j->begin, j->end);
    return NULL;
}
static void parallel_for(int64_t n, range_fn fn, void* ctx) {
    if (t_in_parallel) { fn(ctx, 0, n); return; }
    int threads = g_threads;
    if (threads > n) threads = (int)(n > 0 ? n : 1);
    if (threads <= 1) { fn(ctx, 0, n); return; }
    pthread_t tid[256];
    range_job jobs[256];
    const int64_t per = (n + threads - 1) / threads;
    int started = 0;
    for (int t = 1; t < threads; ++t) {
        const int64_t b = per * t, e = b + per < n ? b + per : n;
        if (b >= n) break;
        jobs[t] = (range_job){fn, ctx, b, e};
        if (pthread_create(&tid[t], NULL, range_thread, &jobs[t]) != 0) {
            fn(ctx, b, e);
            jobs[t].fn = NULL;
        }
        started = t;
    }
    t_in_parallel = 1;
    fn(ctx, 0, per < n ? per : n);
    t_in_parallel = 0;
    for (int t = 1; t <= started; ++t) if (jobs[t].fn) pthread_join(tid[t], NULL);
}

void orc_error(const char* fmt, const char* a, long long b, long long c);
void orc_error(const char* fmt, const char* a, long long b, long long c) {
    snprintf(g_error, sizeof g_error, fmt, a, b, c);
}

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ------------------------------------------------------------------------ */
/* 16-bit floats                                                             */
/* ------------------------------------------------------------------------ */

/* src/io/host_quant.cpp:74-90 (and halves.glsl:61-70): exact widening,
 * subnormals kept as mantissa * 2^-24. */
float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exponent = (h >> 10) & 0x1Fu, mantissa = h & 0x3FFu;
    uint32_t bits;
    if (exponent == 0) {
        bits = f2u((float)mantissa * 5.9604644775390625e-8f) | sign;
    } else if (exponent == 31) {
        bits = sign | 0x7F800000u | (mantissa << 13);
    } else {
        bits = sign | ((exponent + 112u) << 23) | (mantissa << 13);
    }
    return u2f(bits);
}

/* src/io/host_quant.cpp:92-114: round to nearest even; past 65504's
 * rounding range, infinity; NaN keeps its sign and becomes quiet (0x7E00).
 * shaders/include/halves.glsl:73-91 (to_f16) computes the same bits. */
uint16_t orc_f32_to_f16(float f) {
    const uint32_t x = f2u(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t biased = (x >> 23) & 0xFFu;
    uint32_t mantissa = x & 0x7FFFFFu;
    if (biased == 0xFFu) return (uint16_t)(sign | 0x7C00u | (mantissa ? 0x200u : 0u));
    const int exponent = (int)biased - 127 + 15;
    if (exponent >= 31) return (uint16_t)(sign | 0x7C00u);
    if (exponent <= 0) {
        if (exponent < -10) return (uint16_t)sign;
        mantissa |= 0x800000u;
        const int shift = 14 - exponent;
        const uint32_t kept = mantissa >> shift, rest = mantissa & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1);
        return (uint16_t)(sign | (kept + ((rest > half || (rest == half && (kept & 1u))) ? 1u : 0u)));
    }
    const uint32_t value = ((uint32_t)exponent << 23) | mantissa;
    const uint32_t kept = value >> 13, rest = value & 0x1FFFu;
    return (uint16_t)(sign | (kept + ((rest > 0x1000u || (rest == 0x1000u && (kept & 1u))) ? 1u : 0u)));
}

float orc_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); } /* halves.glsl:93 */

/* e^x as a fixed sequence of f32 operations, shared bit for bit with the GPU
 * kernels. The reference calls GLSL exp (unary.comp:22, attend.comp:129,
 * attend_merge.comp:34, softmax.comp), whose accuracy its driver defines:
 * parity with it is unpinned at the last bit; tests pin this function against
 * libm's exp within 2 ulp. Method: Cody-Waite reduction x = n ln2 + r with ln2
 * split into a 15-bit head 0.693145751953125 and a tail, |r| <= ln2/2; e^r by
 * its degree-7 Taylor polynomial (coefficients 1/k! rounded to f32) in Horner
 * form; 2^n through the exponent bits. */
float orc_expf(float x) {
    if (x != x) return x;
    if (x > 88.72283935546875f) return INFINITY;
    if (x < -86.5f) return 0.0f;
    const float n = rintf(x * 1.44269502162933349609375f);
    const float r = (x - n * 0.693145751953125f) - n * 1.428606765330187045037746429443359375e-6f;
    float p = 1.98412701138295233249664306640625e-4f;
    p = p * r + 1.388888922519981861114501953125e-3f;
    p = p * r + 8.333333767950534820556640625e-3f;
    p = p * r + 4.16666679084300994873046875e-2f;
    p = p * r + 1.6666667163372039794921875e-1f;
    p = p * r + 0.5f;
    p = p * r + 1.0f;
    p = p * r + 1.0f;
    const int e = (int)n;
    if (e > 127) return p * 1.70141183460469231731687303715884105728e38f * 2.0f;
    return p * u2f((uint32_t)(e + 127) << 23);
}
void orc_expf_array(const float* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_expf(x[i]);
}

void orc_cast_f32_to_f16(const float* x, uint16_t* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_f32_to_f16(x[i]);
}
void orc_cast_f16_to_f32(const uint16_t* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_f16_to_f32(x[i]);
}

/* ------------------------------------------------------------------------ */
/* ggml block decoders: src/io/gguf.cpp:117-228                              */
/* ------------------------------------------------------------------------ */

static uint16_t rd16(const uint8_t* p) { uint16_t v; memcpy(&v, p, 2); return v; }

/* gguf.cpp:117-120 */
static void dq_q8_0(const uint8_t* b, float* y) {
    const float d = orc_f16_to_f32(rd16(b));
    for (int j = 0; j < 32; ++j) y[j] = (float)(int8_t)b[2 + j] * d;
}

/* gguf.cpp:231-254 (legacy q4_0 / q4_1; the q5 forms are not on the path). */
static void dq_legacy4(const uint8_t* b, float* y, int offset) {
    const float d = orc_f16_to_f32(rd16(b));
    const float m = offset ? orc_f16_to_f32(rd16(b + 2)) : 0.0f;
    const uint8_t* qs = b + (offset ? 4 : 2);
    for (int j = 0; j < 16; ++j) {
        const int q0 = qs[j] & 0x0F, q1 = qs[j] >> 4;
        if (offset) {
            y[j] = (float)q0 * d + m;
            y[j + 16] = (float)q1 * d + m;
        } else {
            y[j] = (float)(q0 - 8) * d;
            y[j + 16] = (float)(q1 - 8) * d;
        }
    }
}

/* gguf.cpp:123-131: 6-bit scale and min of sub-block j. */
static void scale_min_k4(int j, const uint8_t* q, uint8_t* sc, uint8_t* m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* gguf.cpp:203-228 (q4_K: d*scale*q - dmin*min). */
static void dq_q4_k(const uint8_t* b, float* y) {
    const float d = orc_f16_to_f32(rd16(b));
    const float dmin = orc_f16_to_f32(rd16(b + 2));
    const uint8_t* scales = b + 4;
    const uint8_t* q = b + 16;
    for (int j = 0, is = 0; j < 256; j += 64, is += 2) {
        uint8_t sc, m;
        scale_min_k4(is, scales, &sc, &m);
        const float d1 = d * (float)sc, m1 = dmin * (float)m;
        scale_min_k4(is + 1, scales, &sc, &m);
        const float d2 = d * (float)sc, m2 = dmin * (float)m;
        for (int l = 0; l < 32; ++l) *y++ = d1 * (float)(q[l] & 0xF) - m1;
        for (int l = 0; l < 32; ++l) *y++ = d2 * (float)(q[l] >> 4) - m2;
        q += 32;
    }
}

/* gguf.cpp:135-157 (q6_K: (q - 32) * d * scale). */
static void dq_q6_k(const uint8_t* b, float* y) {
    const uint8_t* ql = b;
    const uint8_t* qh = b + 128;
    const int8_t* sc = (const int8_t*)(b + 192);
    const float d = orc_f16_to_f32(rd16(b + 208));
    for (int n = 0; n < 256; n += 128) {
        for (int l = 0; l < 32; ++l) {
            const int is = l / 16;
            const int q1 = ((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
            const int q2 = ((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
            const int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            const int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            y[l] = d * (float)sc[is] * (float)q1;
            y[l + 32] = d * (float)sc[is + 2] * (float)q2;
            y[l + 64] = d * (float)sc[is + 4] * (float)q3;
            y[l + 96] = d * (float)sc[is + 6] * (float)q4;
        }
        y += 128;
        ql += 64;
        qh += 32;
        sc += 8;
    }
}

typedef struct { int values, bytes; void (*decode)(const uint8_t*, float*); } block_t;

static void dq_q4_0(const uint8_t* b, float* y) { dq_legacy4(b, y, 0); }
static void dq_q4_1(const uint8_t* b, float* y) { dq_legacy4(b, y, 1); }

/* gguf.cpp:266-287 restricted to the types on the path. */
static int host_block(int type, block_t* out) {
    switch (type) {
        case ORC_GGML_Q8_0: *out = (block_t){32, 34, dq_q8_0}; return 1;
        case ORC_GGML_Q4_0: *out = (block_t){32, 18, dq_q4_0}; return 1;
        case ORC_GGML_Q4_1: *out = (block_t){32, 20, dq_q4_1}; return 1;
        case ORC_GGML_Q4_K: *out = (block_t){256, 144, dq_q4_k}; return 1;
        case ORC_GGML_Q6_K: *out = (block_t){256, 210, dq_q6_k}; return 1;
        default: return 0;
    }
}

int64_t orc_dequantize_ggml(int type, const uint8_t* blocks, int64_t nbytes, float* out) {
    block_t b;
    if (!host_block(type, &b) || nbytes % b.bytes != 0) return -1;
    const int64_t n = nbytes / b.bytes;
    for (int64_t i = 0; i < n; ++i) b.decode(blocks + i * b.bytes, out + i * b.values);
    return n * b.values;
}

int64_t orc_ggml_row_bytes(int type, int64_t cols) {
    if (type == ORC_GGML_F32) return cols * 4;
    if (type == ORC_GGML_F16 || type == ORC_GGML_BF16) return cols * 2;
    block_t b;
    if (!host_block(type, &b) || cols % b.values != 0) return -1;
    return cols / b.values * b.bytes;
}

/* ------------------------------------------------------------------------ */
/* Load-time repacking: src/io/gguf.cpp:525-638, host_quant.cpp:116-159     */
/* ------------------------------------------------------------------------ */

/* gguf.cpp:552-561: vkml's word holds codes 8w+k (low nibble) and 8w+k+4. */
static void pack_codes(uint32_t* words, const uint8_t codes[32]) {
    for (int w = 0; w < 4; ++w) {
        uint32_t word = 0;
        for (int k = 0; k < 4; ++k) {
            const uint32_t byte = (uint32_t)codes[8 * w + k] | ((uint32_t)codes[8 * w + k + 4] << 4);
            word |= byte << (8 * k);
        }
        words[w] = word;
    }
}

/* gguf.cpp:563-570: ggml's legacy byte j holds value j and j + 16. */
static void split_nibbles(const uint8_t* qs, uint8_t codes[32]) {
    for (int j = 0; j < 16; ++j) {
        codes[j] = qs[j] & 0x0F;
        codes[j + 16] = qs[j] >> 4;
    }
}

int orc_load_quantized(int type, const uint8_t* data, int64_t rows, int64_t cols, uint32_t* words,
                       uint16_t* halves) {
    const int64_t groups = rows * cols / 32;
    uint8_t codes[32];
    if (type == ORC_GGML_Q8_0 || type == ORC_GGML_Q4_0) {
        const int q8 = type == ORC_GGML_Q8_0;
        if (cols % 32) return -1;
        for (int64_t b = 0; b < groups; ++b) {
            const uint8_t* block = data + b * (q8 ? 34 : 18);
            halves[b] = rd16(block);
            if (q8) {
                memcpy(&words[b * 8], block + 2, 32);
            } else {
                split_nibbles(block + 2, codes);
                pack_codes(&words[b * 4], codes);
            }
        }
        return q8 ? ORC_Q8_0 : ORC_Q4_0;
    }
    if (type == ORC_GGML_Q4_1) {
        if (cols % 32) return -1;
        for (int64_t b = 0; b < groups; ++b) {
            const uint8_t* block = data + b * 20;
            halves[2 * b] = rd16(block);
            halves[2 * b + 1] = rd16(block + 2);
            split_nibbles(block + 4, codes);
            pack_codes(&words[b * 4], codes);
        }
        return ORC_Q4_1;
    }
    if (type == ORC_GGML_Q4_K) {
        /* gguf.cpp:596-627: sub-block s is Q4_1 with scale f16(d * sc_s) and
         * offset f16(-(dmin * m_s)); sub-blocks 2c and 2c+1 are the low and
         * high nibbles of bytes 32c .. 32c + 31. */
        if (cols % 256) return -1;
        for (int64_t b = 0; b < groups / 8; ++b) {
            const uint8_t* block = data + b * 144;
            const float d = orc_f16_to_f32(rd16(block));
            const float dmin = orc_f16_to_f32(rd16(block + 2));
            const uint8_t* qs = block + 16;
            for (int sub = 0; sub < 8; ++sub) {
                uint8_t sc, m;
                scale_min_k4(sub, block + 4, &sc, &m);
                const int64_t group = b * 8 + sub;
                halves[2 * group] = orc_f32_to_f16(d * (float)sc);
                halves[2 * group + 1] = orc_f32_to_f16(-(dmin * (float)m));
                const uint8_t* bytes = qs + 32 * (sub / 2);
                for (int l = 0; l < 32; ++l) codes[l] = sub % 2 == 0 ? (bytes[l] & 0x0F) : (bytes[l] >> 4);
                pack_codes(&words[group * 4], codes);
            }
        }
        return ORC_Q4_1;
    }
    return -1;
}

/* host_quant.cpp:63-70: round half to even by the 1.5 * 2^23 addition. */
static float round_even_magic(float x) {
    const volatile float magic = 12582912.0f;
    return (x + magic) - magic;
}

static float clampf(float v, float lo, float hi) { return v < lo ? lo : (hi < v ? hi : v); }

/* host_quant.cpp:125-150: one 32-value group to Q8_0 with an f16 scale. */
static void q8_group_host(const float* x, uint32_t* words, uint16_t* scale) {
    float absmax = 0.0f;
    for (int i = 0; i < 32; ++i) absmax = fmaxf(absmax, fabsf(x[i]));
    *scale = orc_f32_to_f16(absmax / 127.0f);
    const float d = orc_f16_to_f32(*scale);
    const float inv = d > 0.0f ? 1.0f / d : 0.0f;
    for (int w = 0; w < 8; ++w) {
        uint32_t word = 0;
        for (int k = 0; k < 4; ++k) {
            const float v = clampf(round_even_magic(x[4 * w + k] * inv), -127.0f, 127.0f);
            word |= ((uint32_t)(int32_t)v & 0xFFu) << (8 * k);
        }
        words[w] = word;
    }
}

int orc_load_q8(int type, const uint8_t* data, int64_t rows, int64_t cols, uint32_t* words,
                uint16_t* halves) {
    block_t b;
    if (cols % 32) return -1;
    float y[256];
    const int64_t count = rows * cols;
    if (type == ORC_GGML_F32 || type == ORC_GGML_F16 || type == ORC_GGML_BF16) {
        /* Float types go through quantize_q8 on the GPU (gguf.cpp:511); with
         * f16 scales it picks the same codes as the host (quantize.comp). */
        for (int64_t g = 0; g < count / 32; ++g) {
            for (int i = 0; i < 32; ++i) {
                const int64_t e = g * 32 + i;
                y[i] = type == ORC_GGML_F32 ? ((const float*)data)[e]
                       : type == ORC_GGML_F16 ? orc_f16_to_f32(((const uint16_t*)data)[e])
                                              : orc_bf16_to_f32(((const uint16_t*)data)[e]);
            }
            orc_quantize(ORC_Q8_0, 1, y, 1, 32, &words[g * 8], &halves[g]);
        }
        return ORC_Q8_0;
    }
    if (!host_block(type, &b) || count % b.values) return -1;
    for (int64_t u = 0; u < count / b.values; ++u) {
        b.decode(data + u * b.bytes, y);
        for (int g = 0; g < b.values; g += 32) {
            const int64_t group = (u * b.values + g) / 32;
            q8_group_host(y + g, &words[group * 8], &halves[group]);
        }
    }
    return ORC_Q8_0;
}

/* ------------------------------------------------------------------------ */
/* quantize.comp / dequantize.comp                                           */
/* ------------------------------------------------------------------------ */

/* halves.glsl:27 */
static uint32_t q4_shift(uint32_t i) { return 8u * (i & 3u) + 4u * ((i >> 2) & 1u); }

/* quantize.comp:158-165 */
static float kept(float x, int f16, uint16_t* bits) {
    if (!f16) { *bits = 0; return x; }
    *bits = orc_f32_to_f16(x);
    return orc_f16_to_f32(*bits);
}

/* quantize.comp:169-223: block b's codes; returns (scale, offset) as kept. */
static void quantize_block(int quant, int f16, const float* x, uint32_t* q, float* d_out,
                           float* m_out, uint16_t* bits_d, uint16_t* bits_m) {
    *bits_m = 0;
    if (quant == ORC_Q4_1) {
        float lo = x[0], hi = lo;
        for (int i = 1; i < 32; ++i) { lo = fminf(lo, x[i]); hi = fmaxf(hi, x[i]); }
        const float m = kept(lo, f16, bits_m);
        const float d = kept((hi - lo) / 15.0f, f16, bits_d);
        const float inv = d > 0.0f ? 1.0f / d : 0.0f;
        for (int w = 0; w < 4; ++w) {
            uint32_t word = 0;
            for (uint32_t j = 0; j < 8; ++j) {
                const float code = clampf(rintf((x[8 * w + j] - m) * inv), 0.0f, 15.0f);
                word |= (uint32_t)code << q4_shift(j);
            }
            q[w] = word;
        }
        *d_out = d; *m_out = m;
        return;
    }
    if (quant == ORC_Q4_0) {
        float m = 0.0f;
        for (int i = 0; i < 32; ++i) if (fabsf(x[i]) > fabsf(m)) m = x[i];
        const float d = kept(m / -8.0f, f16, bits_d);
        const float inv = d != 0.0f ? 1.0f / d : 0.0f;
        for (int w = 0; w < 4; ++w) {
            uint32_t word = 0;
            for (uint32_t j = 0; j < 8; ++j) {
                const int v = (int)clampf(rintf(x[8 * w + j] * inv), -8.0f, 7.0f);
                word |= (uint32_t)(v + 8) << q4_shift(j);
            }
            q[w] = word;
        }
        *d_out = d; *m_out = 0.0f;
        return;
    }
    float absmax = 0.0f;
    for (int i = 0; i < 32; ++i) absmax = fmaxf(absmax, fabsf(x[i]));
    const float d = kept(absmax / 127.0f, f16, bits_d);
    const float inv = d > 0.0f ? 1.0f / d : 0.0f;
    for (int w = 0; w < 8; ++w) {
        uint32_t word = 0;
        for (int j = 0; j < 4; ++j) {
            const int v = (int)clampf(rintf(x[4 * w + j] * inv), -127.0f, 127.0f);
            word |= ((uint32_t)v & 0xFFu) << (8 * j);
        }
        q[w] = word;
    }
    *d_out = d; *m_out = 0.0f;
}

void orc_quantize(int quant, int f16, const float* x, int64_t rows, int64_t cols, uint32_t* words,
                  void* scales) {
    const int64_t blocks = rows * cols / 32;
    const int per_word = quant == ORC_Q8_0 ? 8 : 4; /* words per block */
    for (int64_t b = 0; b < blocks; ++b) {
        float d, m;
        uint16_t bd, bm;
        quantize_block(quant, f16, x + b * 32, words + b * per_word, &d, &m, &bd, &bm);
        if (!f16) {
            float* s = (float*)scales;
            if (quant == ORC_Q4_1) { s[2 * b] = d; s[2 * b + 1] = m; } else { s[b] = d; }
        } else {
            uint16_t* s = (uint16_t*)scales;
            if (quant == ORC_Q4_1) { s[2 * b] = bd; s[2 * b + 1] = bm; } else { s[b] = bd; }
        }
    }
}

static float scale_at(const void* scales, int f16, int64_t i) {
    return f16 ? orc_f16_to_f32(((const uint16_t*)scales)[i]) : ((const float*)scales)[i];
}

/* dequantize.comp:37-48 */
void orc_dequantize(int quant, int f16, const uint32_t* words, const void* scales, int64_t rows,
                    int64_t cols, float* out) {
    const int64_t count = rows * cols;
    for (int64_t e = 0; e < count; ++e) {
        if (quant == ORC_Q4_1) {
            const int64_t block = e / 32;
            const float code = (float)((words[e / 8] >> q4_shift((uint32_t)e)) & 15u);
            out[e] = code * scale_at(scales, f16, 2 * block) + scale_at(scales, f16, 2 * block + 1);
        } else if (quant == ORC_Q4_0) {
            const float v = (float)((int)((words[e / 8] >> q4_shift((uint32_t)e)) & 15u) - 8);
            out[e] = v * scale_at(scales, f16, e / 32);
        } else {
            const float v = (float)(int8_t)(words[e / 4] >> (8 * (e & 3)));
            out[e] = v * scale_at(scales, f16, e / 32);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* int8 products                                                             */
/* ------------------------------------------------------------------------ */

static int32_t dot4(uint32_t a, uint32_t b) {
    int32_t s = 0;
    for (int k = 0; k < 4; ++k) s += (int32_t)(int8_t)(a >> (8 * k)) * (int32_t)(int8_t)(b >> (8 * k));
    return s;
}

/* gemv_dot.comp:314-316 */
static uint32_t q4_bytes(uint32_t word, uint32_t shift) {
    return (((word >> shift) & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u;
}

/* The four words of weights pairing with half block i of row n's a
 * (gemv_dot.comp:334-344). */
static void half_block_weights(int quant, const uint32_t* b, int64_t idx, uint32_t w[4]) {
    if (quant == ORC_Q8_0) {
        memcpy(w, b + idx * 4, 16);
    } else {
        const uint32_t x = b[idx * 2], y = b[idx * 2 + 1];
        if (quant == ORC_Q4_0) {
            w[0] = q4_bytes(x, 0); w[1] = q4_bytes(x, 4); w[2] = q4_bytes(y, 0); w[3] = q4_bytes(y, 4);
        } else {
            w[0] = x & 0x0F0F0F0Fu; w[1] = (x >> 4) & 0x0F0F0F0Fu;
            w[2] = y & 0x0F0F0F0Fu; w[3] = (y >> 4) & 0x0F0F0F0Fu;
        }
    }
}

/* gemv_dot.comp:318-379 with ROWS = 4: 32 lanes per output stride over half
 * blocks, each half block's exact integer sum scaled in f32, then a shared-
 * memory halving tree over the lanes. */
typedef struct {
    int quant, f16;
    const uint32_t* a_words; const float* a_scales; int64_t M;
    const void* b; const void* sc; int64_t N, K;
    const float* af; int t; float* out;
} prod_ctx;

static void gemv_dot_range(void* p, int64_t n0, int64_t n1) {
    const prod_ctx* c = (const prod_ctx*)p;
    const int quant = c->quant, f16 = c->f16;
    const uint32_t* a_words = c->a_words; const float* a_scales = c->a_scales;
    const uint32_t* b_words = (const uint32_t*)c->b; const void* b_scales = c->sc;
    const int64_t M = c->M, N = c->N, K = c->K;
    float* out = c->out;
    const int64_t lanes = 32, halves = K / 16;
    for (int64_t n = n0; n < n1; ++n) {
        for (int64_t r = 0; r < M; ++r) {
            float partial[32];
            for (int64_t lane = 0; lane < lanes; ++lane) {
                float acc = 0.0f;
                for (int64_t i = lane; i < halves; i += lanes) {
                    uint32_t w[4];
                    const int64_t idx = n * halves + i;
                    half_block_weights(quant, b_words, idx, w);
                    const int64_t block = idx / 2;
                    const float scale = quant == ORC_Q4_1 ? scale_at(b_scales, f16, 2 * block)
                                                          : scale_at(b_scales, f16, block);
                    const float offset = quant == ORC_Q4_1 ? scale_at(b_scales, f16, 2 * block + 1) : 0.0f;
                    const uint32_t* x = a_words + (r * halves + i) * 4;
                    const int32_t d = dot4(x[0], w[0]) + dot4(x[1], w[1]) + dot4(x[2], w[2]) + dot4(x[3], w[3]);
                    const float sa = a_scales[(r * halves + i) / 2];
                    if (quant == ORC_Q4_1) {
                        const uint32_t ones = 0x01010101u;
                        const int32_t sum = dot4(x[0], ones) + dot4(x[1], ones) + dot4(x[2], ones) + dot4(x[3], ones);
                        acc += sa * ((float)d * scale + (float)sum * offset);
                    } else {
                        acc += (float)d * (scale * sa);
                    }
                }
                partial[lane] = acc;
            }
            for (int64_t s = lanes / 2; s > 0; s /= 2)
                for (int64_t l = 0; l < s; ++l) partial[l] += partial[l + s];
            out[r * N + n] = partial[0];
        }
    }
}

void orc_gemv_dot(int quant, int f16, const uint32_t* a_words, const float* a_scales, int64_t M,
                  const uint32_t* b_words, const void* b_scales, int64_t N, int64_t K, float* out) {
    prod_ctx c = {quant, f16, a_words, a_scales, M, b_words, b_scales, N, K, NULL, 0, out};
    parallel_for(N, gemv_dot_range, &c);
}

/* matmul_dot.comp:75-170: per output, one 32-value block per step, the
 * block's exact integer sum scaled in f32 and added in block order. The
 * integer sums are formed from codes unpacked to bytes once per column (and
 * the scales widened once per column), CT columns at a time so that each row
 * of a is read once per tile; an exact integer sum does not depend on how it
 * is formed, and the f32 steps per output are matmul_dot.comp's, in its
 * order. */
enum { MM_CT = 16 };

static int32_t dot32_i8(const int8_t* a, const int8_t* b) {
    int32_t s = 0;
    for (int k = 0; k < 32; ++k) s += (int32_t)a[k] * (int32_t)b[k];
    return s;
}

static void matmul_dot_range(void* p, int64_t c0, int64_t c1) {
    const prod_ctx* c = (const prod_ctx*)p;
    const int quant = c->quant, f16 = c->f16;
    const int8_t* a = (const int8_t*)c->a_words; const float* a_scales = c->a_scales;
    const uint32_t* b_words = (const uint32_t*)c->b; const void* b_scales = c->sc;
    const int64_t M = c->M, N = c->N, K = c->K;
    float* out = c->out;
    const int64_t blocks = K / 32;
    const int q4 = quant != ORC_Q8_0, offs = quant == ORC_Q4_1;
    const int64_t b_row_words = q4 ? K / 8 : K / 4;
    int8_t* bq = (int8_t*)malloc((size_t)(MM_CT * K));
    float* bs = (float*)malloc((size_t)(MM_CT * blocks) * 4);
    float* bo = (float*)malloc((size_t)(MM_CT * blocks) * 4);
    int32_t* asum = offs ? (int32_t*)malloc((size_t)(M * blocks) * 4) : NULL;
    if (offs) {
        for (int64_t r = 0; r < M; ++r)
            for (int64_t blk = 0; blk < blocks; ++blk) {
                int32_t t = 0;
                for (int k = 0; k < 32; ++k) t += a[r * K + blk * 32 + k];
                asum[r * blocks + blk] = t;
            }
    }
    for (int64_t t0 = c0; t0 < c1; t0 += MM_CT) {
        const int64_t nt = c1 - t0 < MM_CT ? c1 - t0 : MM_CT;
        for (int64_t j = 0; j < nt; ++j) {
            const int64_t col = t0 + j;
            int8_t* dst = bq + j * K;
            for (int64_t blk = 0; blk < blocks; ++blk) {
                for (int w = 0; w < 8; ++w) {
                    uint32_t bv;
                    if (q4) {
                        const uint32_t q = b_words[col * b_row_words + blk * 4 + w / 2];
                        if (offs) bv = (w % 2 == 0) ? (q & 0x0F0F0F0Fu) : ((q >> 4) & 0x0F0F0F0Fu);
                        else bv = q4_bytes(q, (uint32_t)(w % 2) * 4);
                    } else {
                        bv = b_words[col * b_row_words + blk * 8 + w];
                    }
                    for (int k = 0; k < 4; ++k) dst[blk * 32 + 4 * w + k] = (int8_t)(bv >> (8 * k));
                }
                const int64_t block = col * blocks + blk;
                bs[j * blocks + blk] = scale_at(b_scales, f16, offs ? 2 * block : block);
                bo[j * blocks + blk] = offs ? scale_at(b_scales, f16, 2 * block + 1) : 0.0f;
            }
        }
        for (int64_t row = 0; row < M; ++row) {
            const int8_t* ar = a + row * K;
            for (int64_t j = 0; j < nt; ++j) {
                const int8_t* br = bq + j * K;
                float acc = 0.0f;
                for (int64_t blk = 0; blk < blocks; ++blk) {
                    const int32_t sums = dot32_i8(ar + blk * 32, br + blk * 32);
                    const float sa = a_scales[row * blocks + blk];
                    if (offs) {
                        acc += sa * ((float)sums * bs[j * blocks + blk] + (float)asum[row * blocks + blk] * bo[j * blocks + blk]);
                    } else {
                        acc += (float)sums * (sa * bs[j * blocks + blk]);
                    }
                }
                out[row * N + t0 + j] = acc;
            }
        }
    }
    free(bq); free(bs); free(bo); free(asum);
}

void orc_matmul_dot(int quant, int f16, const uint32_t* a_words, const float* a_scales, int64_t M,
                    const uint32_t* b_words, const void* b_scales, int64_t N, int64_t K,
                    float* out) {
    prod_ctx c = {quant, f16, a_words, a_scales, M, b_words, b_scales, N, K, NULL, 0, out};
    parallel_for(N, matmul_dot_range, &c);
}

/* ------------------------------------------------------------------------ */
/* Float matrix-vector path: gemv.comp                                       */
/* ------------------------------------------------------------------------ */

/* gemv.comp:62-92 load_b4 / load_b for element type t. */
static void load_b4(int t, int f16, const void* b, const void* sc, int64_t row_start, int64_t i,
                    float w[4]) {
    const int64_t e = row_start + 4 * i;
    if (t == ORC_T_F32) { memcpy(w, (const float*)b + e, 16); return; }
    if (t == ORC_T_F16 || t == ORC_T_BF16) {
        const uint16_t* h = (const uint16_t*)b + e;
        for (int k = 0; k < 4; ++k) w[k] = t == ORC_T_F16 ? orc_f16_to_f32(h[k]) : orc_bf16_to_f32(h[k]);
        return;
    }
    const uint32_t* q = (const uint32_t*)b;
    if (t == ORC_T_Q8) {
        const uint32_t word = q[e / 4];
        const float s = scale_at(sc, f16, e / 32);
        for (int k = 0; k < 4; ++k) w[k] = (float)(int8_t)(word >> (8 * k)) * s;
        return;
    }
    const uint32_t h = q[e / 8] >> (4 * (i & 1));
    const int64_t block = e / 32;
    for (int k = 0; k < 4; ++k) {
        const float code = (float)((h >> (8 * k)) & 15u);
        if (t == ORC_T_Q4_1) {
            w[k] = code * scale_at(sc, f16, 2 * block) + scale_at(sc, f16, 2 * block + 1);
        } else {
            w[k] = (code - 8.0f) * scale_at(sc, f16, block);
        }
    }
}

static float load_b1(int t, int f16, const void* b, const void* sc, int64_t j) {
    if (t == ORC_T_F32) return ((const float*)b)[j];
    if (t == ORC_T_F16) return orc_f16_to_f32(((const uint16_t*)b)[j]);
    if (t == ORC_T_BF16) return orc_bf16_to_f32(((const uint16_t*)b)[j]);
    const uint32_t* q = (const uint32_t*)b;
    if (t == ORC_T_Q8) return (float)(int8_t)(q[j / 4] >> (8 * (j & 3))) * scale_at(sc, f16, j / 32);
    const float code = (float)((q[j / 8] >> q4_shift((uint32_t)j)) & 15u);
    if (t == ORC_T_Q4_1)
        return code * scale_at(sc, f16, 2 * (j / 32)) + scale_at(sc, f16, 2 * (j / 32) + 1);
    return (code - 8.0f) * scale_at(sc, f16, j / 32);
}

static float dotv(const float* a, const float* w) {
    return a[0] * w[0] + a[1] * w[1] + a[2] * w[2] + a[3] * w[3];
}

/* gemv.comp:101-212 with ROWS = 4 (32 lanes per output). The quantized main
 * loops issue four loads lanes apart before using them; the sums they make
 * are the same as load_b4's, in the same order per lane. */
static void gemv_float_range(void* p, int64_t n0, int64_t n1) {
    const prod_ctx* c = (const prod_ctx*)p;
    const int t = c->t, f16 = c->f16;
    const float* a = c->af; const void* b = c->b; const void* sc = c->sc;
    const int64_t M = c->M, K = c->K, N = c->N;
    float* out = c->out;
    const int64_t lanes = 32;
    for (int64_t n = n0; n < n1; ++n) {
        const int64_t b_row = n * K;
        for (int64_t r = 0; r < M; ++r) {
            float partial[32];
            for (int64_t lane = 0; lane < lanes; ++lane) {
                float acc = 0.0f;
                if ((K & 3) == 0) {
                    const int64_t k4 = K / 4;
                    int64_t i = lane;
                    if (t == ORC_T_Q4 || t == ORC_T_Q4_1 || t == ORC_T_Q8) {
                        for (; i + 3 * lanes < k4; i += 4 * lanes) {
                            for (int u = 0; u < 4; ++u) {
                                float w[4];
                                load_b4(t, f16, b, sc, b_row, i + u * lanes, w);
                                acc += dotv(a + r * K + 4 * (i + u * lanes), w);
                            }
                        }
                    }
                    for (; i < k4; i += lanes) {
                        float w[4];
                        load_b4(t, f16, b, sc, b_row, i, w);
                        acc += dotv(a + r * K + 4 * i, w);
                    }
                } else {
                    for (int64_t k = lane; k < K; k += lanes) acc += a[r * K + k] * load_b1(t, f16, b, sc, b_row + k);
                }
                partial[lane] = acc;
            }
            for (int64_t s = lanes / 2; s > 0; s /= 2)
                for (int64_t l = 0; l < s; ++l) partial[l] += partial[l + s];
            out[r * N + n] = partial[0];
        }
    }
}

void orc_gemv_float(int t, int f16, const float* a, int64_t M, const void* b, const void* sc,
                    int64_t N, int64_t K, float* out) {
    prod_ctx c = {0, f16, NULL, NULL, M, b, sc, N, K, a, t, out};
    parallel_for(N, gemv_float_range, &c);
}

/* matmul.comp:117-142 with B_TRANSPOSED: each output sums a[m][k] * b(n, k)
 * in k order, b widened as load_b does (matmul.comp:74-84); the tiles' zero
 * padding adds nothing. */
static void matmul_float_range(void* p, int64_t n0, int64_t n1) {
    const prod_ctx* c = (const prod_ctx*)p;
    for (int64_t n = n0; n < n1; ++n) {
        for (int64_t r = 0; r < c->M; ++r) {
            float acc = 0.0f;
            for (int64_t k = 0; k < c->K; ++k) acc += c->af[r * c->K + k] * load_b1(c->t, c->f16, c->b, c->sc, n * c->K + k);
            c->out[r * c->N + n] = acc;
        }
    }
}

void orc_matmul_float(int t, int f16, const float* a, int64_t M, const void* b, const void* sc,
                      int64_t N, int64_t K, float* out) {
    prod_ctx c = {0, f16, NULL, NULL, M, b, sc, N, K, a, t, out};
    parallel_for(N, matmul_float_range, &c);
}

/* ------------------------------------------------------------------------ */
/* Norms, rope, activations, argmax, embeddings                              */
/* ------------------------------------------------------------------------ */

/* rms_norm.comp:26-57 with a workgroup of 256 (Runtime::workgroup_width):
 * strided per-invocation sums, then a halving tree. inversesqrt is taken as
 * 1 / sqrt, correctly rounded (the reference's accuracy for it is its
 * driver's: parity unpinned at the last bit). */
void orc_rms_norm(const float* x, const float* w, int64_t rows, int64_t cols, float eps, float* out) {
    const int64_t width = 256;
    for (int64_t row = 0; row < rows; ++row) {
        const float* xr = x + row * cols;
        float scratch[256];
        for (int64_t tid = 0; tid < width; ++tid) {
            float s = 0.0f;
            for (int64_t c = tid; c < cols; c += width) s += xr[c] * xr[c];
            scratch[tid] = s;
        }
        for (int64_t n = width; n > 1;) {
            const int64_t half = (n + 1) / 2;
            for (int64_t tid = 0; tid < n - half; ++tid) scratch[tid] += scratch[tid + half];
            n = half;
        }
        const float scale = 1.0f / sqrtf(scratch[0] / (float)cols + eps);
        for (int64_t c = 0; c < cols; ++c) out[row * cols + c] = xr[c] * scale * w[c];
    }
}

/* src/ops/rope.cpp:32-86 without scaling or factors: cos and sin of
 * pos * theta^(-2i/head_dim) in double, stored as f32 pairs. */
void orc_rope_table(int64_t positions, int64_t head_dim, float theta, float* table) {
    const int64_t half = head_dim / 2;
    for (int64_t pos = 0; pos < positions; ++pos) {
        for (int64_t i = 0; i < half; ++i) {
            const double inv = pow((double)theta, -2.0 * (double)i / (double)head_dim);
            const double angle = (double)pos * inv;
            table[(pos * half + i) * 2] = (float)(1.0 * cos(angle));
            table[(pos * half + i) * 2 + 1] = (float)(1.0 * sin(angle));
        }
    }
}

/* rope.comp:94-118; style 0 interleaved pairs (2i, 2i+1), 1 rotate-half. */
void orc_rope(const float* x, const float* table, int64_t rows, int64_t heads, int64_t seq,
              int64_t dim, int64_t half_dim, int64_t start_pos, int style, float* out) {
    const int64_t rest = dim - 2 * half_dim;
    for (int64_t row = 0; row < rows; ++row) {
        const int64_t pos = start_pos + (row / heads) % seq;
        const int64_t base = row * dim;
        for (int64_t i = 0; i < half_dim; ++i) {
            const int64_t ia = base + (style == 0 ? 2 * i : i);
            const int64_t ib = base + (style == 0 ? 2 * i + 1 : i + half_dim);
            const float c = table[(pos * half_dim + i) * 2], s = table[(pos * half_dim + i) * 2 + 1];
            const float a = x[ia], b = x[ib];
            out[ia] = a * c - b * s;
            out[ib] = a * s + b * c;
        }
        for (int64_t q = 0; q < rest; ++q) out[base + 2 * half_dim + q] = x[base + 2 * half_dim + q];
    }
}

/* unary.comp:21-24 */
void orc_silu(const float* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = x[i] / (1.0f + orc_expf(-x[i]));
}

/* binary.comp:26-43: op 0 add, 1 sub, 2 mul, 3 div; b repeats. */
void orc_binary(int op, const float* a, const float* b, int64_t n, int64_t b_count, float* out) {
    for (int64_t i = 0; i < n; ++i) {
        const float x = a[i], y = b[i % b_count];
        out[i] = op == 0 ? x + y : op == 1 ? x - y : op == 2 ? x * y : x / y;
    }
}

/* argmax.comp:27-62: the first of the largest non-NaN entries; all NaN gives 0. */
int32_t orc_argmax(const float* x, int64_t n) {
    int64_t best = -1;
    for (int64_t i = 0; i < n; ++i) {
        if (isnan(x[i])) continue;
        if (best < 0 || x[i] > x[best]) best = i;
    }
    return best < 0 ? 0 : (int32_t)best;
}

/* embedding_quantized.comp:321-336 */
void orc_embedding_quantized(int quant, const uint32_t* words, const uint16_t* halves,
                             int64_t vocab, int64_t dim, const int32_t* ids, int64_t n, float* out) {
    for (int64_t i = 0; i < n * dim; ++i) {
        const int32_t id = ids[i / dim];
        const int64_t col = i % dim;
        if (id < 0 || id >= vocab) { out[i] = 0.0f; continue; }
        const int64_t e = (int64_t)id * dim + col;
        if (quant == ORC_Q4_1) {
            const int64_t block = e / 32;
            const float code = (float)((words[e / 8] >> q4_shift((uint32_t)e)) & 15u);
            out[i] = code * orc_f16_to_f32(halves[2 * block]) + orc_f16_to_f32(halves[2 * block + 1]);
        } else if (quant == ORC_Q4_0) {
            const float v = (float)((int)((words[e / 8] >> q4_shift((uint32_t)e)) & 15u) - 8);
            out[i] = v * orc_f16_to_f32(halves[e / 32]);
        } else {
            out[i] = (float)(int8_t)(words[e / 4] >> (8 * (e & 3))) * orc_f16_to_f32(halves[e / 32]);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Attention                                                                 */
/* ------------------------------------------------------------------------ */

static float kv_at(const void* base, int f16, int64_t i) {
    return f16 ? orc_f16_to_f32(((const uint16_t*)base)[i]) : ((const float*)base)[i];
}

/* attend.comp:80-169 (WG = CHUNK = 128, 4 lanes per key) and
 * attend_merge.comp:194-208. f16 values widen exactly here; the reference
 * widens with unpackHalf2x16, which its driver may flush below 6.1e-5
 * (attend.comp:65-68): parity unpinned for subnormal cache entries. */
void orc_attend_decode(const float* q, int64_t heads, const void* k, const void* v, int f16,
                       int64_t kv_heads, int64_t capacity, int64_t hd, int64_t kv_start,
                       int64_t kv_len, float softcap, float* out) {
    const int64_t WG = 128, CHUNK = 128, LANES = 4;
    const int64_t group = heads / kv_heads;
    const int64_t chunks = (kv_len - kv_start + CHUNK - 1) / CHUNK;
    const float scale = 1.0f / sqrtf((float)hd);
    float* partial = (float*)malloc(sizeof(float) * (size_t)(chunks * hd));
    float* stats = (float*)malloc(sizeof(float) * (size_t)(chunks * 2));
    for (int64_t h = 0; h < heads; ++h) {
        const int64_t kv_row0 = (h / group) * capacity;
        const float* qh = q + h * hd;
        for (int64_t c = 0; c < chunks; ++c) {
            const int64_t key0 = kv_start + c * CHUNK;
            const int64_t n = (kv_len - key0) < CHUNK ? (kv_len - key0) : CHUNK;
            float p[128], red[128];
            for (int64_t key = 0; key < n; ++key) {
                const int64_t row = (kv_row0 + (key0 + key) % capacity) * hd;
                float parts[4];
                for (int64_t g = 0; g < LANES; ++g) {
                    float part = 0.0f;
                    for (int64_t i = g; i < hd / 4; i += LANES) {
                        float kk[4];
                        for (int j = 0; j < 4; ++j) kk[j] = kv_at(k, f16, row + 4 * i + j);
                        part += dotv(qh + 4 * i, kk);
                    }
                    parts[g] = part;
                }
                float dot_qk = 0.0f;
                for (int64_t j = 0; j < LANES; ++j) dot_qk += parts[j];
                const float s = dot_qk * scale;
                p[key] = softcap > 0.0f ? softcap * tanhf(clampf(s / softcap, -10.0f, 10.0f)) : s;
            }
            float m = -INFINITY;
            for (int64_t t = 0; t < n; ++t) m = fmaxf(m, p[t]);
            for (int64_t t = 0; t < WG; ++t) {
                const float weight = t < n ? orc_expf(p[t] - m) : 0.0f;
                if (t < n) p[t] = weight;
                red[t] = weight;
            }
            for (int64_t stride = WG / 2; stride > 0; stride /= 2)
                for (int64_t t = 0; t < stride; ++t) red[t] += red[t + stride];
            const float l = red[0];
            if (hd > WG) {
                for (int64_t d = 0; d < hd; ++d) {
                    float o = 0.0f;
                    for (int64_t key = 0; key < n; ++key)
                        o += p[key] * kv_at(v, f16, (kv_row0 + (key0 + key) % capacity) * hd + d);
                    partial[c * hd + d] = o;
                }
            } else {
                const int64_t slices = WG / hd;
                for (int64_t d = 0; d < hd; ++d) {
                    float sum = 0.0f;
                    for (int64_t slice = 0; slice < slices; ++slice) {
                        float o = 0.0f;
                        for (int64_t key = slice; key < n; key += slices)
                            o += p[key] * kv_at(v, f16, (kv_row0 + (key0 + key) % capacity) * hd + d);
                        sum += o;
                    }
                    partial[c * hd + d] = sum;
                }
            }
            stats[2 * c] = m;
            stats[2 * c + 1] = l;
        }
        for (int64_t d = 0; d < hd; ++d) {
            float top = stats[0];
            for (int64_t c = 1; c < chunks; ++c) top = fmaxf(top, stats[2 * c]);
            float sum = 0.0f, weight = 0.0f;
            for (int64_t c = 0; c < chunks; ++c) {
                const float r = orc_expf(stats[2 * c] - top);
                sum += r * partial[c * hd + d];
                weight += r * stats[2 * c + 1];
            }
            out[h * hd + d] = sum / weight;
        }
    }
    free(partial);
    free(stats);
}

/* attention.cpp:127-138 (attention_block) for queries q0..q0+rows of head
 * h against keys 0..keys: scores q k^T through gemv.comp for rows <= 8
 * (matmul.cpp:96, kGemvMaxRows) and matmul.comp's k order otherwise;
 * softmax.comp's causal rows (max; sum of exp in the shader's 256-wide
 * order; times 1/sum); then probs v in key order (matmul.comp). */
static void prefill_block(const float* q, int64_t q_len, int64_t q0, int64_t rows, int64_t h, const void* k,
                          const void* v, int f16, int64_t hd, int64_t keys, int64_t kv_row0, float softcap, float* s,
                          float* kf, float* vf, float* out) {
    const float scale = 1.0f / sqrtf((float)hd);
    const float* qh = q + (h * q_len + q0) * hd;
    /* the head's keys and values widened to f32 once (exact) */
    for (int64_t e = 0; e < keys * hd; ++e) {
        kf[e] = kv_at(k, f16, kv_row0 * hd + e);
        vf[e] = kv_at(v, f16, kv_row0 * hd + e);
    }
    if (rows <= 8) {
        orc_gemv_float(ORC_T_F32, 0, qh, rows, kf, NULL, keys, hd, s);
    } else {
        for (int64_t i = 0; i < rows; ++i)
            for (int64_t j = 0; j < keys; ++j) {
                float acc = 0.0f;
                for (int64_t c = 0; c < hd; ++c) acc += qh[i * hd + c] * kf[j * hd + c];
                s[i * keys + j] = acc;
            }
    }
    for (int64_t i = 0; i < rows; ++i) {
        float* si = s + i * keys;
        const int64_t position = i + keys - rows;
        const int64_t visible = position + 1 < keys ? position + 1 : keys;
        for (int64_t j = 0; j < visible; ++j) {
            const float sc = si[j] * scale;
            si[j] = softcap > 0.0f ? softcap * tanhf(clampf(sc / softcap, -10.0f, 10.0f)) : sc;
        }
        float m = -INFINITY;
        for (int64_t j = 0; j < visible; ++j) m = fmaxf(m, si[j]);
        /* softmax.comp:104-108: invocation t of 256 sums keys t, t+256, ..;
         * then the halving tree over the 256 partial sums. */
        float part[256];
        for (int64_t t = 0; t < 256; ++t) {
            float acc = 0.0f;
            for (int64_t j = t; j < visible; j += 256) acc += orc_expf(si[j] - m);
            part[t] = acc;
        }
        for (int64_t n = 256; n > 1;) {
            const int64_t half = (n + 1) / 2;
            for (int64_t t = 0; t < n - half; ++t) part[t] += part[t + half];
            n = half;
        }
        const float inv = 1.0f / part[0];
        for (int64_t j = 0; j < keys; ++j) si[j] = j < visible ? orc_expf(si[j] - m) * inv : 0.0f;
        for (int64_t c = 0; c < hd; ++c) {
            float acc = 0.0f;
            for (int64_t j = 0; j < keys; ++j) acc += si[j] * vf[j * hd + c];
            out[(h * q_len + q0 + i) * hd + c] = acc;
        }
    }
}

typedef struct {
    const float* q; int64_t q_len, q0, rows; const void* k; const void* v; int f16;
    int64_t hd, keys, group, capacity; float softcap; float* out;
} prefill_ctx;

/* Heads h0 .. h1 of one query chunk, each with buffers of its own. */
static void prefill_heads(void* p, int64_t h0, int64_t h1) {
    const prefill_ctx* c = (const prefill_ctx*)p;
    float* s = (float*)malloc(sizeof(float) * (size_t)(c->rows * (c->keys > 0 ? c->keys : 1)));
    float* kf = (float*)malloc(sizeof(float) * (size_t)(c->keys * c->hd + 1));
    float* vf = (float*)malloc(sizeof(float) * (size_t)(c->keys * c->hd + 1));
    for (int64_t h = h0; h < h1; ++h)
        prefill_block(c->q, c->q_len, c->q0, c->rows, h, c->k, c->v, c->f16, c->hd, c->keys, (h / c->group) * c->capacity,
                      c->softcap, s, kf, vf, c->out);
    free(s); free(kf); free(vf);
}

/* detail::attention for q_len > 1 (attention.cpp:205-226): queries in chunks
 * whose scores [heads, rows, kv_len] f32 fit max_score_bytes (a multiple of
 * 64 rows when at least 64), each chunk over the keys its last query sees. */
void orc_attention_prefill(const float* q, int64_t heads, int64_t q_len, const void* k,
                           const void* v, int f16, int64_t kv_heads, int64_t capacity, int64_t hd,
                           int64_t kv_len, int64_t max_score_bytes, float softcap, float* out) {
    const int64_t group = heads / kv_heads;
    const int64_t row_bytes = heads * (kv_len > 1 ? kv_len : 1) * 4;
    int64_t chunk = max_score_bytes / row_bytes;
    if (chunk < 1) chunk = 1;
    if (chunk >= 64) chunk -= chunk % 64;
    if (q_len <= chunk) chunk = q_len;
    const int64_t first_position = kv_len - q_len;
    for (int64_t q0 = 0; q0 < q_len; q0 += chunk) {
        const int64_t rows = chunk < q_len - q0 ? chunk : q_len - q0;
        const int64_t keys = q_len <= chunk ? kv_len : first_position + q0 + rows;
        prefill_ctx c = {q, q_len, q0, rows, k, v, f16, hd, keys, group, capacity, softcap, out};
        parallel_for(heads, prefill_heads, &c);
    }
}

/* ------------------------------------------------------------------------ */
/* Sliding-window attention over a ring: detail::sliding_attention            */
/* (attention.cpp:229-294) with attention_block's ring mask (:127-138,         */
/* softmax.comp:85-124 with CausalMask::ring).                                 */
/* ------------------------------------------------------------------------ */

/* attention_block over a ring of kv_len columns (rows 0 .. kv_len of the
 * caches), queries at positions first .. first + rows, each seeing the
 * last `window` positions up to its own, position p in column p % ring. */
static void ring_block(const float* q, int64_t heads, int64_t rows, const void* k, const void* v, int f16,
                       int64_t kv_heads, int64_t ring, int64_t hd, int64_t kv_len, int64_t first, int64_t window,
                       float softcap, float* out) {
    const int64_t group = heads / kv_heads;
    const float scale = 1.0f / sqrtf((float)hd);
    float* s = (float*)malloc(sizeof(float) * (size_t)(rows * kv_len));
    float* kf = (float*)malloc(sizeof(float) * (size_t)(kv_len * hd));
    float* vf = (float*)malloc(sizeof(float) * (size_t)(kv_len * hd));
    for (int64_t h = 0; h < heads; ++h) {
        const int64_t kv_row0 = (h / group) * ring;
        for (int64_t e = 0; e < kv_len * hd; ++e) {
            kf[e] = kv_at(k, f16, kv_row0 * hd + e);
            vf[e] = kv_at(v, f16, kv_row0 * hd + e);
        }
        const float* qh = q + h * rows * hd;
        /* scores: gemv.comp's order for up to 8 rows, matmul.comp's beyond */
        if (rows <= 8) {
            orc_gemv_float(ORC_T_F32, 0, qh, rows, kf, NULL, kv_len, hd, s);
        } else {
            for (int64_t i = 0; i < rows; ++i)
                for (int64_t j = 0; j < kv_len; ++j) {
                    float acc = 0.0f;
                    for (int64_t c = 0; c < hd; ++c) acc += qh[i * hd + c] * kf[j * hd + c];
                    s[i * kv_len + j] = acc;
                }
        }
        for (int64_t i = 0; i < rows; ++i) {
            float* si = s + i * kv_len;
            const int64_t visible = first + i + 1;
            const int64_t lo = window != 0 && visible > window ? visible - window : 0;
#define SCORE(col) (softcap > 0.0f ? softcap * tanhf(clampf(si[(col)] * scale / softcap, -10.0f, 10.0f)) : si[(col)] * scale)
            float m = -INFINITY;
            for (int64_t c = lo; c < visible; ++c) m = fmaxf(m, SCORE(c % ring));
            float part[256];
            for (int64_t t = 0; t < 256; ++t) {
                float acc = 0.0f;
                for (int64_t c = lo + t; c < visible; c += 256) acc += orc_expf(SCORE(c % ring) - m);
                part[t] = acc;
            }
            for (int64_t n = 256; n > 1;) {
                const int64_t half = (n + 1) / 2;
                for (int64_t t = 0; t < n - half; ++t) part[t] += part[t + half];
                n = half;
            }
            const float inv = 1.0f / part[0];
            const int64_t first_col = lo % ring;
            float* pr = (float*)malloc(sizeof(float) * (size_t)kv_len);
            for (int64_t c = 0; c < kv_len; ++c) {
                const int64_t from_first = c >= first_col ? c - first_col : c + ring - first_col;
                pr[c] = from_first < visible - lo ? orc_expf(SCORE(c) - m) * inv : 0.0f;
            }
#undef SCORE
            /* probs . v in key (column) order */
            for (int64_t c = 0; c < hd; ++c) {
                float acc = 0.0f;
                for (int64_t j = 0; j < kv_len; ++j) acc += pr[j] * vf[j * hd + c];
                out[(h * rows + i) * hd + c] = acc;
            }
            free(pr);
        }
    }
    free(s); free(kf); free(vf);
}

static void ring_append(const void* src, int64_t src_rows, int64_t row0, void* ring_cache, int64_t ring,
                        int64_t kv_heads, int64_t hd, int f16, int64_t from, int64_t rows) {
    const size_t esz = f16 ? 2 : 4;
    for (int64_t kh = 0; kh < kv_heads; ++kh)
        for (int64_t r = 0; r < rows; ++r)
            memcpy((char*)ring_cache + (size_t)((kh * ring + (from + r) % ring) * hd) * esz,
                   (const char*)src + (size_t)((kh * src_rows + row0 + r) * hd) * esz, (size_t)hd * esz);
}

void orc_attention_sliding(const float* q, int64_t heads, int64_t t, const void* k, const void* v, void* k_ring,
                           void* v_ring, int f16, int64_t kv_heads, int64_t ring, int64_t hd, int64_t start,
                           int64_t window, int64_t max_score_bytes, float softcap, float* out) {
    for (int64_t q0 = 0; q0 < t;) {
        const int64_t first = start + q0;
        const int64_t unwrapped = ring - first;
        int64_t chunk = ring - window + 1 > unwrapped ? ring - window + 1 : unwrapped;
        const int64_t keys = first + chunk < ring ? first + chunk : ring;
        int64_t budget = max_score_bytes / (heads * keys * 4);
        if (budget < 1) budget = 1;
        if (chunk > budget) chunk = budget;
        if (chunk >= 64) chunk -= chunk % 64;
        const int64_t rows = chunk < t - q0 ? chunk : t - q0;
        const int64_t end = first + rows;
        ring_append(k, t, q0, k_ring, ring, kv_heads, hd, f16, first, rows);
        ring_append(v, t, q0, v_ring, ring, kv_heads, hd, f16, first, rows);
        float* block = (float*)malloc(sizeof(float) * (size_t)(heads * rows * hd));
        float* qc = (float*)malloc(sizeof(float) * (size_t)(heads * rows * hd));
        for (int64_t h = 0; h < heads; ++h) memcpy(qc + h * rows * hd, q + (h * t + q0) * hd, sizeof(float) * (size_t)(rows * hd));
        if (rows == 1) {
            orc_attend_decode(qc, heads, k_ring, v_ring, f16, kv_heads, ring, hd, end - window > 0 ? end - window : 0, end,
                              softcap, block);
        } else {
            ring_block(qc, heads, rows, k_ring, v_ring, f16, kv_heads, ring, hd, end < ring ? end : ring, first, window,
                       softcap, block);
        }
        for (int64_t h = 0; h < heads; ++h) memcpy(out + (h * t + q0) * hd, block + h * rows * hd, sizeof(float) * (size_t)(rows * hd));
        free(block); free(qc);
        q0 += rows;
    }
}
