/* oracle_sampling.c -- test infrastructure: the reference's Sampler
 * (src/io/sampling.cpp:17-139) restated in C, with its generator
 * std::mt19937_64 (Matsumoto and Nishimura's 64-bit Mersenne Twister,
 * the parameters of the C++ standard's [rand.predef]) and libstdc++'s
 * uniform_real_distribution<double> (generate_canonical<double, 53> over
 * one 64-bit draw: x / 2^64, kept below 1). Candidates of equal logit are
 * ordered by token id. Checked against the C++ standard's 10000th output,
 * libstdc++ itself, and the product's sampler. */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "vkml_oracle.h"

#define MT_N 312
#define MT_M 156

struct orc_sampler {
    float temperature, top_p, repetition_penalty, min_p, frequency_penalty, presence_penalty;
    int top_k;
    uint64_t mt[MT_N];
    int mti;
    int32_t* picked_ids; /* tokens this sampler picked and how often, for the penalties */
    int* picked_counts;
    int64_t picked_n, picked_cap;
};

static void mt_seed(orc_sampler* s, uint64_t seed) {
    s->mt[0] = seed;
    for (int i = 1; i < MT_N; ++i) s->mt[i] = 6364136223846793005ULL * (s->mt[i - 1] ^ (s->mt[i - 1] >> 62)) + (uint64_t)i;
    s->mti = MT_N;
}

static uint64_t mt_next(orc_sampler* s) {
    static const uint64_t mag[2] = {0ULL, 0xB5026F5AA96619E9ULL};
    const uint64_t upper = 0xFFFFFFFF80000000ULL, lower = 0x7FFFFFFFULL;
    if (s->mti >= MT_N) {
        int i;
        for (i = 0; i < MT_N - MT_M; ++i) {
            const uint64_t x = (s->mt[i] & upper) | (s->mt[i + 1] & lower);
            s->mt[i] = s->mt[i + MT_M] ^ (x >> 1) ^ mag[x & 1];
        }
        for (; i < MT_N - 1; ++i) {
            const uint64_t x = (s->mt[i] & upper) | (s->mt[i + 1] & lower);
            s->mt[i] = s->mt[i + (MT_M - MT_N)] ^ (x >> 1) ^ mag[x & 1];
        }
        const uint64_t x = (s->mt[MT_N - 1] & upper) | (s->mt[0] & lower);
        s->mt[MT_N - 1] = s->mt[MT_M - 1] ^ (x >> 1) ^ mag[x & 1];
        s->mti = 0;
    }
    uint64_t x = s->mt[s->mti++];
    x ^= (x >> 29) & 0x5555555555555555ULL;
    x ^= (x << 17) & 0x71D67FFFEDA60000ULL;
    x ^= (x << 37) & 0xFFF7EEE000000000ULL;
    x ^= x >> 43;
    return x;
}

/* uniform_real_distribution<double>(0, total): generate_canonical, then scaled. */
static double uniform(orc_sampler* s, double total) {
    double u = (double)mt_next(s) / 18446744073709551616.0;
    if (u >= 1.0) u = nextafter(1.0, 0.0);
    return u * (total - 0.0) + 0.0;
}

orc_sampler* orc_sampler_new(float temperature, int top_k, float top_p, uint64_t seed, float repetition_penalty,
                             float min_p, float frequency_penalty, float presence_penalty) {
    orc_sampler* s = (orc_sampler*)calloc(1, sizeof *s);
    s->temperature = temperature; s->top_k = top_k; s->top_p = top_p;
    s->repetition_penalty = repetition_penalty; s->min_p = min_p;
    s->frequency_penalty = frequency_penalty; s->presence_penalty = presence_penalty;
    mt_seed(s, seed);
    return s;
}

void orc_sampler_free(orc_sampler* s) {
    if (!s) return;
    free(s->picked_ids);
    free(s->picked_counts);
    free(s);
}

uint64_t orc_sampler_draw_u64(orc_sampler* s) { return mt_next(s); }
double orc_sampler_draw_uniform(orc_sampler* s, double total) { return uniform(s, total); }

static const float* g_sort_logits; /* qsort has no context argument */
static int by_logit(const void* a, const void* b) {
    const int32_t x = *(const int32_t*)a, y = *(const int32_t*)b;
    const float lx = g_sort_logits[x], ly = g_sort_logits[y];
    if (lx > ly) return -1;
    if (lx < ly) return 1;
    return x < y ? -1 : x > y;
}

/* Sampler::pick (sampling.cpp:76-139). */
static int32_t pick(orc_sampler* s, const float* logits, int64_t n) {
    int64_t best = 0;
    for (int64_t i = 1; i < n; ++i) if (logits[i] > logits[best]) best = i;
    if (s->temperature == 0.0f || s->top_k == 1) return (int32_t)best;
    const double top = logits[best], temp = s->temperature;
#define W(id) exp(((double)logits[(id)] - top) / temp)
    double everything = 0.0;
    if (s->top_k == 0) for (int64_t i = 0; i < n; ++i) everything += W(i);
    int32_t* order = (int32_t*)malloc(sizeof(int32_t) * (size_t)n);
    for (int64_t i = 0; i < n; ++i) order[i] = (int32_t)i;
    g_sort_logits = logits;
    qsort(order, (size_t)n, sizeof(int32_t), by_logit);
    const int grow = s->top_k == 0 && s->top_p < 1.0f;
    int64_t keep = s->top_k > 0 ? s->top_k : grow ? 256 : n;
    for (;;) {
        if (keep > n) keep = n;
        if (!grow || keep == n) break;
        double mass = 0.0;
        for (int64_t i = 0; i < keep; ++i) mass += W(order[i]);
        if (mass >= (double)s->top_p * everything) break;
        keep *= 4;
    }
    double* p = (double*)malloc(sizeof(double) * (size_t)(keep > 0 ? keep : 1));
    for (int64_t i = 0; i < keep; ++i) p[i] = W(order[i]);
    int64_t m = keep;
    double total = 0.0;
    if (s->top_k > 0) { for (int64_t i = 0; i < m; ++i) total += p[i]; }
    else total = everything;
    if (s->top_p < 1.0f) {
        double cumulative = 0.0;
        int64_t c = 0;
        while (c < m && cumulative < (double)s->top_p * total) cumulative += p[c++];
        m = c > 1 ? c : 1;
        total = 0.0;
        for (int64_t i = 0; i < m; ++i) total += p[i];
    }
    if (s->min_p > 0.0f) {
        int64_t c = 1;
        while (c < m && p[c] >= (double)s->min_p * p[0]) ++c;
        m = c;
        total = 0.0;
        for (int64_t i = 0; i < m; ++i) total += p[i];
    }
#undef W
    double draw = uniform(s, total);
    int32_t out = order[m - 1];
    for (int64_t i = 0; i < m; ++i) {
        draw -= p[i];
        if (draw < 0.0) { out = order[i]; break; }
    }
    free(order);
    free(p);
    return out;
}

/* Sampler::sample (sampling.cpp:46-74). */
int32_t orc_sampler_sample(orc_sampler* s, const float* given, int64_t n, const int32_t* previous, int64_t n_previous) {
    float* l = (float*)malloc(sizeof(float) * (size_t)n);
    memcpy(l, given, sizeof(float) * (size_t)n);
    if (s->repetition_penalty != 1.0f && n_previous > 0) {
        unsigned char* seen = (unsigned char*)calloc((size_t)n, 1);
        for (int64_t i = 0; i < n_previous; ++i) {
            const int32_t id = previous[i];
            if (id < 0 || id >= n || seen[id]) continue;
            seen[id] = 1;
            l[id] = l[id] < 0.0f ? l[id] * s->repetition_penalty : l[id] / s->repetition_penalty;
        }
        free(seen);
    }
    for (int64_t i = 0; i < s->picked_n; ++i) {
        const int32_t id = s->picked_ids[i];
        if (id < n) l[id] -= (float)s->picked_counts[i] * s->frequency_penalty + s->presence_penalty;
    }
    const int32_t id = pick(s, l, n);
    free(l);
    if (s->frequency_penalty != 0.0f || s->presence_penalty != 0.0f) {
        int64_t i = 0;
        while (i < s->picked_n && s->picked_ids[i] != id) ++i;
        if (i == s->picked_n) {
            if (s->picked_n == s->picked_cap) {
                s->picked_cap = s->picked_cap ? 2 * s->picked_cap : 16;
                s->picked_ids = (int32_t*)realloc(s->picked_ids, sizeof(int32_t) * (size_t)s->picked_cap);
                s->picked_counts = (int*)realloc(s->picked_counts, sizeof(int) * (size_t)s->picked_cap);
            }
            s->picked_ids[i] = id;
            s->picked_counts[i] = 0;
            ++s->picked_n;
        }
        ++s->picked_counts[i];
    }
    return id;
}

/* token_logprobs (src/io/sampling.cpp:141-164): token's log-softmax
 * probability, max + log(sum exp(l - max)) in double over the logits in
 * order, each result rounded to float; and the top most likely tokens with
 * theirs (equal logits by ascending id). */
float orc_token_logprobs(const float* logits, int64_t n, int32_t token, int top, int32_t* top_ids, float* top_logprobs) {
    double max = logits[0];
    for (int64_t i = 1; i < n; ++i) if (logits[i] > max) max = logits[i];
    double sum = 0.0;
    for (int64_t i = 0; i < n; ++i) sum += exp((double)logits[i] - max);
    const double log_total = max + log(sum);
    if (top > 0) {
        int32_t* order = (int32_t*)malloc(sizeof(int32_t) * (size_t)n);
        for (int64_t i = 0; i < n; ++i) order[i] = (int32_t)i;
        g_sort_logits = logits;
        qsort(order, (size_t)n, sizeof(int32_t), by_logit);
        for (int j = 0; j < top && j < n; ++j) {
            top_ids[j] = order[j];
            top_logprobs[j] = (float)((double)logits[order[j]] - log_total);
        }
        free(order);
    }
    return (float)((double)logits[token] - log_total);
}
