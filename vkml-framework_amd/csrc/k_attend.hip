// k_attend.hip -- decode attention over the KV cache (the reference's
// shaders/attend.comp + attend_merge.comp, src/ops/attention.cpp:54-84),
// written for gfx950.
//
// The reference gives each (128-key chunk, query head) its own workgroup, so
// with grouped-query attention every KV row is read once per query head of
// its group. Here workgroup (s, g) owns split s of KV head g's keys and
// computes all `group` query heads that share it, reading each K and V row
// once: a key's row is spread over LPK lanes with 16-byte loads (f16 head_dim
// 128: 16 lanes per key, 4 keys per wave64 per step), partial dot products
// are summed across those lanes with shuffles, scores go to LDS, each
// head's max and exp-sum come from wave reductions, and the weighted sum of
// V reuses the same lane mapping. The merge combines the splits with the
// online-softmax rescaling e^(m_s - M) and can quantize the result to Q8_0
// for the o projection in the same pass.
#include <algorithm>

#include "device.hpp"
#include "internal.hpp"

using namespace vkml::dev;

namespace {

constexpr int kThreads = 256;
constexpr uint32_t kMaxChunk = 1024;  // keys per split (LDS: group * chunk floats)

template <int HD, bool F16>
struct Layout {
    static constexpr int kElemBytes = F16 ? 2 : 4;
    static constexpr int kPerLane = 16 / kElemBytes;         // elements per 16-byte load
    static constexpr int kLanesPerKey = HD * kElemBytes / 16;  // 4 .. 64
    static constexpr int kKeysPerWave = kWave / kLanesPerKey;
    static constexpr int kKeysPerStep = kKeysPerWave * (kThreads / kWave);
};

template <bool F16, int N>
__device__ __forceinline__ void load_row(const void* base, uint64_t elem, float (&out)[N]) {
    const uint4 v = *reinterpret_cast<const uint4*>(static_cast<const uint8_t*>(base) + elem * (F16 ? 2 : 4));
    if constexpr (F16) {
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            out[2 * i] = f16_bits_to_float(w[i] & 0xFFFFu);
            out[2 * i + 1] = f16_bits_to_float(w[i] >> 16);
        }
    } else {
        out[0] = __uint_as_float(v.x); out[1] = __uint_as_float(v.y);
        out[2] = __uint_as_float(v.z); out[3] = __uint_as_float(v.w);
    }
}

struct AttendArgs {
    const float* q;
    const void* k;
    const void* v;
    float* partial;
    float* stats;
    const vkml_decode_state* state;
    uint32_t kv_start, kv_len, capacity, splits;
    float scale, softcap;
};

template <int HD, int G, bool F16>
__global__ void __launch_bounds__(kThreads) k_attend(AttendArgs a) {
    using L = Layout<HD, F16>;
    constexpr int EPL = L::kPerLane, LPK = L::kLanesPerKey, KPW = L::kKeysPerWave, KPS = L::kKeysPerStep;
    // Scores and weights [G][kMaxChunk]; after the V pass, the per-wave sums
    // [waves][G][HD] reuse the same memory (HD <= 256 keeps them inside).
    __shared__ float s_buf[G * kMaxChunk];
    static_assert((kThreads / kWave) * HD <= kMaxChunk, "reduction space");
    float (*s_p)[kMaxChunk] = reinterpret_cast<float (*)[kMaxChunk]>(s_buf);
    float (*s_red)[G][HD] = reinterpret_cast<float (*)[G][HD]>(s_buf);
    const uint32_t split = blockIdx.x, g = blockIdx.y;
    const uint32_t wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const uint32_t sub = lane % LPK, key_in_step = wave * KPW + lane / LPK;

    const uint32_t kv_len = a.state ? static_cast<uint32_t>(a.state->position) + 1u : a.kv_len;
    const uint32_t total = kv_len > a.kv_start ? kv_len - a.kv_start : 0u;
    const uint32_t chunk = (total + a.splits - 1) / a.splits;
    const uint32_t k0 = a.kv_start + split * chunk;
    const uint32_t n = k0 < kv_len ? min(chunk, kv_len - k0) : 0u;
    const uint64_t row_base = static_cast<uint64_t>(g) * a.capacity;

    // This lane's slice of each head's query.
    float q[G][EPL];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        const float* qh = a.q + (static_cast<uint64_t>(g) * G + h) * HD + sub * EPL;
#pragma unroll
        for (int e = 0; e < EPL; ++e) q[h][e] = qh[e];
    }

    // Scores.
    for (uint32_t i = 0; i < n; i += KPS) {
        const uint32_t key = i + key_in_step;
        float part[G];
#pragma unroll
        for (int h = 0; h < G; ++h) part[h] = 0.0f;
        if (key < n) {
            float kf[EPL];
            load_row<F16>(a.k, (row_base + (k0 + key) % a.capacity) * HD + sub * EPL, kf);
#pragma unroll
            for (int h = 0; h < G; ++h)
#pragma unroll
                for (int e = 0; e < EPL; ++e) part[h] += q[h][e] * kf[e];
        }
#pragma unroll
        for (int h = 0; h < G; ++h) {
            float s = group_sum<LPK>(part[h]) * a.scale;
            if (a.softcap > 0.0f) s = a.softcap * tanhf(fminf(fmaxf(s / a.softcap, -10.0f), 10.0f));
            if (key < n && sub == 0) s_p[h][key] = s;
        }
    }
    __syncthreads();

    // Per head: max score and the weights e^(s - m), summed.
    __shared__ float s_m[G], s_l[G];
    for (int h = wave; h < G; h += kThreads / kWave) {
        float m = -__builtin_inff();
        for (uint32_t k = lane; k < n; k += kWave) m = fmaxf(m, s_p[h][k]);
        m = wave_max(m);
        float l = 0.0f;
        for (uint32_t k = lane; k < n; k += kWave) {
            const float p = expf(s_p[h][k] - m);
            s_p[h][k] = p;
            l += p;
        }
        l = wave_sum(l);
        if (lane == 0) {
            s_m[h] = m;
            s_l[h] = l;
        }
    }
    __syncthreads();

    // Weighted sum of V.
    float acc[G][EPL];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[h][e] = 0.0f;
    for (uint32_t i = 0; i < n; i += KPS) {
        const uint32_t key = i + key_in_step;
        if (key < n) {
            float vf[EPL];
            load_row<F16>(a.v, (row_base + (k0 + key) % a.capacity) * HD + sub * EPL, vf);
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const float p = s_p[h][key];
#pragma unroll
                for (int e = 0; e < EPL; ++e) acc[h][e] += p * vf[e];
            }
        }
    }
    // Sum the keys of this wave (lanes sub, sub + LPK, ...), then the waves.
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            float v = acc[h][e];
#pragma unroll
            for (int o = LPK; o < kWave; o <<= 1) v += __shfl_xor(v, o, kWave);
            acc[h][e] = v;
        }
    __syncthreads();  // every wave is done reading the weights in s_buf
    if (lane < LPK) {
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int e = 0; e < EPL; ++e) s_red[wave][h][sub * EPL + e] = acc[h][e];
    }
    __syncthreads();
    const uint64_t out_base = (static_cast<uint64_t>(g) * a.splits + split) * G;
    for (uint32_t i = threadIdx.x; i < G * HD; i += kThreads) {
        const uint32_t h = i / HD, d = i % HD;
        float s = 0.0f;
#pragma unroll
        for (int w = 0; w < kThreads / kWave; ++w) s += s_red[w][h][d];
        a.partial[(out_base + h) * HD + d] = s;
    }
    if (threadIdx.x < G) {
        a.stats[(out_base + threadIdx.x) * 2] = s_m[threadIdx.x];
        a.stats[(out_base + threadIdx.x) * 2 + 1] = s_l[threadIdx.x];
    }
}

// One block per query head, head_dim threads.
__global__ void k_attend_merge(const float* partial, const float* stats, float* out, uint8_t* values, float* scales,
                               uint32_t splits, uint32_t group, uint32_t hd) {
    const uint32_t h = blockIdx.x, d = threadIdx.x;
    const uint32_t g = h / group, hh = h % group;
    float top = -__builtin_inff();
    for (uint32_t s = 0; s < splits; ++s) top = fmaxf(top, stats[((static_cast<uint64_t>(g) * splits + s) * group + hh) * 2]);
    float sum = 0.0f, weight = 0.0f;
    for (uint32_t s = 0; s < splits; ++s) {
        const uint64_t at = (static_cast<uint64_t>(g) * splits + s) * group + hh;
        const float m = stats[at * 2];
        if (m == -__builtin_inff()) continue;  // an empty split
        const float r = expf(m - top);
        sum += r * partial[at * hd + d];
        weight += r * stats[at * 2 + 1];
    }
    const float o = sum / weight;
    out[static_cast<uint64_t>(h) * hd + d] = o;
    if (values) {
        // Q8_0 with f32 scales over 32-value blocks (quantize.comp:210-221).
        const float absmax = group_max<32>(fabsf(o));
        const float ds = absmax / 127.0f;
        const float inv = ds > 0.0f ? 1.0f / ds : 0.0f;
        values[static_cast<uint64_t>(h) * hd + d] = static_cast<uint8_t>(static_cast<int8_t>(quant_code(o, inv)));
        if (d % 32 == 0) scales[(static_cast<uint64_t>(h) * hd + d) / 32] = ds;
    }
}

template <int HD, bool F16>
int launch_group(uint32_t group, dim3 grid, const AttendArgs& args) {
    hipStream_t s = vkml::abi::stream();
    switch (group) {
        case 1: hipLaunchKernelGGL((k_attend<HD, 1, F16>), grid, dim3(kThreads), 0, s, args); break;
        case 2: hipLaunchKernelGGL((k_attend<HD, 2, F16>), grid, dim3(kThreads), 0, s, args); break;
        case 4: hipLaunchKernelGGL((k_attend<HD, 4, F16>), grid, dim3(kThreads), 0, s, args); break;
        case 8: hipLaunchKernelGGL((k_attend<HD, 8, F16>), grid, dim3(kThreads), 0, s, args); break;
        default: return vkml::abi::fail(VKML_ERROR_UNSUPPORTED, "attend: query heads per KV head must be 1, 2, 4 or 8");
    }
    return VKML_OK;
}

}  // namespace

extern "C" {

int vkml_attend(const vkml_attend_params* p, const float* q, const void* k_cache, const void* v_cache,
                float* partial, float* stats, const vkml_decode_state* state) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(p, "attend: null params");
    VKML_CHECK_ARG(p->kv_heads > 0 && p->heads % p->kv_heads == 0,
                   "attend: q's " + std::to_string(p->heads) + " heads must be a multiple of k and v's " + std::to_string(p->kv_heads));
    VKML_CHECK_ARG(p->head_dim == 64 || p->head_dim == 128 || p->head_dim == 256,
                   "attend: head_dim " + std::to_string(p->head_dim) + " is not 64, 128 or 256");
    VKML_CHECK_ARG(p->kv_type == VKML_F16 || p->kv_type == VKML_F32, "attend: caches must be f16 or f32");
    VKML_CHECK_ARG(p->splits > 0 && p->capacity > 0, "attend: splits and capacity must be positive");
    VKML_CHECK_ARG(state || (p->kv_len <= p->capacity && p->kv_start < p->kv_len),
                   "attend: keys " + std::to_string(p->kv_start) + ".." + std::to_string(p->kv_len) + " do not fit the cache");
    // Every split must fit LDS: splits * kMaxChunk covers the longest range.
    VKML_CHECK_ARG(static_cast<uint64_t>(p->splits) * kMaxChunk >= (state ? p->capacity : p->kv_len - p->kv_start),
                   "attend: " + std::to_string(p->splits) + " splits leave more than " + std::to_string(kMaxChunk) + " keys per split");
    VKML_CHECK_ARG(q && k_cache && v_cache && partial && stats, "attend: null buffer");
    AttendArgs args{q, k_cache, v_cache, partial, stats, state, p->kv_start, p->kv_len, p->capacity, p->splits, p->scale, p->softcap};
    const dim3 grid(p->splits, p->kv_heads);
    const uint32_t group = p->heads / p->kv_heads;
    const bool f16 = p->kv_type == VKML_F16;
    vkml::abi::ProfileScope prof("attend");
    int r;
    switch (p->head_dim) {
        case 64: r = f16 ? launch_group<64, true>(group, grid, args) : launch_group<64, false>(group, grid, args); break;
        case 128: r = f16 ? launch_group<128, true>(group, grid, args) : launch_group<128, false>(group, grid, args); break;
        default: r = f16 ? launch_group<256, true>(group, grid, args) : launch_group<256, false>(group, grid, args); break;
    }
    if (r != VKML_OK) return r;
    return vkml::abi::check_launch("attend");
}

int vkml_attend_merge(const vkml_attend_params* p, const float* partial, const float* stats, float* out, void* values,
                      float* scales) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(p && partial && stats && out, "attend_merge: null argument");
    VKML_CHECK_ARG(p->kv_heads > 0 && p->heads % p->kv_heads == 0 && p->head_dim % 32 == 0 && p->head_dim <= 1024,
                   "attend_merge: bad head layout");
    VKML_CHECK_ARG(!values || scales, "attend_merge: quantized output needs scales");
    vkml::abi::ProfileScope prof("attend_merge");
    hipLaunchKernelGGL(k_attend_merge, dim3(p->heads), dim3(p->head_dim), 0, vkml::abi::stream(), partial, stats, out,
                       static_cast<uint8_t*>(values), scales, p->splits, p->heads / p->kv_heads, p->head_dim);
    return vkml::abi::check_launch("attend_merge");
}

}  // extern "C"
