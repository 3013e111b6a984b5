// k_attend.hip -- decode attention over the KV cache (the reference's
// shaders/attend.comp + attend_merge.comp, src/ops/attention.cpp:54-84),
// written for gfx950.
//
// Bit-exact by construction: keys are taken in the reference's chunks of 128
// from kv_start, and every f32 value follows its order: each score sums four
// partial dot products (vec4s i = g, g + 4, ... for part g) in turn
// (attend.comp:97-116), the chunk's weight sum is the halving tree over 128
// (:130-137), each output element sums weight * v over the chunk's keys in
// key order, in head_dim-wide slices for heads narrower than 128 (:140-167),
// and the merge walks the chunks in order (attend_merge.comp:30-38). exp is
// vk_expf, which the CPU oracle shares.
//
// What changes is the mapping onto the machine. The reference gives each
// (chunk, query head) a workgroup, so with grouped-query attention each K and
// V row is read once per query head of its group; here workgroup (chunk, KV
// head) computes all `group` query heads that share the KV head, reading each
// row once. The chunk's V rows are loaded into registers while the scores are
// computed and parked in LDS (rows up to 256 bytes), so the V pass waits on
// no memory. Chunks past the live keys (the grid is sized by the cache, so a
// replayed graph covers every position) write a max of -inf, which the merge
// skips.
#include <algorithm>
#include <type_traits>

#include "device.hpp"
#include "internal.hpp"

using namespace vkml::dev;

namespace {

constexpr int kThreads = 256;
constexpr uint32_t kChunk = 128;  // attend.comp's CHUNK = WG
constexpr int kLanes = 4;        // invocations per key while scoring

struct AttendArgs {
    const float* q;
    const void* k;
    const void* v;
    float* partial;
    float* stats;
    const vkml_decode_state* state;
    uint32_t kv_start, kv_len, capacity, chunks;
    float scale, softcap;
};

// Four elements of a K row from vec4 index i, as stored (four f16, or four
// f32), and widened exactly.
template <bool F16>
using KRaw = std::conditional_t<F16, uint2, float4>;

template <bool F16>
__device__ __forceinline__ KRaw<F16> load_k4(const void* base, uint64_t row_elem, uint32_t i) {
    if constexpr (F16) return *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(base) + row_elem + 4 * i);
    else return *reinterpret_cast<const float4*>(static_cast<const float*>(base) + row_elem + 4 * i);
}
__device__ __forceinline__ float4 widen(uint2 w) {
    return make_float4(f16_bits_to_float(w.x & 0xFFFFu), f16_bits_to_float(w.x >> 16),
                       f16_bits_to_float(w.y & 0xFFFFu), f16_bits_to_float(w.y >> 16));
}
__device__ __forceinline__ float4 widen(float4 w) { return w; }

// dot(a, b) as ((a.x b.x + a.y b.y) + a.z b.z) + a.w b.w.
__device__ __forceinline__ float dot4f(float4 a, float4 b) {
#pragma clang fp contract(off)
    return a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
}

template <int HD, int G, bool F16>
__global__ void __launch_bounds__(kThreads) k_attend(AttendArgs a) {
#pragma clang fp contract(off)
    constexpr uint32_t EB = F16 ? 2 : 4;
    constexpr uint32_t RB = HD * EB;                   // bytes per cache row
    constexpr bool kStageV = RB <= 256;                // the chunk's V rows fit 32 KiB of LDS
    constexpr uint32_t kVLoads = kStageV ? RB * kChunk / 16 / kThreads : 1;  // 16-byte loads per thread
    constexpr uint32_t K4 = HD / 4;                    // vec4s per row
    constexpr uint32_t KPL = K4 / kLanes;              // vec4s per lane per key
    constexpr uint32_t kSlots = kThreads / kLanes;     // keys per scoring pass
    constexpr uint32_t kPasses = kChunk / kSlots;

    __shared__ float4 s_q[G][K4];
    __shared__ float s_p[G][kChunk];      // scores, then weights
    __shared__ float s_red[G][kChunk];    // per-slice sums of the V pass
    __shared__ uint4 s_v[kStageV ? RB * kChunk / 16 : 1];
    __shared__ float s_m[G], s_l[G];

    const uint32_t chunk = blockIdx.x, g = blockIdx.y, t = threadIdx.x;
    const uint32_t kv_len = a.state ? static_cast<uint32_t>(a.state->position) + 1u : a.kv_len;
    const uint32_t key0 = a.kv_start + chunk * kChunk;
    const uint64_t head0 = static_cast<uint64_t>(g) * G;
    if (key0 >= kv_len) {
        // Past the live keys: nothing for the merge to take.
        if (t < G) {
            a.stats[((head0 + t) * a.chunks + chunk) * 2] = -__builtin_inff();
            a.stats[((head0 + t) * a.chunks + chunk) * 2 + 1] = 0.0f;
        }
        return;
    }
    const uint32_t n = min(kChunk, kv_len - key0);
    const uint64_t kv_row0 = static_cast<uint64_t>(g) * a.capacity;
    const auto row_elem = [&](uint32_t key) -> uint64_t { return (kv_row0 + (key0 + key) % a.capacity) * HD; };

    // Issue this thread's V loads first; they land while the scores are computed.
    uint4 vreg[kVLoads];
    if constexpr (kStageV) {
#pragma unroll
        for (uint32_t j = 0; j < kVLoads; ++j) {
            const uint32_t u = t + j * kThreads, key = u / (RB / 16), col = u % (RB / 16);
            vreg[j] = key < n ? *reinterpret_cast<const uint4*>(static_cast<const uint8_t*>(a.v) + row_elem(key) * EB + 16 * col)
                              : make_uint4(0, 0, 0, 0);
        }
    }
    // K: lane g of each key's four takes vec4s g, g + 4, ... of the row.
    const uint32_t lane4 = t % kLanes, slot = t / kLanes;
    KRaw<F16> kreg[kPasses][KPL];
#pragma unroll
    for (uint32_t pass = 0; pass < kPasses; ++pass) {
        const uint32_t key = pass * kSlots + slot;
#pragma unroll
        for (uint32_t j = 0; j < KPL; ++j) kreg[pass][j] = key < n ? load_k4<F16>(a.k, row_elem(key), lane4 + kLanes * j) : KRaw<F16>{};
    }
    for (uint32_t i = t; i < G * K4; i += kThreads) {
        const float* qh = a.q + (head0 + i / K4) * HD + 4 * (i % K4);
        s_q[i / K4][i % K4] = make_float4(qh[0], qh[1], qh[2], qh[3]);
    }
    __syncthreads();

    // Scores: part g, then ((0 + part0) + part1) + part2) + part3 in the key's first lane.
#pragma unroll
    for (uint32_t pass = 0; pass < kPasses; ++pass) {
        const uint32_t key = pass * kSlots + slot;
#pragma unroll
        for (int h = 0; h < G; ++h) {
            float part = 0.0f;
#pragma unroll
            for (uint32_t j = 0; j < KPL; ++j) part += dot4f(s_q[h][lane4 + kLanes * j], widen(kreg[pass][j]));
            const float p1 = __shfl_down(part, 1, kWave), p2 = __shfl_down(part, 2, kWave), p3 = __shfl_down(part, 3, kWave);
            if (lane4 == 0 && key < n) {
                const float dot_qk = 0.0f + part + p1 + p2 + p3;
                const float s = dot_qk * a.scale;
                s_p[h][key] = a.softcap > 0.0f ? a.softcap * tanhf(fminf(fmaxf(s / a.softcap, -10.0f), 10.0f)) : s;
            }
        }
    }
    if constexpr (kStageV) {
#pragma unroll
        for (uint32_t j = 0; j < kVLoads; ++j) s_v[t + j * kThreads] = vreg[j];
    }
    __syncthreads();

    // Per head (a wave each): the max, each key's weight, and their sum by the
    // halving tree: lane k first adds keys k and k + 64, then strides 32 .. 1.
    const uint32_t wave = t / kWave, lane = t % kWave;
    for (int h = wave; h < G; h += kThreads / kWave) {
        const float s0 = lane < n ? s_p[h][lane] : -__builtin_inff();
        const float s1 = lane + 64 < n ? s_p[h][lane + 64] : -__builtin_inff();
        const float m = wave_max(fmaxf(s0, s1));
        const float w0 = lane < n ? vk_expf(s0 - m) : 0.0f;
        const float w1 = lane + 64 < n ? vk_expf(s1 - m) : 0.0f;
        s_p[h][lane] = w0;
        s_p[h][lane + 64] = w1;
        float l = w0 + w1;
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) l += __shfl_xor(l, o, kWave);
        if (lane == 0) {
            s_m[h] = m;
            s_l[h] = l;
        }
    }
    __syncthreads();

    const auto v_at = [&](uint32_t key, uint32_t d) -> float {
        if constexpr (kStageV) {
            if constexpr (F16) return f16_bits_to_float(reinterpret_cast<const uint16_t*>(s_v)[key * HD + d]);
            else return reinterpret_cast<const float*>(s_v)[key * HD + d];
        } else {
            if constexpr (F16) return f16_bits_to_float(static_cast<const uint16_t*>(a.v)[row_elem(key) + d]);
            else return static_cast<const float*>(a.v)[row_elem(key) + d];
        }
    };
    const uint64_t out0 = head0 * a.chunks + chunk;  // (head0, chunk) in [heads, chunks]
    if constexpr (HD > kChunk) {
        // Heads wider than the workgroup of 128: element d over every key.
        for (uint32_t d = t; d < HD; d += kThreads) {
            float o[G];
#pragma unroll
            for (int h = 0; h < G; ++h) o[h] = 0.0f;
            for (uint32_t key = 0; key < n; ++key) {
                const float v = v_at(key, d);
#pragma unroll
                for (int h = 0; h < G; ++h) o[h] += s_p[h][key] * v;
            }
#pragma unroll
            for (int h = 0; h < G; ++h) a.partial[(out0 + static_cast<uint64_t>(h) * a.chunks) * HD + d] = o[h];
        }
    } else {
        // 128 / HD slices; slice i takes keys i, i + slices, ...; thread t
        // computes slot t % 128 for heads t / 128, t / 128 + 2, ...
        constexpr uint32_t slices = kChunk / HD;
        const uint32_t c = t % kChunk, d = c % HD, sl = c / HD;
        constexpr int HPT = G >= 2 ? G / 2 : 1;
        const int h0 = static_cast<int>(t / kChunk);
        if (G >= 2 || h0 == 0) {
            float o[HPT];
#pragma unroll
            for (int j = 0; j < HPT; ++j) o[j] = 0.0f;
            for (uint32_t key = sl; key < n; key += slices) {
                const float v = v_at(key, d);
#pragma unroll
                for (int j = 0; j < HPT; ++j) o[j] += s_p[h0 + 2 * j][key] * v;
            }
#pragma unroll
            for (int j = 0; j < HPT; ++j) s_red[h0 + 2 * j][c] = o[j];
        }
        __syncthreads();
        for (uint32_t i = t; i < G * HD; i += kThreads) {
            const uint32_t h = i / HD, e = i % HD;
            float sum = 0.0f;
#pragma unroll
            for (uint32_t s = 0; s < slices; ++s) sum += s_red[h][s * HD + e];
            a.partial[(out0 + static_cast<uint64_t>(h) * a.chunks) * HD + e] = sum;
        }
    }
    if (t < G) {
        a.stats[(out0 + static_cast<uint64_t>(t) * a.chunks) * 2] = s_m[t];
        a.stats[(out0 + static_cast<uint64_t>(t) * a.chunks) * 2 + 1] = s_l[t];
    }
}

// attend_merge.comp:25-38 for head blockIdx.x, element threadIdx.x; chunks
// with a max of -inf hold no keys and are skipped. Optionally quantizes the
// result to Q8_0 with f32 scales (quantize.comp:210-221), the o projection's
// input.
__global__ void k_attend_merge(const float* partial, const float* stats, float* out, uint8_t* values, float* scales,
                               uint32_t chunks, uint32_t hd) {
#pragma clang fp contract(off)
    const uint32_t h = blockIdx.x, d = threadIdx.x;
    const uint64_t first = static_cast<uint64_t>(h) * chunks;
    float top = stats[first * 2];
    for (uint32_t c = 1; c < chunks; ++c) top = fmaxf(top, stats[(first + c) * 2]);
    float sum = 0.0f, weight = 0.0f;
    for (uint32_t c = 0; c < chunks; ++c) {
        const float m = stats[(first + c) * 2];
        if (m == -__builtin_inff()) continue;
        const float r = vk_expf(m - top);
        sum += r * partial[(first + c) * hd + d];
        weight += r * stats[(first + c) * 2 + 1];
    }
    const float o = sum / weight;
    out[static_cast<uint64_t>(h) * hd + d] = o;
    if (values) {
        const float absmax = group_max<32>(fabsf(o));
        const float ds = absmax / 127.0f;
        const float inv = ds != 0.0f ? 1.0f / ds : 0.0f;
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

int check_layout(const vkml_attend_params* p, const char* what) {
    VKML_CHECK_ARG(p, std::string(what) + ": null params");
    VKML_CHECK_ARG(p->kv_heads > 0 && p->heads % p->kv_heads == 0,
                   std::string(what) + ": q's " + std::to_string(p->heads) + " heads must be a multiple of k and v's " +
                       std::to_string(p->kv_heads));
    VKML_CHECK_ARG(p->head_dim == 64 || p->head_dim == 128 || p->head_dim == 256,
                   std::string(what) + ": head_dim " + std::to_string(p->head_dim) + " is not 64, 128 or 256");
    VKML_CHECK_ARG(p->chunks > 0, std::string(what) + ": chunks must be positive");
    return VKML_OK;
}

}  // namespace

extern "C" {

int vkml_attend(const vkml_attend_params* p, const float* q, const void* k_cache, const void* v_cache,
                float* partial, float* stats, const vkml_decode_state* state) {
    VKML_REQUIRE_INIT();
    if (int r = check_layout(p, "attend")) return r;
    VKML_CHECK_ARG(p->kv_type == VKML_F16 || p->kv_type == VKML_F32, "attend: caches must be f16 or f32");
    VKML_CHECK_ARG(p->capacity > 0 && p->kv_start < p->capacity, "attend: kv_start must lie inside the cache");
    VKML_CHECK_ARG(state || (p->kv_len <= p->capacity && p->kv_start < p->kv_len),
                   "attend: keys " + std::to_string(p->kv_start) + ".." + std::to_string(p->kv_len) + " do not fit the cache");
    // With a decode state, kv_len can reach the capacity: cover every chunk of it.
    const uint64_t keys = state ? p->capacity - p->kv_start : p->kv_len - p->kv_start;
    VKML_CHECK_ARG(static_cast<uint64_t>(p->chunks) * kChunk >= keys,
                   "attend: " + std::to_string(p->chunks) + " chunks of " + std::to_string(kChunk) + " keys do not cover " +
                       std::to_string(keys) + " keys");
    VKML_CHECK_ARG(q && k_cache && v_cache && partial && stats, "attend: null buffer");
    AttendArgs args{q, k_cache, v_cache, partial, stats, state, p->kv_start, p->kv_len, p->capacity, p->chunks, p->scale, p->softcap};
    const dim3 grid(p->chunks, p->kv_heads);
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
    if (int r = check_layout(p, "attend_merge")) return r;
    VKML_CHECK_ARG(partial && stats && out, "attend_merge: null buffer");
    VKML_CHECK_ARG(!values || scales, "attend_merge: quantized output needs scales");
    vkml::abi::ProfileScope prof("attend_merge");
    hipLaunchKernelGGL(k_attend_merge, dim3(p->heads), dim3(p->head_dim), 0, vkml::abi::stream(), partial, stats, out,
                       static_cast<uint8_t*>(values), scales, p->chunks, p->head_dim);
    return vkml::abi::check_launch("attend_merge");
}

}  // extern "C"
