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
// Mapping. Workgroup (chunk, KV head, query head) as the reference's
// (chunk, head), but numbered so that the query heads sharing a KV head run
// on the same XCD one after another (the dispatcher deals workgroups to the
// 8 XCDs round-robin): the K and V rows come from HBM once and from that
// XCD's L2 for the other heads. A decode step gives several workgroups per
// CU, so one's loads overlap another's arithmetic. Every load of a chunk is
// issued before any is used: K into registers (four lanes a key, as the
// reference splits it), V into LDS. The decode-step entry point also rotates
// q and the new key (RoPE) and appends the new key and value to the caches,
// the work of rope + cast + write_rows in llama.cpp:320-355: the workgroup
// whose chunk holds the new position computes them itself (its staged copy of
// that cache row predates the append). Chunks past the live keys (the grid
// covers the whole cache, so a replayed graph serves every position) record
// a max of -inf, which the merge skips. The merge is its own launch, every
// load of a head's chunks issued at once, and can quantize its output to
// Q8_0 for the o projection.
#include <algorithm>
#include <type_traits>

#include "device.hpp"
#include "internal.hpp"

using namespace vkml::dev;

namespace {

constexpr int kThreads = 256;
constexpr uint32_t kChunk = 128;  // attend.comp's CHUNK = WG
constexpr int kLanes = 4;        // lanes per key while scoring
constexpr uint32_t kXcds = 8;    // workgroups are dealt to the XCDs round-robin

struct ChunkArgs {
    const float* q;      // [heads, hd] (plain) or the token's [q | k | v] (step)
    const float* table;  // step: RoPE cos/sin pairs [positions, hd / 2, 2]
    void* k_cache;
    void* v_cache;
    float* partial;
    float* stats;
    const vkml_decode_state* state;
    uint32_t heads, kv_heads, group, capacity, kv_start, kv_len, position, chunks;
    uint32_t step, style, rotate;
    float scale, softcap;
};

// Four elements of a cache row, as stored (four f16, or four f32), and widened exactly.
template <bool F16>
using KRaw = std::conditional_t<F16, uint2, float4>;

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

__device__ __forceinline__ uint32_t cache_bits(float v, bool f16) {
    return f16 ? f32_to_f16_bits(__float_as_uint(v)) : __float_as_uint(v);
}

// RoPE of the pair (x[ia], x[ib]) with cos/sin (c, s) (rope.comp:94-118 in the
// arithmetic of vkml_rope_kv_append).
__device__ __forceinline__ void rotate_pair(float& x, float& y, float c, float s) {
#pragma clang fp contract(off)
    const float rx = x * c - y * s, ry = x * s + y * c;
    x = rx;
    y = ry;
}

// HPW query heads (of one KV head) per workgroup: 2 when the group allows,
// sharing the K registers and the V tile.
template <int HD, bool F16, int HPW>
__global__ void __launch_bounds__(kThreads) k_attend_chunk(ChunkArgs a) {
#pragma clang fp contract(off)
    constexpr uint32_t EB = F16 ? 2 : 4;
    constexpr uint32_t RB = HD * EB;               // bytes per cache row
    constexpr bool kStageV = RB <= 512;            // V tile in LDS (up to 64 KiB)
    constexpr uint32_t kVLoads = kStageV ? RB * kChunk / 16 / kThreads : 1;
    constexpr uint32_t K4 = HD / 4;                // vec4s per row
    constexpr uint32_t KPL = K4 / kLanes;          // vec4s per lane per key
    constexpr uint32_t kSlots = kThreads / kLanes; // keys per scoring pass
    constexpr uint32_t kPasses = kChunk / kSlots;
    __shared__ float s_q[HPW][HD];
    __shared__ uint32_t s_knew[HD], s_vnew[HD];    // the new key and value, as cache bits
    __shared__ __align__(16) uint8_t s_v[kStageV ? kChunk * RB : 16];
    __shared__ __align__(16) float s_p[HPW][kChunk];
    __shared__ float s_red[HPW][kChunk];
    __shared__ float s_m[HPW], s_l[HPW];

    // Workgroup number -> (chunk, KV head, head group): the head groups of a
    // (chunk, KV head) pair get numbers 8 apart, so the same XCD.
    const uint32_t G = a.group, groups = G / HPW, pairs = a.chunks * a.kv_heads;
    const uint32_t L = blockIdx.x, pair_lo = L % kXcds, rest = L / kXcds;
    const uint32_t hl = rest % groups, pair = (rest / groups) * kXcds + pair_lo;
    if (pair >= pairs) return;
    const uint32_t chunk = pair / a.kv_heads, kvh = pair % a.kv_heads, head0 = kvh * G + hl * HPW;
    const uint32_t t = threadIdx.x;
    const uint32_t pos = a.step ? (a.state ? static_cast<uint32_t>(a.state->position) : a.position) : 0u;
    const uint32_t kv_len = a.step ? pos + 1 : (a.state ? static_cast<uint32_t>(a.state->position) + 1u : a.kv_len);
    const uint32_t key0 = a.kv_start + chunk * kChunk;
    const auto stats_at = [&](uint32_t h) -> uint64_t { return static_cast<uint64_t>(head0 + h) * a.chunks + chunk; };
    if (key0 >= kv_len) {
        if (t < HPW) {
            a.stats[stats_at(t) * 2] = -__builtin_inff();
            a.stats[stats_at(t) * 2 + 1] = 0.0f;
        }
        return;
    }
    const uint32_t n = min(kChunk, kv_len - key0);
    const bool holds_new = a.step && key0 + n == kv_len;  // the appended key is this chunk's last
    const uint64_t kv_row0 = static_cast<uint64_t>(kvh) * a.capacity;
    const auto row_of = [&](uint32_t key) -> uint64_t { return kv_row0 + (key0 + key) % a.capacity; };

    // Issue every load of the chunk: K for both scoring passes (lane g of a
    // key's four takes vec4s g, g + 4, ...), and the V tile straight into LDS
    // (the compiler issues every load before the first store waits). Keys
    // past n re-read key n - 1.
    const uint32_t lane4 = t % kLanes, slot = t / kLanes;
    KRaw<F16> kreg[kPasses][KPL];
#pragma unroll
    for (uint32_t p = 0; p < kPasses; ++p) {
        const uint64_t row = row_of(min(p * kSlots + slot, n - 1)) * HD;
#pragma unroll
        for (uint32_t j = 0; j < KPL; ++j) {
            const uint32_t i = lane4 + kLanes * j;
            if constexpr (F16) kreg[p][j] = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(a.k_cache) + row + 4 * i);
            else kreg[p][j] = *reinterpret_cast<const float4*>(static_cast<const float*>(a.k_cache) + row + 4 * i);
        }
    }
    if constexpr (kStageV) {
#pragma unroll
        for (uint32_t j = 0; j < kVLoads; ++j) {
            const uint32_t u = t + j * kThreads, key = min(u / (RB / 16), n - 1), col = u % (RB / 16);
            reinterpret_cast<uint4*>(s_v)[u] =
                *reinterpret_cast<const uint4*>(static_cast<const uint8_t*>(a.v_cache) + row_of(key) * RB + 16ull * col);
        }
    }

    // The queries (rotated in a step), and in the chunk holding it the new
    // key and value, rounded to the cache type and appended by head group
    // 0's workgroup.
    const uint32_t half = HD / 2;
    if (a.step) {
        const float* tab = a.table + static_cast<uint64_t>(pos) * half * 2;
        const float* ksrc = a.q + static_cast<uint64_t>(a.heads) * HD + static_cast<uint64_t>(kvh) * HD;
        const float* vsrc = a.q + static_cast<uint64_t>(a.heads + a.kv_heads) * HD + static_cast<uint64_t>(kvh) * HD;
        const uint64_t new_row = (kv_row0 + pos % a.capacity) * HD;
        for (uint32_t i = t; i < (HPW + 1) * half; i += kThreads) {
            const uint32_t h = i / half, k = i % half;  // h == HPW: the new key
            const uint32_t ia = a.style == 0 ? 2 * k : k, ib = a.style == 0 ? 2 * k + 1 : k + half;
            const float c = tab[2 * k], sn = tab[2 * k + 1];
            if (h < HPW) {
                const float* qsrc = a.q + static_cast<uint64_t>(head0 + h) * HD;
                float qx = qsrc[ia], qy = qsrc[ib];
                if (a.rotate) rotate_pair(qx, qy, c, sn);
                s_q[h][ia] = qx;
                s_q[h][ib] = qy;
            } else if (holds_new) {
                float kx = ksrc[ia], ky = ksrc[ib];
                if (a.rotate) rotate_pair(kx, ky, c, sn);
                const uint32_t kb[2] = {cache_bits(kx, F16), cache_bits(ky, F16)};
                const uint32_t vb[2] = {cache_bits(vsrc[ia], F16), cache_bits(vsrc[ib], F16)};
                const uint32_t el[2] = {ia, ib};
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    s_knew[el[e]] = kb[e];
                    s_vnew[el[e]] = vb[e];
                    if (hl == 0) {
                        if constexpr (F16) {
                            static_cast<uint16_t*>(a.k_cache)[new_row + el[e]] = static_cast<uint16_t>(kb[e]);
                            static_cast<uint16_t*>(a.v_cache)[new_row + el[e]] = static_cast<uint16_t>(vb[e]);
                        } else {
                            static_cast<uint32_t*>(a.k_cache)[new_row + el[e]] = kb[e];
                            static_cast<uint32_t*>(a.v_cache)[new_row + el[e]] = vb[e];
                        }
                    }
                }
            }
        }
    } else {
        for (uint32_t i = t; i < HPW * HD; i += kThreads) s_q[i / HD][i % HD] = a.q[static_cast<uint64_t>(head0) * HD + i];
    }
    __syncthreads();
    if (kStageV && holds_new) {
        for (uint32_t i = t; i < HD; i += kThreads) {
            if constexpr (F16) reinterpret_cast<uint16_t*>(s_v)[(n - 1) * HD + i] = static_cast<uint16_t>(s_vnew[i]);
            else reinterpret_cast<uint32_t*>(s_v)[(n - 1) * HD + i] = s_vnew[i];
        }
    }

    // Scores: part g of each head, then ((0 + p0) + p1) + p2) + p3.
    float4 qr[HPW][KPL];
#pragma unroll
    for (int h = 0; h < HPW; ++h)
#pragma unroll
        for (uint32_t j = 0; j < KPL; ++j) {
            const uint32_t i = lane4 + kLanes * j;
            qr[h][j] = make_float4(s_q[h][4 * i], s_q[h][4 * i + 1], s_q[h][4 * i + 2], s_q[h][4 * i + 3]);
        }
#pragma unroll
    for (uint32_t p = 0; p < kPasses; ++p) {
        const uint32_t key = p * kSlots + slot;
        const bool fresh = holds_new && key == n - 1;
        float part[HPW];
#pragma unroll
        for (int h = 0; h < HPW; ++h) part[h] = 0.0f;
#pragma unroll
        for (uint32_t j = 0; j < KPL; ++j) {
            float4 kv = widen(kreg[p][j]);
            if (fresh) {
                const uint32_t i = lane4 + kLanes * j;
                if constexpr (F16) kv = widen(make_uint2(s_knew[4 * i] | (s_knew[4 * i + 1] << 16), s_knew[4 * i + 2] | (s_knew[4 * i + 3] << 16)));
                else kv = make_float4(__uint_as_float(s_knew[4 * i]), __uint_as_float(s_knew[4 * i + 1]),
                                      __uint_as_float(s_knew[4 * i + 2]), __uint_as_float(s_knew[4 * i + 3]));
            }
#pragma unroll
            for (int h = 0; h < HPW; ++h) part[h] += dot4f(qr[h][j], kv);
        }
#pragma unroll
        for (int h = 0; h < HPW; ++h) {
            const float p1 = __shfl_down(part[h], 1, kWave), p2 = __shfl_down(part[h], 2, kWave), p3 = __shfl_down(part[h], 3, kWave);
            if (lane4 == 0 && key < n) {
                const float sc = (0.0f + part[h] + p1 + p2 + p3) * a.scale;
                s_p[h][key] = a.softcap > 0.0f ? a.softcap * tanhf(fminf(fmaxf(sc / a.softcap, -10.0f), 10.0f)) : sc;
            }
        }
    }
    __syncthreads();

    // Per head (a wave each): max, weights and their halving-tree sum.
    const uint32_t wave = t / kWave, lane = t % kWave;
    if (wave < HPW) {
        const uint32_t h = wave;
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

    // V: chain (head, element d, slice sl) over the slice's keys in order. A
    // thread carries two neighbouring elements (one 32-bit V read a key) and
    // reads the weights four keys at a time; 32 keys' reads are in flight
    // together, and whole chunks need no per-key guard.
    constexpr uint32_t slices = HD >= kChunk ? 1 : kChunk / HD;
    constexpr uint32_t NP = HD / 2;  // element pairs
    constexpr uint32_t KB = 32;      // keys of a slice per batch
    const auto v_pair = [&](uint32_t key, uint32_t dp, float& x, float& y) {
        if constexpr (kStageV) {
            if constexpr (F16) {
                const uint32_t w = reinterpret_cast<const uint32_t*>(s_v)[key * NP + dp];
                x = f16_bits_to_float(w & 0xFFFFu);
                y = f16_bits_to_float(w >> 16);
            } else {
                const float2 w = reinterpret_cast<const float2*>(s_v)[key * NP + dp];
                x = w.x;
                y = w.y;
            }
        } else {
            if (holds_new && key == n - 1) {
                x = F16 ? f16_bits_to_float(s_vnew[2 * dp]) : __uint_as_float(s_vnew[2 * dp]);
                y = F16 ? f16_bits_to_float(s_vnew[2 * dp + 1]) : __uint_as_float(s_vnew[2 * dp + 1]);
            } else if constexpr (F16) {
                const uint32_t w = static_cast<const uint32_t*>(a.v_cache)[(row_of(key) * HD) / 2 + dp];
                x = f16_bits_to_float(w & 0xFFFFu);
                y = f16_bits_to_float(w >> 16);
            } else {
                const float2 w = static_cast<const float2*>(a.v_cache)[(row_of(key) * HD) / 2 + dp];
                x = w.x;
                y = w.y;
            }
        }
    };
    for (uint32_t c = t; c < HPW * slices * NP; c += kThreads) {
        const uint32_t dp = c % NP, sl = (c / NP) % slices, h = c / (NP * slices);
        const uint32_t keys = n > sl ? (n - sl + slices - 1) / slices : 0;  // this slice's keys: sl, sl + slices, ...
        float o0 = 0.0f, o1 = 0.0f;
        for (uint32_t j0 = 0; j0 < keys; j0 += KB) {
            float w[KB], x[KB], y[KB];
            const float4* wp = reinterpret_cast<const float4*>(&s_p[h][slices * j0]);
#pragma unroll
            for (uint32_t m = 0; m < KB * slices / 4; ++m) {
                const float4 q = wp[m];
                if constexpr (slices == 1) {
                    w[4 * m] = q.x; w[4 * m + 1] = q.y; w[4 * m + 2] = q.z; w[4 * m + 3] = q.w;
                } else {
                    w[2 * m] = sl ? q.y : q.x;
                    w[2 * m + 1] = sl ? q.w : q.z;
                }
            }
#pragma unroll
            for (uint32_t jj = 0; jj < KB; ++jj) v_pair(min(sl + slices * (j0 + jj), n - 1), dp, x[jj], y[jj]);
            if (j0 + KB <= keys) {
#pragma unroll
                for (uint32_t jj = 0; jj < KB; ++jj) {
                    o0 += w[jj] * x[jj];
                    o1 += w[jj] * y[jj];
                }
            } else {
#pragma unroll
                for (uint32_t jj = 0; jj < KB; ++jj) {
                    if (j0 + jj < keys) {
                        o0 += w[jj] * x[jj];
                        o1 += w[jj] * y[jj];
                    }
                }
            }
        }
        if constexpr (HD > kChunk) {
            // heads wider than the reference's workgroup: no slice sum
            a.partial[stats_at(h) * HD + 2 * dp] = o0;
            a.partial[stats_at(h) * HD + 2 * dp + 1] = o1;
        } else {
            s_red[h][sl * HD + 2 * dp] = o0;
            s_red[h][sl * HD + 2 * dp + 1] = o1;
        }
    }
    if constexpr (HD <= kChunk) {
        __syncthreads();
        for (uint32_t i = t; i < HPW * HD; i += kThreads) {
            const uint32_t h = i / HD, d = i % HD;
            float sum = 0.0f;
#pragma unroll
            for (uint32_t sl = 0; sl < slices; ++sl) sum += s_red[h][sl * HD + d];
            a.partial[stats_at(h) * HD + d] = sum;
        }
    }
    if (t < HPW) {
        a.stats[stats_at(t) * 2] = s_m[t];
        a.stats[stats_at(t) * 2 + 1] = s_l[t];
    }
}

// attend_merge.comp:25-38 for head blockIdx.x, element threadIdx.x; chunks
// with a max of -inf hold no keys and are skipped. Every invocation of the
// reference computes the same max M and the same factors exp(m_c - M) and
// weight sum; here each is computed once per head (the factors by one thread
// per chunk, in parallel) and shared through LDS, which leaves each element
// its chain sum += r_c * partial_c. Its partials are loaded 64 chunks at a
// time with every load in flight. Optionally quantizes the result to Q8_0
// with f32 scales (quantize.comp:100-111), the o projection's input.
constexpr uint32_t kMergeMaxChunks = 1024;  // 131072 keys

__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
k_attend_merge(const float* partial, const float* stats, float* out, uint8_t* values, float* scales, uint32_t chunks, uint32_t hd) {
#pragma clang fp contract(off)
    constexpr uint32_t B = 64;
    __shared__ float s_r[kMergeMaxChunks];   // exp(m_c - M), or -1 for a chunk past the live keys
    __shared__ float s_l[kMergeMaxChunks];   // the chunk's sum of weights
    __shared__ float s_wmax[8];
    const uint32_t h = blockIdx.x, d = threadIdx.x, nt = blockDim.x;
    const uint64_t first = static_cast<uint64_t>(h) * chunks;
    const float2* st = reinterpret_cast<const float2*>(stats) + first;
    const float* pc = partial + first * hd + d;
    float p[B];
#pragma unroll
    for (uint32_t j = 0; j < B; ++j) p[j] = pc[static_cast<uint64_t>(min(j, chunks - 1)) * hd];
    // M = max over the chunks' maxima (exact in any order).
    float m = -__builtin_inff();
    for (uint32_t c = d; c < chunks; c += nt) m = fmaxf(m, st[c].x);
    m = wave_max(m);
    if (d % kWave == 0) s_wmax[d / kWave] = m;
    __syncthreads();
    float top = s_wmax[0];
    for (uint32_t w = 1; w < (nt + kWave - 1) / kWave; ++w) top = fmaxf(top, s_wmax[w]);
    for (uint32_t c = d; c < chunks; c += nt) {
        const float2 ml = st[c];
        s_r[c] = ml.x == -__builtin_inff() ? -1.0f : vk_expf(ml.x - top);
        s_l[c] = ml.y;
    }
    __syncthreads();
    // sum += r_c * partial_c and weight += r_c * l_c over the live chunks in
    // order (every thread carries the weight chain too: the same value).
    float sum = 0.0f, weight = 0.0f;
    for (uint32_t c0 = 0; c0 < chunks; c0 += B) {
        if (c0 > 0) {
#pragma unroll
            for (uint32_t j = 0; j < B; ++j) p[j] = pc[static_cast<uint64_t>(min(c0 + j, chunks - 1)) * hd];
        }
        float r[B], l[B];
#pragma unroll
        for (uint32_t j = 0; j < B; ++j) {
            r[j] = s_r[min(c0 + j, chunks - 1)];
            l[j] = s_l[min(c0 + j, chunks - 1)];
        }
#pragma unroll
        for (uint32_t j = 0; j < B; ++j) {
            if (c0 + j < chunks && r[j] >= 0.0f) {
                sum += r[j] * p[j];
                weight += r[j] * l[j];
            }
        }
    }
    const float o = sum / weight;
    out[static_cast<uint64_t>(h) * hd + d] = o;
    if (values) {
        const float absmax = group_max<32>(fabsf(o));
        const float ds = absmax / 127.0f;
        const float inv = ds > 0.0f ? 1.0f / ds : 0.0f;
        values[static_cast<uint64_t>(h) * hd + d] = static_cast<uint8_t>(static_cast<int8_t>(quant_code(o, inv)));
        if (d % 32 == 0) scales[(static_cast<uint64_t>(h) * hd + d) / 32] = ds;
    }
}

template <int HD, bool F16>
void launch_hd(const ChunkArgs& args, uint32_t pair_blocks) {
    hipStream_t s = vkml::abi::stream();
    if (args.group % 2 == 0) {
        const dim3 grid(pair_blocks * kXcds * (args.group / 2));
        hipLaunchKernelGGL((k_attend_chunk<HD, F16, 2>), grid, dim3(kThreads), 0, s, args);
    } else {
        const dim3 grid(pair_blocks * kXcds * args.group);
        hipLaunchKernelGGL((k_attend_chunk<HD, F16, 1>), grid, dim3(kThreads), 0, s, args);
    }
}

int launch_chunks(uint32_t head_dim, bool f16, const ChunkArgs& args) {
    const uint32_t pair_blocks = (args.chunks * args.kv_heads + kXcds - 1) / kXcds;
    switch (head_dim) {
        case 64: f16 ? launch_hd<64, true>(args, pair_blocks) : launch_hd<64, false>(args, pair_blocks); break;
        case 128: f16 ? launch_hd<128, true>(args, pair_blocks) : launch_hd<128, false>(args, pair_blocks); break;
        default: f16 ? launch_hd<256, true>(args, pair_blocks) : launch_hd<256, false>(args, pair_blocks); break;
    }
    return VKML_OK;
}

int launch_merge(uint32_t heads, uint32_t head_dim, uint32_t chunks, const float* partial, const float* stats, float* out,
                 void* values, float* scales) {
    hipLaunchKernelGGL(k_attend_merge, dim3(heads), dim3(head_dim), 0, vkml::abi::stream(), partial, stats, out,
                       static_cast<uint8_t*>(values), scales, chunks, head_dim);
    return VKML_OK;
}

int check_heads(uint32_t heads, uint32_t kv_heads, uint32_t head_dim, const char* what) {
    VKML_CHECK_ARG(kv_heads > 0 && heads % kv_heads == 0,
                   std::string(what) + ": q's " + std::to_string(heads) + " heads must be a multiple of k and v's " + std::to_string(kv_heads));
    VKML_CHECK_ARG(head_dim == 64 || head_dim == 128 || head_dim == 256,
                   std::string(what) + ": head_dim " + std::to_string(head_dim) + " is not 64, 128 or 256");
    return VKML_OK;
}

}  // namespace

extern "C" {

int vkml_attend(const vkml_attend_params* p, const float* q, const void* k_cache, const void* v_cache,
                float* partial, float* stats, const vkml_decode_state* state) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(p, "attend: null params");
    if (int r = check_heads(p->heads, p->kv_heads, p->head_dim, "attend")) return r;
    VKML_CHECK_ARG(p->kv_type == VKML_F16 || p->kv_type == VKML_F32, "attend: caches must be f16 or f32");
    VKML_CHECK_ARG(p->chunks > 0 && p->capacity > 0 && p->kv_start < p->capacity, "attend: chunks and capacity must be positive, kv_start inside the cache");
    VKML_CHECK_ARG(state || (p->kv_len <= p->capacity && p->kv_start < p->kv_len),
                   "attend: keys " + std::to_string(p->kv_start) + ".." + std::to_string(p->kv_len) + " do not fit the cache");
    // With a decode state, kv_len can reach the capacity: cover every chunk of it.
    const uint64_t keys = state ? p->capacity - p->kv_start : p->kv_len - p->kv_start;
    VKML_CHECK_ARG(static_cast<uint64_t>(p->chunks) * kChunk >= keys,
                   "attend: " + std::to_string(p->chunks) + " chunks of " + std::to_string(kChunk) + " keys do not cover " +
                       std::to_string(keys) + " keys");
    VKML_CHECK_ARG(q && k_cache && v_cache && partial && stats, "attend: null buffer");
    ChunkArgs args{q, nullptr, const_cast<void*>(k_cache), const_cast<void*>(v_cache), partial, stats, state,
                   p->heads, p->kv_heads, p->heads / p->kv_heads, p->capacity, p->kv_start, p->kv_len, 0, p->chunks,
                   0, 0, 0, p->scale, p->softcap};
    vkml::abi::ProfileScope prof("attend");
    launch_chunks(p->head_dim, p->kv_type == VKML_F16, args);
    return vkml::abi::check_launch("attend");
}

int vkml_attend_merge(const vkml_attend_params* p, const float* partial, const float* stats, float* out, void* values,
                      float* scales) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(p, "attend_merge: null params");
    if (int r = check_heads(p->heads, p->kv_heads, p->head_dim, "attend_merge")) return r;
    VKML_CHECK_ARG(p->chunks > 0 && p->chunks <= kMergeMaxChunks,
                   "attend_merge: chunks must be 1 to " + std::to_string(kMergeMaxChunks));
    VKML_CHECK_ARG(partial && stats && out, "attend_merge: null buffer");
    VKML_CHECK_ARG(!values || scales, "attend_merge: quantized output needs scales");
    vkml::abi::ProfileScope prof("attend_merge");
    launch_merge(p->heads, p->head_dim, p->chunks, partial, stats, out, values, scales);
    return vkml::abi::check_launch("attend_merge");
}

int vkml_attend_step(const vkml_attend_step_params* p, const float* qkv, const float* rope_table, void* k_cache, void* v_cache,
                     float* partial, float* stats, float* out, void* values, float* scales, const vkml_decode_state* state) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(p, "attend_step: null params");
    if (int r = check_heads(p->heads, p->kv_heads, p->head_dim, "attend_step")) return r;
    VKML_CHECK_ARG(p->kv_type == VKML_F16 || p->kv_type == VKML_F32, "attend_step: caches must be f16 or f32");
    VKML_CHECK_ARG(p->capacity > 0 && p->kv_start < p->capacity, "attend_step: kv_start must lie inside the cache");
    VKML_CHECK_ARG(state || (p->position < p->capacity && p->kv_start <= p->position),
                   "attend_step: position " + std::to_string(p->position) + " is outside the cache");
    VKML_CHECK_ARG(static_cast<uint64_t>(p->chunks) * kChunk >= p->capacity - p->kv_start && p->chunks <= kMergeMaxChunks,
                   "attend_step: " + std::to_string(p->chunks) + " chunks do not cover the cache (or exceed " +
                       std::to_string(kMergeMaxChunks) + ")");
    VKML_CHECK_ARG(qkv && rope_table && k_cache && v_cache && partial && stats && out, "attend_step: null buffer");
    VKML_CHECK_ARG(!values || scales, "attend_step: quantized output needs scales");
    ChunkArgs args{qkv, rope_table, k_cache, v_cache, partial, stats, state, p->heads, p->kv_heads, p->heads / p->kv_heads,
                   p->capacity, p->kv_start, 0, p->position, p->chunks, 1, p->rope_style, p->rotate, p->scale, p->softcap};
    {
        vkml::abi::ProfileScope prof("attend_step");
        launch_chunks(p->head_dim, p->kv_type == VKML_F16, args);
        if (int r = vkml::abi::check_launch("attend_step")) return r;
    }
    vkml::abi::ProfileScope prof("attend_merge");
    launch_merge(p->heads, p->head_dim, p->chunks, partial, stats, out, values, scales);
    return vkml::abi::check_launch("attend_merge");
}

}  // extern "C"
