// attend.hpp -- decode attention's device code (the reference's
// shaders/attend.comp + attend_merge.comp, src/ops/attention.cpp:54-84),
// used by the attention kernels (k_attend.hip).
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
// Within a chunk item every load is issued before any is used: K into
// registers (four lanes a key, as the reference splits it), V into
// registers and, once the scores are done, LDS. In a
// decode step the item also rotates q and the new key (RoPE) and appends the
// new key and value to the caches, the work of rope + cast + write_rows in
// llama.cpp:320-355: the item whose chunk holds the new position computes
// them itself (its staged copy of that cache row predates the append).
#pragma once

#include <type_traits>

#include "../../include/vkml_hip.h"
#include "device.hpp"

namespace vkml::attend {

using namespace vkml::dev;

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
    // When non-null: the sync words of the merge + o launch that follows
    // (OSync), whose counter and flags workgroup 0 zeroes.
    uint32_t* o_sync;
    // A sliding window (0: none): keys from max(kv_start, kv_len - window).
    uint32_t window;
    // A step whose q was rotated and whose new key and value were appended
    // by the q|k|v GEMV before (vkml_gemv_rope): q is read as it is and the
    // caches as they are.
    uint32_t prepared;
    // Chunks live at every position the launch may see (a hint): the one
    // launch's items of these issue their q, K and V loads before reading
    // the position (prepared steps without a window).
    uint32_t ready;
    // When non-null: the sticky error flag the chunk pass sets to 2 when the
    // position lies past the keys of its chunks (a launch sized for fewer
    // chunks than the cache holds), as the one-launch form does.
    uint32_t* error;
};

// Sync words of the launch that merges the chunks and runs the o GEMV on
// the result (one 256-byte line each): [0] a sticky error flag, then kCopies
// copies of the merge workgroups' arrival counter (each merging workgroup
// adds to every copy; a GEMV workgroup polls copy wg % kCopies, so no one
// line serves every poll).
struct OSync {
    static constexpr uint32_t kLine = 64;
    static constexpr uint32_t kCopies = 16;
    static constexpr uint32_t kWords = kLine * (1 + kCopies);
    __device__ static uint32_t* error(uint32_t* s) { return s; }
    __device__ static uint32_t* counter(uint32_t* s, uint32_t i) { return s + kLine * (1 + i); }
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

// The same with b four f16 values (two per word), each product as
// fma(a, b, nz) with nz = -0: exact products rounded once, as a * b, where
// the f16 operand is widened inside v_fma_mix_f32 (nz comes from an asm, so
// the fma is not folded back into a multiply).
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float dot4h(float4 a, uint2 b, float nz) {
#pragma clang fp contract(off)
    const half2_t lo = __builtin_bit_cast(half2_t, b.x), hi = __builtin_bit_cast(half2_t, b.y);
    return __builtin_fmaf(a.x, static_cast<float>(lo.x), nz) + __builtin_fmaf(a.y, static_cast<float>(lo.y), nz) +
           __builtin_fmaf(a.z, static_cast<float>(hi.x), nz) + __builtin_fmaf(a.w, static_cast<float>(hi.y), nz);
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

// LDS of one chunk item.
template <int HD, bool F16, int HPW>
struct AttendSmem {
    static constexpr uint32_t kRowBytes = HD * (F16 ? 2 : 4);
    static constexpr bool kStageV = kRowBytes <= 512;  // V tile in LDS (up to 64 KiB); as ChunkShape
    float q[HPW][HD];
    uint32_t knew[HD], vnew[HD];  // the new key and value, as cache bits
    alignas(16) uint8_t v[kStageV ? kChunk * kRowBytes : 16];
    alignas(16) float p[HPW][kChunk];
    float red[HPW][kChunk];
    float m[HPW], l[HPW];
};

// Shapes of a chunk item's loads.
template <int HD, bool F16>
struct ChunkShape {
    static constexpr uint32_t kRowBytes = HD * (F16 ? 2 : 4);
    static constexpr bool kStageV = kRowBytes <= 512;                         // V tile in LDS
    static constexpr uint32_t kVLoads = kStageV ? kRowBytes * kChunk / 16 / kThreads : 1;  // 16-byte V loads a thread
    static constexpr uint32_t KPL = HD / 4 / kLanes;                          // vec4s per lane per key
    static constexpr uint32_t kSlots = kThreads / kLanes;                     // keys per scoring pass
    static constexpr uint32_t kPasses = kChunk / kSlots;
};

// A chunk's K rows in registers (lane g of a key's four holds vec4s g, g +
// 4, ...), and, when it is staged, its V tile copied straight into LDS by
// the memory unit (global_load_lds: no registers, nothing to store
// afterwards): every load of the chunk, issued at once. Keys past the live
// ones re-read the last live key.
template <int HD, bool F16>
struct ChunkLoads {
    using S = ChunkShape<HD, F16>;
    KRaw<F16> k[S::kPasses][S::KPL];
};

typedef __attribute__((address_space(3))) void lds_void;

// 16 bytes at src into LDS: lane l of the wave writes lds_wave + 16 l
// (lds_wave the same for the whole wave).
__device__ __forceinline__ void load_to_lds16(const void* src, void* lds_wave) {
    __builtin_amdgcn_global_load_lds(src, (lds_void*)lds_wave, 16, 0, 0);
}

template <int HD, bool F16>
__device__ __forceinline__ void attend_chunk_load(const ChunkArgs& a, uint32_t chunk, uint32_t kvh, uint32_t kv_len,
                                                  ChunkLoads<HD, F16>& r, uint8_t* v_lds) {
    using S = ChunkShape<HD, F16>;
    constexpr uint32_t RB = S::kRowBytes;
    const uint32_t t = thread_index();
    const uint32_t key0 = a.kv_start + chunk * kChunk;
    const uint32_t n = min(kChunk, kv_len - key0);
    const uint64_t kv_row0 = static_cast<uint64_t>(kvh) * a.capacity;
    const auto row_of = [&](uint32_t key) -> uint64_t { return kv_row0 + (key0 + key) % a.capacity; };
    const uint32_t lane4 = t % kLanes, slot = t / kLanes;
#pragma unroll
    for (uint32_t p = 0; p < S::kPasses; ++p) {
        const uint64_t row = row_of(min(p * S::kSlots + slot, n - 1)) * HD;
#pragma unroll
        for (uint32_t j = 0; j < S::KPL; ++j) {
            const uint32_t i = lane4 + kLanes * j;
            if constexpr (F16) r.k[p][j] = ldg(reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(a.k_cache) + row + 4 * i));
            else r.k[p][j] = ldg(reinterpret_cast<const float4*>(static_cast<const float*>(a.k_cache) + row + 4 * i));
        }
    }
    if constexpr (S::kStageV) {
        // the tile row-major, as the cache rows: piece u = t + j * kThreads
        // (16 bytes) of the tile at byte 16 u, lane by lane within a wave
        const uint32_t wave_first = t - t % kWave;
#pragma unroll
        for (uint32_t j = 0; j < S::kVLoads; ++j) {
            const uint32_t u = t + j * kThreads, key = min(u / (RB / 16), n - 1), col = u % (RB / 16);
            load_to_lds16(static_cast<const uint8_t*>(a.v_cache) + row_of(key) * RB + 16ull * col, v_lds + 16 * (j * kThreads + wave_first));
        }
    }
}

// The item's query operands, loaded by attend_q_load: in a step, per
// rotation item (a query pair, or the new key's pair with its value pair)
// the pair and its cos/sin; otherwise q itself. Loaded before the item's K
// and V where q is ready by then, so that waiting for them does not wait
// for K and V.
template <int HD, int HPW>
struct QLoads {
    static constexpr uint32_t kRot = (HPW + 1) * HD / 2;  // rotation items: HPW heads' pairs, then the new key's
    static constexpr uint32_t kItems = ((kRot > HPW * HD ? kRot : HPW * HD) + kThreads - 1) / kThreads;
    float x[kItems], y[kItems], c[kItems], s[kItems], vx[kItems], vy[kItems];
};

template <int HD, int HPW>
__device__ __forceinline__ void attend_q_load(const ChunkArgs& a, uint32_t kvh, uint32_t hl, uint32_t pos, QLoads<HD, HPW>& r) {
    using Q = QLoads<HD, HPW>;
    const uint32_t t = thread_index(), head0 = kvh * a.group + hl * HPW, half = HD / 2;
    if (a.step && !a.prepared) {
        const float* tab = a.table + static_cast<uint64_t>(pos) * half * 2;
        const float* ksrc = a.q + static_cast<uint64_t>(a.heads) * HD + static_cast<uint64_t>(kvh) * HD;
        const float* vsrc = a.q + static_cast<uint64_t>(a.heads + a.kv_heads) * HD + static_cast<uint64_t>(kvh) * HD;
#pragma unroll
        for (uint32_t u = 0; u < Q::kItems; ++u) {
            const uint32_t i = min(t + u * kThreads, static_cast<uint32_t>(Q::kRot - 1));
            const uint32_t h = i / half, k = i % half;  // h == HPW: the new key
            const uint32_t ia = a.style == 0 ? 2 * k : k, ib = a.style == 0 ? 2 * k + 1 : k + half;
            const float* src = h < HPW ? a.q + static_cast<uint64_t>(head0 + h) * HD : ksrc;
            r.c[u] = ldg(tab + 2 * k);
            r.s[u] = ldg(tab + 2 * k + 1);
            r.x[u] = ldg(src + ia);
            r.y[u] = ldg(src + ib);
            r.vx[u] = ldg(vsrc + ia);
            r.vy[u] = ldg(vsrc + ib);
        }
    } else {
#pragma unroll
        for (uint32_t u = 0; u < Q::kItems; ++u)
            r.x[u] = ldg(a.q + static_cast<uint64_t>(head0) * HD + min(t + u * kThreads, static_cast<uint32_t>(HPW * HD - 1)));
    }
}

// One (chunk, KV head, head group hl) item of the chunk pass, for a chunk
// holding live keys (key0 < kv_len), given its loads: scores, softmax and V over its keys,
// writing the HPW heads' partials and (max, weight sum); in a step, RoPE of
// q and of the new key and the append of the new key and value. HPW query
// heads (of one KV head) share the K registers and the V tile. With COH, the
// partials and stats are stored write-through, coherently across XCDs, for
// a merge in another workgroup of the same launch. KB: keys of a slice whose
// weights and values the V pass holds in registers at once.
template <int HD, bool F16, int HPW, bool COH, uint32_t KB = 32>
__device__ __forceinline__ void attend_chunk_item(const ChunkArgs& a, uint32_t chunk, uint32_t kvh, uint32_t hl, uint32_t pos,
                                                  uint32_t kv_len, const QLoads<HD, HPW>& qv, const ChunkLoads<HD, F16>& ld,
                                                  AttendSmem<HD, F16, HPW>& sm) {
#pragma clang fp contract(off)
    using S = ChunkShape<HD, F16>;
    constexpr bool kStageV = S::kStageV;
    constexpr uint32_t KPL = S::KPL;
    constexpr uint32_t kSlots = S::kSlots;
    constexpr uint32_t kPasses = S::kPasses;
    const uint32_t G = a.group, head0 = kvh * G + hl * HPW;
    const uint32_t t = thread_index();
    const uint32_t key0 = a.kv_start + chunk * kChunk;
    const auto stats_at = [&](uint32_t h) -> uint64_t { return static_cast<uint64_t>(head0 + h) * a.chunks + chunk; };
    const uint32_t n = min(kChunk, kv_len - key0);
    const bool rot = a.step && !a.prepared;            // rotate q and append the new key and value here
    const bool holds_new = rot && key0 + n == kv_len;  // the appended key is this chunk's last
    const uint64_t kv_row0 = static_cast<uint64_t>(kvh) * a.capacity;
    const auto row_of = [&](uint32_t key) -> uint64_t { return kv_row0 + (key0 + key) % a.capacity; };

    const uint32_t lane4 = t % kLanes, slot = t / kLanes;
    // The queries (rotated in a step), and in the chunk holding it the new
    // key and value, rounded to the cache type and appended by head group
    // 0's workgroup.
    const uint32_t half = HD / 2;
    using Q = QLoads<HD, HPW>;
    if (rot) {
        const uint64_t new_row = (kv_row0 + pos % a.capacity) * HD;
#pragma unroll
        for (uint32_t u = 0; u < Q::kItems; ++u) {
            const uint32_t i = t + u * kThreads;
            if (i >= Q::kRot) break;
            const uint32_t h = i / half, k = i % half;  // h == HPW: the new key
            const uint32_t ia = a.style == 0 ? 2 * k : k, ib = a.style == 0 ? 2 * k + 1 : k + half;
            const float c = qv.c[u], sn = qv.s[u];
            if (h < HPW) {
                float qx = qv.x[u], qy = qv.y[u];
                if (a.rotate) rotate_pair(qx, qy, c, sn);
                sm.q[h][ia] = qx;
                sm.q[h][ib] = qy;
            } else if (holds_new) {
                float kx = qv.x[u], ky = qv.y[u];
                if (a.rotate) rotate_pair(kx, ky, c, sn);
                const uint32_t kb[2] = {cache_bits(kx, F16), cache_bits(ky, F16)};
                const uint32_t vb[2] = {cache_bits(qv.vx[u], F16), cache_bits(qv.vy[u], F16)};
                const uint32_t el[2] = {ia, ib};
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    sm.knew[el[e]] = kb[e];
                    sm.vnew[el[e]] = vb[e];
                    if (hl == 0) {
                        if constexpr (F16) {
                            stg(static_cast<uint16_t*>(a.k_cache) + new_row + el[e], static_cast<uint16_t>(kb[e]));
                            stg(static_cast<uint16_t*>(a.v_cache) + new_row + el[e], static_cast<uint16_t>(vb[e]));
                        } else {
                            stg(static_cast<uint32_t*>(a.k_cache) + new_row + el[e], kb[e]);
                            stg(static_cast<uint32_t*>(a.v_cache) + new_row + el[e], vb[e]);
                        }
                    }
                }
            }
        }
    } else {
#pragma unroll
        for (uint32_t u = 0; u < Q::kItems; ++u) {
            const uint32_t i = t + u * kThreads;
            if (i < HPW * HD) sm.q[i / HD][i % HD] = qv.x[u];
        }
    }
    __syncthreads();

    // -0 for the products of f32 and f16 values taken as fma(a, b, -0) (dot4h)
    float nz = -0.0f;
    asm volatile("" : "+v"(nz));
    // Scores: part g of each head, then ((0 + p0) + p1) + p2) + p3; HB heads
    // a pass (their q in registers) over the K registers. Two a pass at two
    // heads a workgroup; at four, one a pass keeps the chunk pass at 106
    // VGPRs (four workgroups a CU instead of three at 137), and every
    // product is then one v_fma_mix_f32 rather than a widening shared by
    // two heads and two fmas.
    constexpr int HB = HPW == 2 ? 2 : 1;
    // K as loaded, except that in the chunk holding the appended key its
    // row takes the new key's bits (its copy in the cache may predate the
    // append): one patch here, branch-free scores below.
    KRaw<F16> kr[kPasses][KPL];
#pragma unroll
    for (uint32_t p = 0; p < kPasses; ++p)
#pragma unroll
        for (uint32_t j = 0; j < KPL; ++j) kr[p][j] = ld.k[p][j];
    if (holds_new) {
#pragma unroll
        for (uint32_t p = 0; p < kPasses; ++p) {
            if (p * kSlots + slot != n - 1) continue;
#pragma unroll
            for (uint32_t j = 0; j < KPL; ++j) {
                const uint32_t i = lane4 + kLanes * j;
                if constexpr (F16) kr[p][j] = make_uint2(sm.knew[4 * i] | (sm.knew[4 * i + 1] << 16), sm.knew[4 * i + 2] | (sm.knew[4 * i + 3] << 16));
                else kr[p][j] = make_float4(__uint_as_float(sm.knew[4 * i]), __uint_as_float(sm.knew[4 * i + 1]),
                                            __uint_as_float(sm.knew[4 * i + 2]), __uint_as_float(sm.knew[4 * i + 3]));
            }
        }
    }
#pragma unroll
    for (int hb = 0; hb < HPW; hb += HB) {
        float4 qr[HB][KPL];
#pragma unroll
        for (int h = 0; h < HB; ++h)
#pragma unroll
            for (uint32_t j = 0; j < KPL; ++j) {
                const uint32_t i = lane4 + kLanes * j;
                qr[h][j] = make_float4(sm.q[hb + h][4 * i], sm.q[hb + h][4 * i + 1], sm.q[hb + h][4 * i + 2], sm.q[hb + h][4 * i + 3]);
            }
#pragma unroll
        for (uint32_t p = 0; p < kPasses; ++p) {
            const uint32_t key = p * kSlots + slot;
            float part[HB];
#pragma unroll
            for (int h = 0; h < HB; ++h) part[h] = 0.0f;
#pragma unroll
            for (uint32_t j = 0; j < KPL; ++j) {
                const KRaw<F16> kw = kr[p][j];
#pragma unroll
                for (int h = 0; h < HB; ++h) {
                    if constexpr (F16) part[h] += dot4h(qr[h][j], kw, nz);
                    else part[h] += dot4f(qr[h][j], kw);
                }
            }
#pragma unroll
            for (int h = 0; h < HB; ++h) {
                const float p1 = dpp_f<dpp::shl(1)>(part[h]), p2 = dpp_f<dpp::shl(2)>(part[h]), p3 = dpp_f<dpp::shl(3)>(part[h]);
                if (lane4 == 0 && key < n) {
                    const float sc = (0.0f + part[h] + p1 + p2 + p3) * a.scale;
                    sm.p[hb + h][key] = a.softcap > 0.0f ? a.softcap * tanhf(fminf(fmaxf(sc / a.softcap, -10.0f), 10.0f)) : sc;
                }
            }
        }
    }
    // The V tile's copies into LDS (issued last, after the K loads the
    // scores waited for) have landed once the wave's loads are all done.
    if constexpr (kStageV) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (kStageV && holds_new) {
        for (uint32_t i = t; i < HD; i += kThreads) {
            if constexpr (F16) reinterpret_cast<uint16_t*>(sm.v)[(n - 1) * HD + i] = static_cast<uint16_t>(sm.vnew[i]);
            else reinterpret_cast<uint32_t*>(sm.v)[(n - 1) * HD + i] = sm.vnew[i];
        }
    }

    // Per head (a wave each): max, weights and their halving-tree sum.
    const uint32_t wave = t / kWave, lane = t % kWave;
    if (wave < HPW) {
        const uint32_t h = wave;
        const float s0 = lane < n ? sm.p[h][lane] : -__builtin_inff();
        const float s1 = lane + 64 < n ? sm.p[h][lane + 64] : -__builtin_inff();
        const float m = wave_max(fmaxf(s0, s1));
        const float w0 = lane < n ? vk_expf(s0 - m) : 0.0f;
        const float w1 = lane + 64 < n ? vk_expf(s1 - m) : 0.0f;
        sm.p[h][lane] = w0;
        sm.p[h][lane + 64] = w1;
        const float l = tree_to_first<64>(w0 + w1);  // the tree's stride 64, then 32 .. 1 toward lane 0
        if (lane == 0) {
            sm.m[h] = m;
            sm.l[h] = l;
        }
    }
    __syncthreads();

    // V: chain (head, element d, slice sl) over the slice's keys in order,
    // one chain a thread (HPW * slices * HD chains: at head_dim 128 with two
    // heads a workgroup, one for each of its 256 threads, so every wave
    // works); the weights are read four keys at a time (one address for the
    // whole wave), KB keys' V reads are in flight together, and whole chunks
    // need no per-key guard.
    constexpr uint32_t slices = HD >= kChunk ? 1 : kChunk / HD;
    const auto v_elem = [&](uint32_t key, uint32_t d) -> float {  // V rows not staged: from the cache
        if (holds_new && key == n - 1) return F16 ? f16_bits_to_float(sm.vnew[d]) : __uint_as_float(sm.vnew[d]);
        if constexpr (F16) return f16_bits_to_float(ldg(static_cast<const uint16_t*>(a.v_cache) + row_of(key) * HD + d));
        else return ldg(static_cast<const float*>(a.v_cache) + row_of(key) * HD + d);
    };
    // w * v as fma(w, v, -0) for an f16 v, as in dot4h.
    const auto prod = [&](float w, float x) {
        if constexpr (F16 && kStageV) return __builtin_fmaf(w, x, nz);
        else return w * x;
    };
    for (uint32_t c = t; c < HPW * slices * HD; c += kThreads) {
        const uint32_t d = c % HD, sl = (c / HD) % slices, h = c / (HD * slices);
        const uint32_t keys = n > sl ? (n - sl + slices - 1) / slices : 0;  // this slice's keys: sl, sl + slices, ...
        // the chain's V column in LDS: key sl + slices j at j * slices * HD (immediate offsets)
        const auto vcol = reinterpret_cast<const std::conditional_t<F16, _Float16, float>*>(sm.v) + sl * HD + d;
        const auto weights = [&](uint32_t j0, float (&w)[KB]) {  // keys j0 .. j0 + KB - 1 of the slice
            const float4* wp = reinterpret_cast<const float4*>(&sm.p[h][slices * j0]);
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
        };
        float o = 0.0f;
        if (kStageV && n == kChunk) {
            // A whole chunk: kChunk / slices keys a chain, whole batches, no
            // bound on a key; each product reads its V element itself.
#pragma unroll 1
            for (uint32_t j0 = 0; j0 < kChunk / slices; j0 += KB) {
                float w[KB];
                weights(j0, w);
#pragma unroll
                for (uint32_t jj = 0; jj < KB; ++jj) o += prod(w[jj], static_cast<float>(vcol[(j0 + jj) * slices * HD]));
            }
        } else {
            for (uint32_t j0 = 0; j0 < keys; j0 += KB) {
                float w[KB], x[KB];
                weights(j0, w);
                if constexpr (kStageV) {
#pragma unroll
                    for (uint32_t jj = 0; jj < KB; ++jj) x[jj] = static_cast<float>(vcol[min(j0 + jj, keys - 1) * slices * HD]);
                } else {
#pragma unroll
                    for (uint32_t jj = 0; jj < KB; ++jj) x[jj] = v_elem(min(sl + slices * (j0 + jj), n - 1), d);
                }
#pragma unroll
                for (uint32_t jj = 0; jj < KB; ++jj)
                    if (j0 + jj < keys) o += prod(w[jj], x[jj]);
            }
        }
        if constexpr (HD > kChunk) {
            st_f32<COH>(a.partial + stats_at(h) * HD + d, o);  // heads wider than the reference's workgroup: no slice sum
        } else {
            sm.red[h][sl * HD + d] = o;
        }
    }
    if constexpr (HD <= kChunk) {
        __syncthreads();
        for (uint32_t i = t; i < HPW * HD; i += kThreads) {
            const uint32_t h = i / HD, d = i % HD;
            float sum = 0.0f;
#pragma unroll
            for (uint32_t sl = 0; sl < slices; ++sl) sum += sm.red[h][sl * HD + d];
            st_f32<COH>(a.partial + stats_at(h) * HD + d, sum);
        }
    }
    if (t < HPW) {
        st_f32<COH>(a.stats + stats_at(t) * 2, sm.m[t]);
        st_f32<COH>(a.stats + stats_at(t) * 2 + 1, sm.l[t]);
    }
}

// attend_merge.comp:25-38 for head h over chunks [0, count) of its `stride`
// (the partials and stats of head h start at chunk h * stride), element d of
// nt = hd threads (d = 0 .. nt - 1; the caller's threads of this head).
// Chunks with a max of -inf hold no keys and are skipped. Every invocation
// of the reference computes the same max M and the same factors
// exp(m_c - M) and weight sum; here each is computed once per head (the
// factors by one thread per chunk, in parallel) and shared through LDS, which
// leaves each element its chain sum += r_c * partial_c. Its partials are
// loaded B chunks at a time with every load in flight. Optionally quantizes
// the result to Q8_0 with f32 scales (quantize.comp:100-111), the o
// projection's input. s_rl: count (factor, weight sum) pairs of LDS; s_wmax:
// nt / 64 floats. Every thread of the workgroup calls it (it synchronizes
// the workgroup). With COH, the partials and stats are read and the results
// stored coherently across XCDs (they come from, and go to, other
// workgroups of the same launch), and out may be null (no f32 output).
template <bool COH, uint32_t B = 64>
__device__ __forceinline__ void merge_head(const float* partial, const float* stats, float* out, uint8_t* values, float* scales,
                                           uint32_t h, uint32_t stride, uint32_t count, uint32_t hd, uint32_t d, float2* s_rl,
                                           float* s_wmax) {
#pragma clang fp contract(off)
    const uint32_t nt = hd;
    const uint64_t first = static_cast<uint64_t>(h) * stride;
    const uint64_t* st = reinterpret_cast<const uint64_t*>(stats) + first;  // (max, weight sum) pairs
    const float* pc = partial + first * hd + d;
    // This thread's first chunk's (max, weight sum), loaded before the
    // partials so that waiting for it does not wait for them, and kept for
    // the factors below (later chunks of a thread, past hd chunks, are
    // loaded again there).
    const uint64_t ml0 = ld_u64<COH>(st + min(d, count - 1));
    float p[B];
#pragma unroll
    for (uint32_t j = 0; j < B; ++j) p[j] = ld_f32<COH>(pc + static_cast<uint64_t>(min(j, count - 1)) * hd);
    // M = max over the chunks' maxima (exact in any order).
    float m = d < count ? __uint_as_float(static_cast<uint32_t>(ml0)) : -__builtin_inff();
    for (uint32_t c = d + nt; c < count; c += nt) m = fmaxf(m, __uint_as_float(static_cast<uint32_t>(ld_u64<COH>(st + c))));
    m = wave_max(m);
    if (d % kWave == 0) s_wmax[d / kWave] = m;
    __syncthreads();
    float top = s_wmax[0];
    for (uint32_t w = 1; w < (nt + kWave - 1) / kWave; ++w) top = fmaxf(top, s_wmax[w]);
    for (uint32_t c = d; c < count; c += nt) {
        const uint64_t ml = c == d ? ml0 : ld_u64<COH>(st + c);
        const float mc = __uint_as_float(static_cast<uint32_t>(ml)), lc = __uint_as_float(static_cast<uint32_t>(ml >> 32));
        s_rl[c] = make_float2(mc == -__builtin_inff() ? -1.0f : vk_expf(mc - top), lc);
    }
    __syncthreads();
    // sum += r_c * partial_c and weight += r_c * l_c over the live chunks in
    // order (every thread carries the weight chain too: the same value).
    // Branch-free: a skipped chunk (and a slot past count) adds +0 * +0 to
    // each chain instead (its operands' bits masked off), which leaves it
    // unchanged: both start at +0 and an f32 sum is -0 only when both
    // addends are, so neither is ever -0 and x + (+0) = x. Eight chunks'
    // (factor, weight sum) pairs are read from LDS at once, then summed.
    float sum = 0.0f, weight = 0.0f;
    for (uint32_t c0 = 0; c0 < count; c0 += B) {
        if (c0 > 0) {
#pragma unroll
            for (uint32_t j = 0; j < B; ++j) p[j] = ld_f32<COH>(pc + static_cast<uint64_t>(min(c0 + j, count - 1)) * hd);
        }
#pragma unroll
        for (uint32_t j0 = 0; j0 < B; j0 += 8) {
            float2 f[8];
#pragma unroll
            for (uint32_t j = 0; j < 8; ++j) f[j] = s_rl[min(c0 + j0 + j, count - 1)];
#pragma unroll
            for (uint32_t j = 0; j < 8 && j0 + j < B; ++j) {
                const uint32_t keep = c0 + j0 + j < count && f[j].x >= 0.0f ? ~0u : 0u;
                const float rr = __uint_as_float(__float_as_uint(f[j].x) & keep);
                sum += rr * __uint_as_float(__float_as_uint(p[j0 + j]) & keep);
                weight += rr * __uint_as_float(__float_as_uint(f[j].y) & keep);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    const float o = sum / weight;
    if (!COH || out) st_f32<COH>(out + static_cast<uint64_t>(h) * hd + d, o);
    if (values) {
        const float absmax = group_max<32>(fabsf(o));
        const float ds = absmax / 127.0f;
        const float inv = ds > 0.0f ? 1.0f / ds : 0.0f;
        st_u8<COH>(values + static_cast<uint64_t>(h) * hd + d, static_cast<uint8_t>(static_cast<int8_t>(quant_code(o, inv))));
        if (d % 32 == 0) st_f32<COH>(scales + (static_cast<uint64_t>(h) * hd + d) / 32, ds);
    }
}

// ------------------------------------------------------------ launch sync

// One block of the sync words of vkml_attend_step_fused: the OSync words
// (the o GEMV's arrival counters), then an arrival counter per set of chunk
// items (KV head, head group), kArriveStride words apart. The sticky error
// flag of every block is word 0 of block 0.
struct FusedSync {
    static constexpr uint32_t kArriveStride = 8;
    static constexpr uint32_t kMaxSets = 256;
    static constexpr uint32_t kWords = OSync::kWords + kArriveStride * kMaxSets;
    __host__ __device__ static uint32_t* arrive(uint32_t* s, uint32_t set) { return s + OSync::kWords + kArriveStride * set; }
};

// Polls a waiting workgroup makes before it gives up, unless the host set
// another limit (vkml_set_wait_limit).
constexpr uint32_t kOSpinCap = 1u << 20;

// Lane 0 polls counter copy wg % kCopies until every merging workgroup has
// arrived; false if the wait gave up (the spin limit, or another
// workgroup's error). The error flag is the sync words' own unless given. Called by every thread; ends with a workgroup barrier
// (the weight loads issued before it stay in flight).
__device__ inline bool await_merged(uint32_t* sync, uint32_t wg, uint32_t arrivals, uint32_t* error, uint32_t cap) {
    __shared__ uint32_t s_ok;
    if (!error) error = OSync::error(sync);
    if (threadIdx.x == 0) {
        uint32_t ok = 1;
        uint32_t* c = OSync::counter(sync, wg % OSync::kCopies);
        for (uint32_t spins = 0;; ++spins) {
            if (__hip_atomic_load(c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= arrivals) break;
            if (spins % 64 == 63 && __hip_atomic_load(error, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) {
                ok = 0;
                break;
            }
            if (spins >= cap) {
                __hip_atomic_store(error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                ok = 0;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        s_ok = ok;
    }
    __syncthreads();
    return s_ok != 0;
}

}  // namespace vkml::attend
