// attend_fast.hpp -- decode attention on the matrix cores: the device code of
// the tolerance form of the reference's attend.comp + attend_merge.comp
// (src/ops/attention.cpp:54-84), used by k_attend_fast.hip.
//
// Not the reference's order of f32 operations. The results are those of
// f32 attention, to within f32 rounding: every product q.k and p.v is exact
// (f16 x f16 in the matrix unit) and every sum is accumulated in f32, but in
// the matrix unit's order rather than attend.comp's chains. The exact form
// (attend.hpp) stays the default; this one is the option that gives up the
// bit-identity for speed.
//
// An item is (chunk of 128 keys, KV head) with every query head of the KV
// head: K and V come from HBM once for the whole group. Its four waves take
// 32 keys each, independently until the end:
//   - scores S^T [32 keys x 16 heads] = K [keys x hd] . Q^T [hd x heads] by
//     v_mfma_f32_16x16x32_f16, q (f32) split in two f16 terms q = hi + lo
//     (hi = f16(q), lo = f16(q - hi)), so each product of q with the f16 key
//     is that of q to about 22 bits;
//   - the wave's max and sum of 2^(s - max) per head (scores in log2 units);
//   - O [heads x hd] = P [heads x keys] . V [keys x hd], P split the same way.
//     The score tile's accumulator layout is the A operand's of the second
//     product (both hold row i = lane % 16, four consecutive k per lane
//     group), so P goes from one to the other in registers; V is read from
//     LDS (copied there by global_load_lds, 16-byte pieces swizzled so that
//     the four lane groups of a read hit different banks).
// The four waves' (max, sum, O) are combined in LDS into the item's partial,
// stored with its (max, weight sum). The last item of a KV head to arrive
// merges that KV head's chunks, and can publish the Q8_0 of the output to
// the o GEMV of the same launch (k_attend_fast.hip).
#pragma once

#include "attend.hpp"

namespace vkml::attend_fast {

using namespace vkml::dev;
using vkml::attend::kThreads;

constexpr uint32_t kItemKeys = 128;  // keys of an item: four waves of 32
constexpr uint32_t kSegment = 32;    // chunks a first-level merge takes (two-level merges)
constexpr uint32_t kOneLevel = 64;   // chunks one merge takes alone
constexpr uint32_t kWaveKeys = 32;
constexpr float kLog2e = 1.44269504088896340736f;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct FastArgs {
    const float* q;  // [heads, hd] f32 (a step: the token's [q | k | v])
    const void* k_cache;
    const void* v_cache;
    float* partial;  // [heads, stride, hd]: an item's unnormalized output
    float* stats;    // [heads, stride, 2]: its (max, weight sum), max in log2 units
    const vkml_decode_state* state;  // a step: the position from here
    uint32_t heads, kv_heads, group, capacity, kv_start, kv_len, chunks;
    float scale, softcap;
    uint32_t ready;  // chunks live at every position of the launch: their loads go before the position is read
    // Arrival counters, kArriveStride words apart (zero before the launch;
    // the last arrival resets each): one per KV head, then with segs > 1
    // one per (KV head, segment of kSegment chunks).
    uint32_t* arrive;
    // 1: the last item of a KV head merges its chunks. More: the last item
    // of each segment merges the segment's chunks, and the last of those
    // merges the segments (long contexts, where one workgroup walking every
    // chunk would take longer than the items).
    uint32_t segs;
    // Chunks an item takes (1, or more for long contexts: a run, whose
    // partial lands in the slot of its first chunk; then segs is 1).
    uint32_t run;
    // The merged output [heads, hd] f32 (may be null), its Q8_0 codes and f32 scales (may be null).
    float* out;
    uint8_t* values;
    float* scales;
};

// LDS of an item. GQ: query heads a KV head has, rounded up to 4 or 8.
template <int HD, int GQ>
struct FastSmem {
    alignas(16) uint8_t v[kItemKeys * HD * 2];  // V rows [key][hd] f16, 16-byte pieces swizzled
    float o[4][GQ][HD];                         // each wave's unnormalized output
    float m[4][GQ], l[4][GQ];
};

// Byte offset in the V tile of element d of row r: piece d / 8 of the row is
// stored at piece (d / 8) ^ (2 ((r / 4) % 4)).
template <int HD>
__device__ __forceinline__ uint32_t v_offset(uint32_t r, uint32_t d) {
    return r * (HD * 2) + 16 * ((d / 8) ^ (2 * ((r / 4) % 4))) + 2 * (d % 8);
}

template <int HD>
struct FastLoads {
    static constexpr int kSteps = HD / 32;  // 32 dims a matrix instruction
    uint4 k[2][kSteps];                     // the wave's two 16-key tiles, 8 f16 a lane a step
    float4 q[kSteps][2];                    // 8 f32 of q a lane a step
};

// Key kk of the item (0 .. 127) at row (key0 + min(kk, n - 1)) % capacity of its KV head.
__device__ __forceinline__ uint64_t fast_row(const FastArgs& a, uint32_t kvh, uint32_t key0, uint32_t kk, uint32_t n) {
    return static_cast<uint64_t>(kvh) * a.capacity + (key0 + min(kk, n - 1)) % a.capacity;
}

// Every load of an item, issued at once: q (lanes of the group's heads), the
// wave's K fragments into registers, and its 32 V rows into LDS. n: keys
// the item holds (rows past them re-read the last).
template <int HD>
__device__ __forceinline__ void fast_load(const FastArgs& a, uint32_t chunk, uint32_t kvh, uint32_t n, FastLoads<HD>& r,
                                          uint8_t* v_lds) {
    constexpr uint32_t RB = HD * 2;
    const uint32_t t = thread_index(), w = t / kWave, l = t % kWave, j = l % 16, g = l / 16;
    const uint32_t key0 = a.kv_start + chunk * kItemKeys;
    if (j < a.group) {
        const float* qp = a.q + static_cast<uint64_t>(kvh * a.group + j) * HD + 8 * g;
#pragma unroll
        for (int s = 0; s < FastLoads<HD>::kSteps; ++s) {
            r.q[s][0] = ldg(reinterpret_cast<const float4*>(qp + 32 * s));
            r.q[s][1] = ldg(reinterpret_cast<const float4*>(qp + 32 * s + 4));
        }
    } else {
#pragma unroll
        for (int s = 0; s < FastLoads<HD>::kSteps; ++s) r.q[s][0] = r.q[s][1] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    const auto* kc = static_cast<const uint8_t*>(a.k_cache);
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
        const uint64_t row = fast_row(a, kvh, key0, kWaveKeys * w + 16 * tt + j, n);
#pragma unroll
        for (int s = 0; s < FastLoads<HD>::kSteps; ++s) r.k[tt][s] = ldg(reinterpret_cast<const uint4*>(kc + row * RB + 64 * s + 16 * g));
    }
    // V: the wave's rows 32 w .. 32 w + 31, 1 KB an instruction
    const auto* vc = static_cast<const uint8_t*>(a.v_cache);
    uint8_t* base = v_lds + kWaveKeys * w * RB;
#pragma unroll
    for (uint32_t i = 0; i < kWaveKeys * RB / 1024; ++i) {
        const uint32_t at = 1024 * i + 16 * l;  // byte in the wave's rows
        const uint32_t rr = kWaveKeys * w + at / RB, piece = (at % RB) / 16;
        const uint32_t src_piece = piece ^ (2 * ((rr / 4) % 4));
        vkml::attend::load_to_lds16(vc + fast_row(a, kvh, key0, rr, n) * RB + 16 * src_piece, base + 1024 * i);
    }
}

// A run's K and V loads for one chunk (fast_load without q): the wave's K
// fragments into registers and its 32 V rows into its rows of the LDS tile.
template <int HD>
__device__ __forceinline__ void fast_load_kv(const FastArgs& a, uint32_t chunk, uint32_t kvh, uint32_t n, uint4 (&k)[2][HD / 32],
                                             uint8_t* v_lds) {
    constexpr uint32_t RB = HD * 2;
    const uint32_t t = thread_index(), w = t / kWave, l = t % kWave, j = l % 16, g = l / 16;
    const uint32_t key0 = a.kv_start + chunk * kItemKeys;
    const auto* kc = static_cast<const uint8_t*>(a.k_cache);
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
        const uint64_t row = fast_row(a, kvh, key0, kWaveKeys * w + 16 * tt + j, n);
#pragma unroll
        for (int s = 0; s < HD / 32; ++s) k[tt][s] = ldg(reinterpret_cast<const uint4*>(kc + row * RB + 64 * s + 16 * g));
    }
    const auto* vc = static_cast<const uint8_t*>(a.v_cache);
    uint8_t* base = v_lds + kWaveKeys * w * RB;
#pragma unroll
    for (uint32_t i = 0; i < kWaveKeys * RB / 1024; ++i) {
        const uint32_t at = 1024 * i + 16 * l;
        const uint32_t rr = kWaveKeys * w + at / RB, piece = (at % RB) / 16;
        const uint32_t src_piece = piece ^ (2 * ((rr / 4) % 4));
        vkml::attend::load_to_lds16(vc + fast_row(a, kvh, key0, rr, n) * RB + 16 * src_piece, base + 1024 * i);
    }
}

// An item over keys key0 .. key0 + n - 1 of KV head kvh, given its loads:
// the partial of each of the group's heads and its (max, weight sum), stored
// coherently (for a merge in another workgroup of the launch).
template <int HD, int GQ>
__device__ __forceinline__ void fast_item(const FastArgs& a, uint32_t chunk, uint32_t kvh, uint32_t n, const FastLoads<HD>& r,
                                          FastSmem<HD, GQ>& sm) {
    constexpr int kSteps = FastLoads<HD>::kSteps;
    const uint32_t t = thread_index(), w = t / kWave, l = t % kWave, j = l % 16, g = l / 16;
    const bool cap = a.softcap > 0.0f;
    // q scaled (and in log2 units without a soft cap), as hi + lo f16 terms
    const float qs = cap ? a.scale : a.scale * kLog2e;
    half8 qh[kSteps], ql[kSteps];
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
        const float x[8] = {r.q[s][0].x, r.q[s][0].y, r.q[s][0].z, r.q[s][0].w, r.q[s][1].x, r.q[s][1].y, r.q[s][1].z, r.q[s][1].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            // The f32 product through an empty asm: both terms come from
            // this one value. Otherwise the compiler folds f16(x qs) into one
            // rounding (v_fma_mixlo_f16) for the residual while the packed
            // operand rounds the f32 product, and where the two differ by an
            // f16 ulp the residual belongs to another high term.
            float v = x[e] * qs;
            asm volatile("" : "+v"(v));
            qh[s][e] = static_cast<_Float16>(v);
            ql[s][e] = static_cast<_Float16>(v - static_cast<float>(qh[s][e]));
        }
    }
    // scores: lane (j, g) holds key 32 w + 16 tt + 4 g + e of head j
    f32x4 acc[2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
        acc[tt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            const half8 kf = __builtin_bit_cast(half8, r.k[tt][s]);
            acc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qh[s], acc[tt], 0, 0, 0);
            acc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, ql[s], acc[tt], 0, 0, 0);
        }
    }
    float sc[2][4];
    float m = -__builtin_inff();
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float x = acc[tt][e];
            if (cap) x = a.softcap * tanhf(fminf(fmaxf(x / a.softcap, -10.0f), 10.0f)) * kLog2e;
            const uint32_t kk = kWaveKeys * w + 16 * tt + 4 * g + e;
            sc[tt][e] = kk < n ? x : -__builtin_inff();
            m = fmaxf(m, sc[tt][e]);
        }
    // the wave's max per head: lanes j, j + 16, j + 32, j + 48
    {
        const uint2 a16 = swap_rows<16>(__float_as_uint(m));
        m = fmaxf(__uint_as_float(a16.x), __uint_as_float(a16.y));
        const uint2 a32 = swap_rows<32>(__float_as_uint(m));
        m = fmaxf(__uint_as_float(a32.x), __uint_as_float(a32.y));
    }
    const bool live = m != -__builtin_inff() && j < a.group;
    float lsum = 0.0f;
    half8 ph, pl;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float p = live ? __builtin_amdgcn_exp2f(sc[tt][e] - m) : 0.0f;
            lsum += p;
            const _Float16 hi = static_cast<_Float16>(p);
            ph[4 * tt + e] = hi;
            pl[4 * tt + e] = static_cast<_Float16>(p - static_cast<float>(hi));
        }
    {
        const uint2 a16 = swap_rows<16>(__float_as_uint(lsum));
        lsum = __uint_as_float(a16.x) + __uint_as_float(a16.y);
        const uint2 a32 = swap_rows<32>(__float_as_uint(lsum));
        lsum = __uint_as_float(a32.x) + __uint_as_float(a32.y);
    }
    // The wave's V rows have landed once its loads are done.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    // O: lane (j, g) gives V at dim 16 dt + j of keys 4 g + e (e < 4) and
    // 16 + 4 g + e - 4 (e >= 4) of the wave's, the keys its P elements hold
    const uint32_t r0 = kWaveKeys * w + 4 * g;
#pragma unroll
    for (int dt = 0; dt < HD / 16; ++dt) {
        const uint32_t d = 16 * dt + j;
        half8 vb;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t rr = r0 + (e < 4 ? e : 12 + e);
            vb[e] = *reinterpret_cast<const _Float16*>(sm.v + v_offset<HD>(rr, d));
        }
        f32x4 o = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        o = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph, vb, o, 0, 0, 0);
        o = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl, vb, o, 0, 0, 0);
        // lane (j, g) holds heads 4 g .. 4 g + 3 at dim d
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (4 * g + e < GQ) sm.o[w][4 * g + e][d] = o[e];
    }
    if (l < GQ) {
        sm.m[w][l] = m;
        sm.l[w][l] = lsum;
    }
    __syncthreads();
    // The item's partial: the waves' outputs at the item's max.
    const uint64_t stride = a.chunks;
    for (uint32_t u = t; u < GQ * HD / 2; u += kThreads) {
        const uint32_t h = 2 * u / HD, d = 2 * u % HD;
        if (h >= a.group) continue;
        float M = -__builtin_inff();
#pragma unroll
        for (int q = 0; q < 4; ++q) M = fmaxf(M, sm.m[q][h]);
        float o0 = 0.0f, o1 = 0.0f, ls = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float mq = sm.m[q][h];
            const float f = mq == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(mq - M);
            o0 += f * sm.o[q][h][d];
            o1 += f * sm.o[q][h][d + 1];
            ls += f * sm.l[q][h];
        }
        const uint64_t at = static_cast<uint64_t>(kvh * a.group + h) * stride + chunk;
        st_f32<true>(a.partial + at * HD + d, o0);
        st_f32<true>(a.partial + at * HD + d + 1, o1);
        if (d == 0) {
            st_f32<true>(a.stats + at * 2, M);
            st_f32<true>(a.stats + at * 2 + 1, ls);
        }
    }
}

// A run of chunks first .. first + count - 1 of KV head kvh (all holding
// live keys; kv_len bounds the last) in one workgroup, for long contexts.
// Each wave keeps its own online softmax per head across the run (its 32
// keys of every chunk): running max M and sum L, and O rescaled by
// 2^(M_old - M_new) as M grows. A wave's V rows are its own, so the chunks
// need no barrier: each waits for its own loads, issues the next chunk's (K
// into the other register set, V into the other LDS tile), then computes.
// At the end the waves combine, as in fast_item, into the run's partial in
// the slot of chunk `first`. v_other: the second V tile (kItemKeys rows).
template <int HD, int GQ>
__device__ __forceinline__ void fast_run(const FastArgs& a, uint32_t first, uint32_t count, uint32_t kvh, uint32_t kv_len,
                                         FastSmem<HD, GQ>& sm, uint8_t* v_other) {
    constexpr int kSteps = HD / 32;
    const uint32_t t = thread_index(), w = t / kWave, l = t % kWave, j = l % 16, g = l / 16;
    const bool cap = a.softcap > 0.0f;
    const auto keys_of = [&](uint32_t c) { return min(kItemKeys, kv_len - (a.kv_start + c * kItemKeys)); };
    uint4 k0[2][kSteps], k1[2][kSteps];
    fast_load_kv<HD>(a, first, kvh, keys_of(first), k0, sm.v);
    // q of head j, scaled (in log2 units without a soft cap), as hi + lo f16
    half8 qh[kSteps], ql[kSteps];
    {
        const float qs = cap ? a.scale : a.scale * kLog2e;
        const float* qp = a.q + static_cast<uint64_t>(kvh * a.group + min(j, a.group - 1)) * HD + 8 * g;
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            const float4 x0 = ldg(reinterpret_cast<const float4*>(qp + 32 * s));
            const float4 x1 = ldg(reinterpret_cast<const float4*>(qp + 32 * s + 4));
            const float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                // the f32 product through an empty asm, as in fast_item
                float v = j < a.group ? x[e] * qs : 0.0f;
                asm volatile("" : "+v"(v));
                qh[s][e] = static_cast<_Float16>(v);
                ql[s][e] = static_cast<_Float16>(v - static_cast<float>(qh[s][e]));
            }
        }
    }
    f32x4 o[HD / 16];
#pragma unroll
    for (int dt = 0; dt < HD / 16; ++dt) o[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float M = -__builtin_inff(), L = 0.0f;  // head j's running max (log2 units) and sum over the wave's keys
    const auto chunk = [&](uint32_t c, const uint4 (&kc)[2][kSteps], uint4 (&kn)[2][kSteps], const uint8_t* vt, uint8_t* vn) {
        const uint32_t n = keys_of(first + c);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's K and V of chunk c have landed
        if (c + 1 < count) fast_load_kv<HD>(a, first + c + 1, kvh, keys_of(first + c + 1), kn, vn);
        f32x4 acc[2];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            acc[tt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int s = 0; s < kSteps; ++s) {
                const half8 kf = __builtin_bit_cast(half8, kc[tt][s]);
                acc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qh[s], acc[tt], 0, 0, 0);
                acc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, ql[s], acc[tt], 0, 0, 0);
            }
        }
        float sc[2][4];
        float m = -__builtin_inff();
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float x = acc[tt][e];
                if (cap) x = a.softcap * tanhf(fminf(fmaxf(x / a.softcap, -10.0f), 10.0f)) * kLog2e;
                const uint32_t kk = kWaveKeys * w + 16 * tt + 4 * g + e;
                sc[tt][e] = kk < n && j < a.group ? x : -__builtin_inff();
                m = fmaxf(m, sc[tt][e]);
            }
        {
            const uint2 a16 = swap_rows<16>(__float_as_uint(m));
            m = fmaxf(__uint_as_float(a16.x), __uint_as_float(a16.y));
            const uint2 a32 = swap_rows<32>(__float_as_uint(m));
            m = fmaxf(__uint_as_float(a32.x), __uint_as_float(a32.y));
        }
        const float mn = fmaxf(M, m);
        const float factor = M == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(M - mn);
        const bool any = mn != -__builtin_inff();
        float bs = 0.0f;
        half8 ph, pl;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float p = any && sc[tt][e] != -__builtin_inff() ? __builtin_amdgcn_exp2f(sc[tt][e] - mn) : 0.0f;
                bs += p;
                const _Float16 hi = static_cast<_Float16>(p);
                ph[4 * tt + e] = hi;
                pl[4 * tt + e] = static_cast<_Float16>(p - static_cast<float>(hi));
            }
        {
            const uint2 a16 = swap_rows<16>(__float_as_uint(bs));
            bs = __uint_as_float(a16.x) + __uint_as_float(a16.y);
            const uint2 a32 = swap_rows<32>(__float_as_uint(bs));
            bs = __uint_as_float(a32.x) + __uint_as_float(a32.y);
        }
        L = L * factor + bs;
        M = mn;
        // O holds heads 4 g + e: their factors come from lanes 4 g + e
        float f4[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) f4[e] = __shfl(factor, 4 * g + e, kWave);
        const uint32_t r0 = kWaveKeys * w + 4 * g;
#pragma unroll
        for (int dt = 0; dt < HD / 16; ++dt) {
            const uint32_t d = 16 * dt + j;
            half8 vb;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t rr = r0 + (e < 4 ? e : 12 + e);
                vb[e] = *reinterpret_cast<const _Float16*>(vt + v_offset<HD>(rr, d));
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) o[dt][e] *= f4[e];
            o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph, vb, o[dt], 0, 0, 0);
            o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl, vb, o[dt], 0, 0, 0);
        }
    };
    for (uint32_t c = 0; c < count; c += 2) {
        chunk(c, k0, k1, sm.v, v_other);
        if (c + 1 < count) chunk(c + 1, k1, k0, v_other, sm.v);
    }
    // lane (j, g) holds heads 4 g .. 4 g + 3 at dim 16 dt + j
#pragma unroll
    for (int dt = 0; dt < HD / 16; ++dt)
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (4 * g + e < GQ) sm.o[w][4 * g + e][16 * dt + j] = o[dt][e];
    if (l < GQ) {
        sm.m[w][l] = M;
        sm.l[w][l] = L;
    }
    __syncthreads();
    // The run's partial: the waves' outputs at the run's max.
    for (uint32_t u = t; u < GQ * HD / 2; u += kThreads) {
        const uint32_t h = 2 * u / HD, d = 2 * u % HD;
        if (h >= a.group) continue;
        float mx = -__builtin_inff();
#pragma unroll
        for (int q = 0; q < 4; ++q) mx = fmaxf(mx, sm.m[q][h]);
        float o0 = 0.0f, o1 = 0.0f, ls = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float mq = sm.m[q][h];
            const float f = mq == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(mq - mx);
            o0 += f * sm.o[q][h][d];
            o1 += f * sm.o[q][h][d + 1];
            ls += f * sm.l[q][h];
        }
        const uint64_t at = static_cast<uint64_t>(kvh * a.group + h) * a.chunks + first;
        st_f32<true>(a.partial + at * HD + d, o0);
        st_f32<true>(a.partial + at * HD + d + 1, o1);
        if (d == 0) {
            st_f32<true>(a.stats + at * 2, mx);
            st_f32<true>(a.stats + at * 2 + 1, ls);
        }
    }
}

// A merge of KV head kvh's heads over the partials in chunk slots first,
// first + stride, ... (count of them): F = sum_c 2^(m_c - M) partial_c and
// L = sum_c 2^(m_c - M) l_c with M the largest m_c. With to_slot >= 0 the
// result is a partial itself (F, and (M, L)), stored in that chunk slot
// (a two-level merge's first level); otherwise the output out = F / L and
// its Q8_0 (quantize.comp's rule: d = absmax / 127, codes rne(x / d)
// clamped). Everything is stored coherently. Thread t takes four
// consecutive elements of a head and every S-th of the slots (S =
// kThreads / (GQ hd / 4)); the S parts meet in LDS (xch: 6 kThreads
// floats). Called by every thread of the workgroup.
template <int HD, int GQ, uint32_t B = 18>
__device__ __forceinline__ void fast_merge(const FastArgs& a, uint32_t kvh, uint32_t first, uint32_t count, uint32_t stride,
                                           int32_t to_slot, float* xch) {
    constexpr uint32_t V4 = GQ * HD / 4;  // float4 groups of the outputs
    constexpr uint32_t S = kThreads / V4;
    static_assert(S >= 1 && kThreads % V4 == 0, "an output group per thread");
    const uint32_t t = thread_index(), vec = t % V4, part = t / V4;
    const uint32_t h = 4 * vec / HD, d = 4 * vec % HD;
    const bool mine = h < a.group;
    const uint64_t row = static_cast<uint64_t>(kvh * a.group + (mine ? h : 0)) * a.chunks;  // the head's slot 0
    const float4* pp = reinterpret_cast<const float4*>(a.partial + row * HD + d);
    const uint64_t* sp = reinterpret_cast<const uint64_t*>(a.stats) + row;
    float M = -__builtin_inff(), L = 0.0f;
    float4 F = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (uint32_t j0 = part; j0 < count; j0 += S * B) {
        float4 pv[B];
        uint64_t st[B];
#pragma unroll
        for (uint32_t b = 0; b < B; ++b) {
            const uint64_t c = first + static_cast<uint64_t>(min(j0 + S * b, count - 1)) * stride;
            st[b] = ld_u64<true>(sp + c);
            pv[b] = ld_f32x4<true>(pp + c * (HD / 4));
        }
        float mb = M;
#pragma unroll
        for (uint32_t b = 0; b < B; ++b)
            if (j0 + S * b < count) mb = fmaxf(mb, __uint_as_float(static_cast<uint32_t>(st[b])));
        const float r = M == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(M - mb);
        F.x *= r; F.y *= r; F.z *= r; F.w *= r;
        L *= r;
        M = mb;
#pragma unroll
        for (uint32_t b = 0; b < B; ++b) {
            const float mc = __uint_as_float(static_cast<uint32_t>(st[b]));
            const float f = j0 + S * b < count && mc != -__builtin_inff() ? __builtin_amdgcn_exp2f(mc - M) : 0.0f;
            F.x += f * pv[b].x; F.y += f * pv[b].y; F.z += f * pv[b].z; F.w += f * pv[b].w;
            L += f * __uint_as_float(static_cast<uint32_t>(st[b] >> 32));
        }
    }
    if constexpr (S > 1) {
        xch[6 * t] = M;
        xch[6 * t + 1] = L;
        xch[6 * t + 2] = F.x; xch[6 * t + 3] = F.y; xch[6 * t + 4] = F.z; xch[6 * t + 5] = F.w;
        __syncthreads();
        if (part == 0) {
#pragma unroll
            for (uint32_t q = 1; q < S; ++q) M = fmaxf(M, xch[6 * (vec + q * V4)]);
            float4 G = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            float LL = 0.0f;
#pragma unroll
            for (uint32_t q = 0; q < S; ++q) {
                const float* x = xch + 6 * (vec + q * V4);
                const float f = x[0] == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(x[0] - M);
                LL += f * x[1];
                G.x += f * x[2]; G.y += f * x[3]; G.z += f * x[4]; G.w += f * x[5];
            }
            F = G;
            L = LL;
        }
    }
    if (part != 0) return;
    if (to_slot >= 0) {
        // a partial of the segment, in the slot of its first chunk
        if (mine) {
            const uint64_t at = row + static_cast<uint32_t>(to_slot);
            float* o = a.partial + at * HD + d;
            st_f32<true>(o, F.x); st_f32<true>(o + 1, F.y); st_f32<true>(o + 2, F.z); st_f32<true>(o + 3, F.w);
            if (d == 0) {
                st_f32<true>(a.stats + at * 2, M);
                st_f32<true>(a.stats + at * 2 + 1, L);
            }
        }
        return;
    }
    const float inv_l = 1.0f / L;
    const float o[4] = {F.x * inv_l, F.y * inv_l, F.z * inv_l, F.w * inv_l};
    const uint64_t out_at = static_cast<uint64_t>(kvh * a.group + h) * HD + d;
    if (mine && a.out) {
#pragma unroll
        for (int e = 0; e < 4; ++e) st_f32<true>(a.out + out_at + e, o[e]);
    }
    if (a.values) {
        // a Q8_0 block of 32 is 8 consecutive lanes
        const float absmax = group_max<8>(fmaxf(fmaxf(fabsf(o[0]), fabsf(o[1])), fmaxf(fabsf(o[2]), fabsf(o[3]))));
        const float ds = absmax / 127.0f;
        const float inv = ds > 0.0f ? 1.0f / ds : 0.0f;
        uint32_t codes = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) codes |= (static_cast<uint32_t>(quant_code(o[e], inv)) & 0xFFu) << (8 * e);
        if (mine) {
            st_u32<true>(reinterpret_cast<uint32_t*>(a.values + out_at), codes);
            if (d % 32 == 0) st_f32<true>(a.scales + out_at / 32, ds);
        }
    }
}

}  // namespace vkml::attend_fast
