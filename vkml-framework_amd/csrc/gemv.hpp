// gemv.hpp -- the int8 GEMV's device code (the reference's
// shaders/gemv_dot.comp), shared by the GEMV kernels (k_gemv.hip) and the
// merge + o launch (k_attend.hip).
//
// Bit-exact by construction. The reference sums each output over 32
// accumulators: accumulator L takes the terms of half-blocks (16 values) L,
// L + 32, L + 64, ... in that order, each term an exact int8 dot product
// scaled in f32 (gemv_dot.comp:85-118), and the 32 are added in a halving
// tree (:121-131). Every f32 operation here happens in that order, so the
// outputs are the reference's bits, and so are the Q8_0 codes the next layer
// quantizes from them.
//
// Mapping. A row's 32 accumulators live in LPR lanes (16 or 8), 32 / LPR
// each. A "round" is the 32 half-blocks (512 values) that give every
// accumulator its next term. Which accumulators a lane holds is chosen per
// weight format so that a lane's share of a round is one or two contiguous
// 16-byte loads and the LPR lanes of a row read one contiguous span:
// - q4_K (16 lanes): lane 8p + 2c + h loads code bytes 16 lane of the
//   round's two super-blocks; low nibbles are half-block 16p + 4c + h, high
//   nibbles 16p + 4c + h + 2. (8 lanes: lane j loads bytes 32j .. 32j + 31,
//   half-blocks 4j .. 4j + 3.)
// - q4_0 / q4_1 (16 lanes): lane l loads block l of the round, half-blocks
//   2l, 2l + 1. (8 lanes: blocks 2j, 2j + 1, half-blocks 4j .. 4j + 3.)
// - q8_0 (16 lanes): lane l loads half-blocks l and l + 16. (8 lanes: j,
//   j + 8, j + 16, j + 24.)
// - 32 lanes (q4_K, q8_0): lane l holds accumulator l, half-block l of the
//   round alone; for q4_K it loads the 16 code bytes that hold it in their
//   low or high nibbles (so lanes l and l ^ 2 load the same bytes).
// The halving tree's strides 16 .. 1 then become, per mapping, additions
// within a lane or exchanges between lanes (xor shuffles).
//
// Each lane keeps two batches of rounds in flight (the next batch loads while
// the current one is summed); the first batch is issued before the workgroup
// stages the activation codes, their per-half-block sums and block scales in
// LDS (GemvRows::start, stage_activation, GemvRows::finish). No MFMA: these
// are matrix-vector products, bound by HBM.
#pragma once

#include <type_traits>

#include "../../include/vkml_hip.h"
#include "device.hpp"

namespace vkml::gemv {

using namespace vkml::dev;

constexpr uint32_t kMaxK = VKML_GEMV_STAGED_MAX_K;  // LDS staging: K + K / 16 * 8 bytes
constexpr uint32_t kLow = 0x0F0F0F0Fu;

struct GemvArgs {
    const uint4* a_values;  // K bytes of activation codes
    const float* a_scales;  // K / 32
    const void* b_values;
    const void* b_scales;
    const void* b2_values;  // SwiGLU: the up matrix
    const void* b2_scales;
    float* out;
    const float* residual;
    uint32_t n, k;
    // With the RMSNorm (or plain Q8_0) prologue: the f32 input row, its norm
    // weight and eps (the activation codes are then computed, not read).
    const float* x;
    const float* norm_weight;
    float eps;
    // SwiGLU with the Q8_0 epilogue: the codes and f32 scales of h.
    uint8_t* out_values;
    float* out_scales;
    // The store epilogue of a decode step's q|k|v projection with RoPE and
    // the KV append (vkml_gemv_rope), when table is not null: output row j
    // is row row0 + j of [q | k | v] (q_rows + 2 kv_rows rows, heads of hd
    // values); q and k rows are rotated in interleaved pairs (rows 2i, 2i + 1
    // of a head) by the state's position, and the k and v rows also go to
    // the caches' row position % capacity, as f16 or f32 bits.
    const float* table;  // cos/sin pairs [positions, hd / 2, 2]
    const vkml_decode_state* state;
    void* k_cache;
    void* v_cache;
    uint32_t row0, q_rows, kv_rows, hd, capacity, kv_f16, rotate;
};

// The accumulator (= half-block of the round) held in slot e of lane l.
template <int FMT, int LPR>
__device__ __forceinline__ constexpr uint32_t acc_index(uint32_t l, uint32_t e) {
    if constexpr (LPR == 32) return l;
    else if constexpr (FMT == VKML_Q8_0) return LPR == 16 ? l + 16 * e : l + 8 * e;
    else if constexpr (FMT == VKML_Q4_K && LPR == 16) return 16 * (l / 8) + 4 * ((l / 2) % 4) + (l % 2) + 2 * e;
    else return (32 / LPR) * l + e;  // q4_0 / q4_1, and q4_K with 8 lanes
}

template <int FMT, int LPR>
struct Plan {
    static constexpr int NS = 32 / LPR;                        // accumulators (slots) per lane
    static constexpr int NQ = FMT == VKML_Q8_0 || LPR == 32 ? NS : NS / 2;  // 16-byte code loads per lane and round
};

// One lane's weights for one round of one matrix: codes, and scales (q4_K:
// the super-block header; q8_0 / q4_0: one scale per slot or block; q4_1:
// scale and offset per block), as raw bits.
template <int FMT, int LPR>
struct RoundW {
    uint4 q[Plan<FMT, LPR>::NQ];
    uint32_t s[FMT == VKML_Q4_K ? 4 : Plan<FMT, LPR>::NS];
};

__device__ __forceinline__ uint32_t ld16(const void* p, uint64_t i) { return ldg(static_cast<const uint16_t*>(p) + i); }
__device__ __forceinline__ uint32_t ld32(const void* p, uint64_t i) { return ldg(static_cast<const uint32_t*>(p) + i); }
__device__ __forceinline__ uint4 ld128(const uint8_t* p) { return ldg(reinterpret_cast<const uint4*>(p)); }

// A raw buffer over `bytes` bytes at p (the gfx9 descriptor word 3), and
// loads at a lane offset plus a scalar offset.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_of(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, static_cast<int>(bytes), 0x00020000);
}
__device__ __forceinline__ uint4 bload128(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(voff), static_cast<int>(soff), 0));
}
__device__ __forceinline__ uint32_t bload32(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, static_cast<int>(voff), static_cast<int>(soff), 0);
}
__device__ __forceinline__ uint32_t bload16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, static_cast<int>(voff), static_cast<int>(soff), 0);
}

// Bytes of an [n, k] matrix's codes and scales (q4_K: 16-byte headers).
template <int FMT>
__host__ __device__ constexpr uint64_t code_bytes(uint64_t n, uint64_t k) {
    return FMT == VKML_Q4_K || FMT == VKML_Q4_0 || FMT == VKML_Q4_1 ? n * k / 2 : n * k;
}
template <int FMT, bool F16S>
__host__ __device__ constexpr uint64_t scale_bytes(uint64_t n, uint64_t k) {
    return FMT == VKML_Q4_K ? n * (k / 256) * 16 : n * (k / 32) * (F16S ? 2 : 4) * (FMT == VKML_Q4_1 ? 2 : 1);
}

// Loads lane l's share of round r of row `row`. Every load is issued
// unconditionally (positions past the row's end, in a last round shorter
// than 512 values, are clamped to its last block and their terms skipped),
// so the compiler can count outstanding loads and wait for one batch while
// the next is still in flight.
template <int FMT, bool F16S, int LPR>
__device__ __forceinline__ void load_round(const void* bv, const void* bs, uint32_t K, uint32_t row, uint32_t r, uint32_t l,
                                           RoundW<FMT, LPR>& w) {
    constexpr int NS = Plan<FMT, LPR>::NS;
    const uint64_t R = row;
    const uint8_t* codes = static_cast<const uint8_t*>(bv);
    if constexpr (FMT == VKML_Q8_0) {
        const uint8_t* base = codes + R * K;
        const uint64_t blocks = R * (K / 32);
#pragma unroll
        for (int e = 0; e < NS; ++e) {
            const uint32_t hb = min(32 * r + acc_index<FMT, LPR>(l, e), K / 16 - 1);
            w.q[e] = ld128(base + 16ull * hb);
            w.s[e] = F16S ? ld16(bs, blocks + hb / 2) : ld32(bs, blocks + hb / 2);
        }
    } else if constexpr (FMT == VKML_Q4_K) {
        const uint32_t p = LPR == 32 ? l / 16 : LPR == 16 ? l / 8 : l / 4;  // which super-block of the round
        const uint32_t sb = min(2 * r + p, K / 256 - 1);
        const uint8_t* base = codes + R * (K / 2) + 128ull * sb;
        if constexpr (LPR == 32) {
            const uint32_t h = l % 16;  // half-block h of the super-block: group h / 4, bytes 16 (h % 2) of it
            w.q[0] = ld128(base + 32 * (h / 4) + 16 * (h % 2));
        } else if constexpr (LPR == 16) {
            w.q[0] = ld128(base + 16 * (l % 8));
        } else {
            w.q[0] = ld128(base + 32 * (l % 4));
            w.q[1] = ld128(base + 32 * (l % 4) + 16);
        }
        const uint4 h = ldg(static_cast<const uint4*>(bs) + R * (K / 256) + sb);
        w.s[0] = h.x; w.s[1] = h.y; w.s[2] = h.z; w.s[3] = h.w;
    } else {
        const uint8_t* base = codes + R * (K / 2);
#pragma unroll
        for (int b = 0; b < NS / 2; ++b) {
            const uint32_t blk = min(16 * r + (LPR == 16 ? l : 2 * l) + b, K / 32 - 1);  // block of the row
            const uint64_t block = R * (K / 32) + blk;
            w.q[b] = ld128(base + 16ull * blk);
            if constexpr (FMT == VKML_Q4_1) {
                if constexpr (F16S) {
                    w.s[2 * b] = ld32(bs, block);  // f16 scale | f16 offset << 16
                } else {
                    const uint2 so = ldg(static_cast<const uint2*>(bs) + block);
                    w.s[2 * b] = so.x;
                    w.s[2 * b + 1] = so.y;
                }
            } else {
                w.s[b] = F16S ? ld16(bs, block) : ld32(bs, block);
            }
        }
    }
}

// The exact dot product of one half-block: 16 weight codes as bytes (four
// words) with 16 activation codes (gemv_dot.comp:105-106).
__device__ __forceinline__ int half_dot(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3, uint4 a) {
    return dot4(w3, a.w, dot4(w2, a.z, dot4(w1, a.y, dot4(w0, a.x, 0))));
}

__device__ __forceinline__ float scale_of(uint32_t bits, bool f16) {
    return f16 ? f16_bits_to_float(bits & 0xFFFFu) : __uint_as_float(bits);
}

// Scale and offset of sub-blocks 2c (low nibbles) and 2c + 1 (high) of a
// q4_K super-block with header h: f16(d * sc) and f16(-(dmin * m)), the
// reference's rounding of its q4_1 repack (src/io/gguf.cpp:123-131,603-617),
// computed as f16 products (exact operands, one rounding to nearest even).
__device__ __forceinline__ void q4k_sub_scales(const uint32_t (&h)[4], uint32_t c, float& s0, float& o0, float& s1, float& o1) {
    const uint32_t shift = (c & 1u) * 16u;
    const uint32_t Y = (h[1] >> shift) & 0xFFFFu, Z = (h[2] >> shift) & 0xFFFFu, W = (h[3] >> shift) & 0xFFFFu;
    uint32_t sc, mn;
    if (c < 2) {
        sc = Y & 0x3F3Fu;
        mn = Z & 0x3F3Fu;
    } else {
        sc = (W & 0x0F0Fu) | ((Y & 0xC0C0u) >> 2);
        mn = ((W >> 4) & 0x0F0Fu) | ((Z & 0xC0C0u) >> 2);
    }
    const _Float16 d = __builtin_bit_cast(_Float16, static_cast<uint16_t>(h[0] & 0xFFFFu));
    const _Float16 nd = -__builtin_bit_cast(_Float16, static_cast<uint16_t>(h[0] >> 16));
    s0 = static_cast<float>(d * static_cast<_Float16>(sc & 0xFFu));
    s1 = static_cast<float>(d * static_cast<_Float16>(sc >> 8));
    o0 = static_cast<float>(nd * static_cast<_Float16>(mn & 0xFFu));
    o1 = static_cast<float>(nd * static_cast<_Float16>(mn >> 8));
}

// The same for sub-block j alone (0 .. 7): the 6-bit scale and min of the
// reference's layout (bytes j, j + 4 of the 12; for j >= 4 their high bits
// in bytes j - 4, j and the low nibbles in byte j + 4). A lane's j is fixed,
// so the bit-field positions are computed once (Q4kField) and each round
// costs two selects and four field extracts.
struct Q4kField {
    uint32_t hi;                   // j >= 4: low bits from word 3
    uint32_t pos_sc, pos_mn, wlo;  // first field: position in its word (scale, min) and width
    uint32_t pos_top, wtop;        // j >= 4: the two high bits in words 1 and 2 (width 0 otherwise)
};
__device__ __forceinline__ Q4kField q4k_field(uint32_t j) {
    const uint32_t b = 8 * (j % 4);
    if (j < 4) return {0u, b, b, 6u, 0u, 0u};
    return {1u, b, b + 4, 4u, b + 6, 2u};
}
__device__ __forceinline__ void q4k_sub_scale(const uint32_t (&h)[4], const Q4kField& f, float& s, float& o) {
    const uint32_t wsc = f.hi ? h[3] : h[1], wmn = f.hi ? h[3] : h[2];
    const uint32_t sc = __builtin_amdgcn_ubfe(wsc, f.pos_sc, f.wlo) | (__builtin_amdgcn_ubfe(h[1], f.pos_top, f.wtop) << 4);
    const uint32_t mn = __builtin_amdgcn_ubfe(wmn, f.pos_mn, f.wlo) | (__builtin_amdgcn_ubfe(h[2], f.pos_top, f.wtop) << 4);
    const _Float16 d = __builtin_bit_cast(_Float16, static_cast<uint16_t>(h[0] & 0xFFFFu));
    const _Float16 nd = -__builtin_bit_cast(_Float16, static_cast<uint16_t>(h[0] >> 16));
    s = static_cast<float>(d * static_cast<_Float16>(static_cast<uint16_t>(sc)));
    o = static_cast<float>(nd * static_cast<_Float16>(static_cast<uint16_t>(mn)));
}

// One lane's activation operands of one round: each slot's 16 codes and its
// half-block's (code sum, block scale), read from LDS before the round's
// arithmetic so a batch's reads are in flight together.
template <int FMT, int LPR>
struct RoundA {
    uint4 a[Plan<FMT, LPR>::NS];
    float2 ss[Plan<FMT, LPR>::NS];
};

template <int FMT, int LPR, bool FULL>
__device__ __forceinline__ void fetch_act(uint32_t r, uint32_t l, uint32_t K, const uint4* s_codes, const float2* s_ss,
                                          RoundA<FMT, LPR>& x) {
#pragma unroll
    for (int e = 0; e < Plan<FMT, LPR>::NS; ++e) {
        const uint32_t hb = 32 * r + acc_index<FMT, LPR>(l, e);
        const bool live = FULL || hb < K / 16;
        x.a[e] = live ? s_codes[hb] : make_uint4(0, 0, 0, 0);
        x.ss[e] = live ? s_ss[hb] : make_float2(0.0f, 0.0f);
    }
}

// Adds one lane's terms of round r to acc[0 .. NS) with the reference's
// expressions (gemv_dot.comp:112,114): q8_0 / q4_0 float(d) * (scale * sa);
// q4_1 and q4_K sa * (float(d) * scale + float(sum) * offset). The
// activation codes, and each half-block's code sum with its block's scale,
// come from LDS (fetch_act). FULL: every half-block of the round is in the
// row (K a multiple of 512). jf: the lane's q4_K sub-block fields (32 lanes).
template <int FMT, bool F16S, int LPR, bool FULL = false>
__device__ __forceinline__ void round_terms(const RoundW<FMT, LPR>& w, const RoundA<FMT, LPR>& x, uint32_t r, uint32_t l,
                                            uint32_t K, const Q4kField& jf, float (&acc)[Plan<FMT, LPR>::NS]) {
#pragma clang fp contract(off)
    constexpr int NS = Plan<FMT, LPR>::NS;
    const uint32_t halves = K / 16;
    float s[NS], o[NS];
    int d[NS];
    uint4 a[NS];
    bool live[NS];
#pragma unroll
    for (int e = 0; e < NS; ++e) {
        live[e] = FULL || 32 * r + acc_index<FMT, LPR>(l, e) < halves;
        a[e] = x.a[e];
    }
    if constexpr (FMT == VKML_Q8_0) {
#pragma unroll
        for (int e = 0; e < NS; ++e) {
            d[e] = half_dot(w.q[e].x, w.q[e].y, w.q[e].z, w.q[e].w, a[e]);
            s[e] = scale_of(w.s[e], F16S);
        }
    } else if constexpr (FMT == VKML_Q4_K && LPR == 32) {
        // Half-block hb of the super-block is in sub-block hb / 2: the low
        // nibbles of its bytes for an even sub-block, the high for an odd one.
        const uint32_t sh = 4 * ((l / 2) % 2);
        q4k_sub_scale(w.s, jf, s[0], o[0]);
        const uint4 q = w.q[0];
        d[0] = half_dot((q.x >> sh) & kLow, (q.y >> sh) & kLow, (q.z >> sh) & kLow, (q.w >> sh) & kLow, a[0]);
    } else if constexpr (FMT == VKML_Q4_K) {
        const uint32_t c = LPR == 16 ? (l / 2) % 4 : l % 4;
        float s0, o0, s1, o1;
        q4k_sub_scales(w.s, c, s0, o0, s1, o1);
        if constexpr (LPR == 16) {
            const uint4 q = w.q[0];
            d[0] = half_dot(q.x & kLow, q.y & kLow, q.z & kLow, q.w & kLow, a[0]);
            d[1] = half_dot((q.x >> 4) & kLow, (q.y >> 4) & kLow, (q.z >> 4) & kLow, (q.w >> 4) & kLow, a[1]);
            s[0] = s0; o[0] = o0; s[1] = s1; o[1] = o1;
        } else {
            const uint4 q0 = w.q[0], q1 = w.q[1];
            d[0] = half_dot(q0.x & kLow, q0.y & kLow, q0.z & kLow, q0.w & kLow, a[0]);
            d[1] = half_dot(q1.x & kLow, q1.y & kLow, q1.z & kLow, q1.w & kLow, a[1]);
            d[2] = half_dot((q0.x >> 4) & kLow, (q0.y >> 4) & kLow, (q0.z >> 4) & kLow, (q0.w >> 4) & kLow, a[2]);
            d[3] = half_dot((q1.x >> 4) & kLow, (q1.y >> 4) & kLow, (q1.z >> 4) & kLow, (q1.w >> 4) & kLow, a[3]);
            s[0] = s0; o[0] = o0; s[1] = s0; o[1] = o0; s[2] = s1; o[2] = o1; s[3] = s1; o[3] = o1;
        }
    } else {
        // QuantizedMatrix q4 words: byte j holds value j (low) and j + 4 (high).
#pragma unroll
        for (int b = 0; b < NS / 2; ++b) {
            const uint4 q = w.q[b];
            d[2 * b] = half_dot(q.x & kLow, (q.x >> 4) & kLow, q.y & kLow, (q.y >> 4) & kLow, a[2 * b]);
            d[2 * b + 1] = half_dot(q.z & kLow, (q.z >> 4) & kLow, q.w & kLow, (q.w >> 4) & kLow, a[2 * b + 1]);
            if constexpr (FMT == VKML_Q4_1) {
                const float sc = F16S ? f16_bits_to_float(w.s[2 * b] & 0xFFFFu) : __uint_as_float(w.s[2 * b]);
                const float of = F16S ? f16_bits_to_float(w.s[2 * b] >> 16) : __uint_as_float(w.s[2 * b + 1]);
                s[2 * b] = s[2 * b + 1] = sc;
                o[2 * b] = o[2 * b + 1] = of;
            } else {
                s[2 * b] = s[2 * b + 1] = scale_of(w.s[b], F16S);
            }
        }
    }
#pragma unroll
    for (int e = 0; e < NS; ++e) {
        if (!live[e]) continue;
        const float2 ss = x.ss[e];  // (code sum, block scale)
        const float sa = ss.y;
        if constexpr (FMT == VKML_Q4_1 || FMT == VKML_Q4_K) {
            acc[e] += sa * (static_cast<float>(d[e]) * s[e] + ss.x * o[e]);
        } else {
            // q4_0 codes are q + 8: the reference's signed bytes (q4_bytes)
            // give the same exact sum, d - 8 * sum(a).
            if constexpr (FMT == VKML_Q4_0) d[e] -= 8 * static_cast<int>(ss.x);
            acc[e] += static_cast<float>(d[e]) * (s[e] * sa);
        }
    }
}

// The halving tree over the 32 accumulators of a row, strides 16, 8, 4, 2,
// 1 (gemv_dot.comp:121-131), each a move from lane l + stride down to lane
// l or an addition within a lane as the mapping places accumulator
// L + stride. The row's sum lands on its lane 0 (the only one read).
template <int FMT, int LPR>
__device__ __forceinline__ float row_tree(float (&acc)[32 / LPR]) {
#pragma clang fp contract(off)
    const auto down = [](float v, int mask) {
        switch (mask) {
            case 16: return lane_down<16>(v);
            case 8: return lane_down<8>(v);
            case 4: return lane_down<4>(v);
            case 2: return lane_down<2>(v);
            default: return lane_down<1>(v);
        }
    };
    const auto x = [&](int mask, int slots) {
#pragma unroll
        for (int e = 0; e < 32 / LPR; ++e)
            if (e < slots) acc[e] += down(acc[e], mask);
    };
    if constexpr (LPR == 32) {  // L = l
        x(16, 1); x(8, 1); x(4, 1); x(2, 1); x(1, 1);
    } else if constexpr (FMT == VKML_Q8_0 && LPR == 16) {  // L = l + 16e
        acc[0] += acc[1];
        x(8, 1); x(4, 1); x(2, 1); x(1, 1);
    } else if constexpr (FMT == VKML_Q8_0) {  // L = j + 8e
        acc[0] += acc[2]; acc[1] += acc[3];
        acc[0] += acc[1];
        x(4, 1); x(2, 1); x(1, 1);
    } else if constexpr (FMT == VKML_Q4_K && LPR == 16) {  // L = 16p + 4c + h + 2e, l = 8p + 2c + h
        x(8, 2); x(4, 2); x(2, 2);
        acc[0] += acc[1];
        x(1, 1);
    } else if constexpr (LPR == 16) {  // q4_0 / q4_1: L = 2l + e
        x(8, 2); x(4, 2); x(2, 2); x(1, 2);
        acc[0] += acc[1];
    } else {  // L = 4j + e: q4_0 / q4_1 / q4_K with 8 lanes
        x(4, 4); x(2, 4); x(1, 4);
        acc[0] += acc[2]; acc[1] += acc[3];
        acc[0] += acc[1];
    }
    return acc[0];
}

enum { kStore = 0, kAdd = 1, kSwiglu = 2 };

// The prologue that replaces a separate rms_norm + quantize launch: RMSNorm
// of x in rms_norm.comp's order at its workgroup width of 256 (invocation v
// sums x[c]^2 over c = v, v + 256, ...; then the halving tree), emulated by
// T threads; then y = x * scale * w and Q8_0 per 32 values
// (quantize.comp:100-111), written to LDS as the activation codes and each
// half-block's (code sum, block scale): vkml_rms_norm_quantize's results bit
// for bit. K <= 4096 and T >= 128. Every load is coalesced and issued at
// once, into registers: the strided elements of the sum (lanes take
// consecutive c), and x and w four values a lane (lane q of the workgroup
// takes values 4q .. 4q + 3, so a 32-value block is 8 consecutive lanes,
// whose absmax is a shuffle reduction among them).
template <uint32_t T>
struct NormLoads {
    static constexpr uint32_t V = T >= 256 ? 1 : 256 / T;  // invocations per thread (t, t + T, ... below 256)
    static constexpr uint32_t kMaxPer = 4096 / 256;        // elements per invocation at K <= 4096
    static constexpr uint32_t Q4 = (4096 / 4 + T - 1) / T; // float4s of x (and w) per thread
    float4 xq[Q4], wq[Q4];                                 // x and w at float4 t + T i
    float xv[V][kMaxPer];                                  // its invocations' strided elements
};

template <uint32_t T, bool COH, bool PLAIN = false>
__device__ __forceinline__ void norm_loads(const float* x, const float* w, uint32_t K, NormLoads<T>& r) {
    const uint32_t t = thread_index();
#pragma unroll
    for (uint32_t i = 0; i < NormLoads<T>::Q4; ++i) {
        const uint32_t q = min(t + T * i, K / 4 - 1);
        r.xq[i] = ld_f32x4<COH>(reinterpret_cast<const float4*>(x) + q);
        if constexpr (!PLAIN) r.wq[i] = ldg(reinterpret_cast<const float4*>(w) + q);
    }
    if (!PLAIN && (T <= 256 || t < 256)) {  // threads past the 256 invocations load none; no sum without the norm
#pragma unroll
        for (uint32_t v = 0; v < NormLoads<T>::V; ++v)
#pragma unroll
            for (uint32_t j = 0; j < NormLoads<T>::kMaxPer; ++j) r.xv[v][j] = ld_f32<COH>(x + min((t + v * T) % 256 + 256 * j, K - 1));
    }
}

template <uint32_t T, bool PLAIN = false>
__device__ void norm_quantize_prologue(const NormLoads<T>& r, float eps, uint32_t K, uint4* s_codes, float2* s_ss, float* s_red) {
#pragma clang fp contract(off)
    static_assert(T >= 128 && T % 64 == 0, "workgroup width");
    const uint32_t t = thread_index();
    float scale = 1.0f;  // PLAIN (quantize.comp on x itself, no norm): unused
    if constexpr (!PLAIN) {
#pragma unroll
        for (uint32_t v = 0; v < NormLoads<T>::V; ++v) {
            const uint32_t inv = t + v * T;
            float part = 0.0f;
#pragma unroll
            for (uint32_t j = 0; j < NormLoads<T>::kMaxPer; ++j)
                if (inv + 256 * j < K) part += r.xv[v][j] * r.xv[v][j];
            if (inv < 256) s_red[inv] = part;
        }
        // The halving tree over the 256 invocations: strides 128, 64, then 32 .. 1 in wave 0.
        __syncthreads();
        if (t < 128) s_red[t] = s_red[t] + s_red[t + 128];
        __syncthreads();
        if (t < 64) {
            const float v = tree_to_first<64>(s_red[t] + s_red[t + 64]);
            if (t == 0) s_red[256] = v;
        }
        __syncthreads();
        scale = 1.0f / sqrtf(s_red[256] / static_cast<float>(K) + eps);
    }
    uint32_t* s_words = reinterpret_cast<uint32_t*>(s_codes);
#pragma unroll
    for (uint32_t i = 0; i < NormLoads<T>::Q4; ++i) {
        const uint32_t q = t + T * i;  // values 4q .. 4q + 3: block q / 8, half-block q / 4
        const float xs[4] = {r.xq[i].x, r.xq[i].y, r.xq[i].z, r.xq[i].w};
        float ws[4] = {1.0f, 1.0f, 1.0f, 1.0f};
        if constexpr (!PLAIN) {
            ws[0] = r.wq[i].x; ws[1] = r.wq[i].y; ws[2] = r.wq[i].z; ws[3] = r.wq[i].w;
        }
        float y[4];
        float absmax = 0.0f;
#pragma unroll
        for (uint32_t e = 0; e < 4; ++e) {
            y[e] = PLAIN ? xs[e] : xs[e] * scale * ws[e];  // PLAIN: quantize.comp on x itself
            absmax = fmaxf(absmax, fabsf(y[e]));
        }
        absmax = group_max<8>(absmax);  // the block's 8 lanes (T is a multiple of 8)
        const float d = absmax / 127.0f;
        const float inv = d > 0.0f ? 1.0f / d : 0.0f;
        const uint32_t word = (static_cast<uint32_t>(quant_code(y[0], inv)) & 0xFFu) |
                              ((static_cast<uint32_t>(quant_code(y[1], inv)) & 0xFFu) << 8) |
                              ((static_cast<uint32_t>(quant_code(y[2], inv)) & 0xFFu) << 16) |
                              (static_cast<uint32_t>(quant_code(y[3], inv)) << 24);
        const int part = dot4(word, 0x01010101u, 0);
        const int sum = part + dpp_i<dpp::shl(1)>(part) + dpp_i<dpp::shl(2)>(part) + dpp_i<dpp::shl(3)>(part);  // on lanes q % 4 == 0
        if (q < K / 4) {
            s_words[q] = word;
            if (q % 4 == 0) s_ss[q / 4] = make_float2(static_cast<float>(sum), d);
        }
    }
}


// The rows of one item (T / LPR consecutive rows) of a GEMV: start() issues
// the item's first PRE batches of weight loads (1 or 2), which depend on
// nothing computed at run time, so a caller can issue them early (before the
// activation is staged, or before a grid barrier); finish() sums the rounds
// over the staged activation and applies the epilogue, keeping two batches
// in flight. PRE = 0: the row's every round is one batch (K at most 512 B),
// all issued by start(), so a short row costs one round trip to memory, not
// one a batch. With COH, the outputs (and the Q8_0 output) are stored
// write-through, coherently across XCDs, for readers in other workgroups of
// the same launch; g.out may then be null (no f32 output). FULL: K a
// multiple of 1024 B (every round whole, and the rounds whole pairs of
// batches, so no round is skipped); with PRE = 0, K = 512 B.
//
// q4_K and q8_0 weights are read with buffer loads: a lane's byte offset
// into the matrix is computed once per item, and each round adds a scalar
// offset (the matrix must be under 4 GiB).
template <int FMT, bool F16S, int LPR, int EPI, int B, uint32_t T, bool QOUT, bool COH, int PRE = 1, bool FULL = false>
struct GemvRows {
    static constexpr int NS = Plan<FMT, LPR>::NS;
    static constexpr int NM = EPI == kSwiglu ? 2 : 1;
    static constexpr uint32_t kRows = T / LPR;
    static constexpr bool kBuf = FMT == VKML_Q4_K || FMT == VKML_Q8_0;
    RoundW<FMT, LPR> wa[B][NM], wb[B][NM];
    uint32_t item, row, r_row, l, rounds;
    float res;     // + residual: the row's residual, loaded by start()
    int32_t pos;   // RoPE epilogue: the state's position, loaded by start()
    __amdgpu_buffer_rsrc_t rc[NM], rs[NM];  // kBuf: codes and scales of each matrix
    uint32_t vq, vs;                        // kBuf: the lane's byte offsets at round 0

    // Per-round byte strides of codes and scales (kBuf).
    static constexpr uint32_t kCodeStride = FMT == VKML_Q4_K ? 256 : 512;
    static constexpr uint32_t kScaleStride = FMT == VKML_Q4_K ? 32 : (F16S ? 32 : 64);

    // Byte distance from slot 0's code / scale load to slot e's (kBuf): q4_K
    // at 8 lanes loads bytes 32j .. 32j + 31 as two 16-byte loads; q8_0 slot e
    // is half-block acc_index(l, e) = acc_index(l, 0) + (32 / LPR) ... apart.
    static constexpr uint32_t code_delta(int e) {
        return FMT == VKML_Q4_K ? 16u * e : 16u * (acc_index<FMT, LPR>(0, e) - acc_index<FMT, LPR>(0, 0));
    }
    static constexpr uint32_t scale_delta(int e) {
        return (F16S ? 2u : 4u) * ((acc_index<FMT, LPR>(0, e) - acc_index<FMT, LPR>(0, 0)) / 2);
    }

    __device__ __forceinline__ void load_batch(const GemvArgs& g, RoundW<FMT, LPR> (&w)[B][NM], uint32_t r0) {
        // Rounds past the last reload the last one (cache hits): unconditional loads.
#pragma unroll
        for (int i = 0; i < B; ++i) {
            const uint32_t r = min(r0 + i, rounds - 1);
            if constexpr (kBuf) {
#pragma unroll
                for (int m = 0; m < NM; ++m) {
#pragma unroll
                    for (int e = 0; e < Plan<FMT, LPR>::NQ; ++e) w[i][m].q[e] = bload128(rc[m], vq + code_delta(e), kCodeStride * r);
                    if constexpr (FMT == VKML_Q4_K) {
                        const uint4 h = bload128(rs[m], vs, kScaleStride * r);
                        w[i][m].s[0] = h.x; w[i][m].s[1] = h.y; w[i][m].s[2] = h.z; w[i][m].s[3] = h.w;
                    } else {
#pragma unroll
                        for (int e = 0; e < NS; ++e)
                            w[i][m].s[e] = F16S ? bload16(rs[m], vs + scale_delta(e), kScaleStride * r)
                                                : bload32(rs[m], vs + scale_delta(e), kScaleStride * r);
                    }
                }
            } else {
                load_round<FMT, F16S, LPR>(g.b_values, g.b_scales, g.k, r_row, r, l, w[i][0]);
                if constexpr (NM == 2) load_round<FMT, F16S, LPR>(g.b2_values, g.b2_scales, g.k, r_row, r, l, w[i][NM - 1]);
            }
        }
    }

    __device__ __forceinline__ void start(const GemvArgs& g, uint32_t it) {
        item = it;
        rounds = (g.k + 511) / 512;
        const uint32_t t = thread_index();
        l = t % LPR;
        row = it * kRows + t / LPR;
        r_row = min(row, g.n - 1);
        if constexpr (kBuf) {
            const uint32_t K = g.k, R = r_row;
            rc[0] = buffer_of(g.b_values, static_cast<uint32_t>(code_bytes<FMT>(g.n, K)));
            rs[0] = buffer_of(g.b_scales, static_cast<uint32_t>(scale_bytes<FMT, F16S>(g.n, K)));
            if constexpr (NM == 2) {
                rc[1] = buffer_of(g.b2_values, static_cast<uint32_t>(code_bytes<FMT>(g.n, K)));
                rs[1] = buffer_of(g.b2_scales, static_cast<uint32_t>(scale_bytes<FMT, F16S>(g.n, K)));
            }
            if constexpr (FMT == VKML_Q4_K) {
                // the lane's super-block of the round and its first code byte in it
                const uint32_t p = LPR == 32 ? l / 16 : LPR == 16 ? l / 8 : l / 4;
                const uint32_t off = LPR == 32 ? 32 * ((l % 16) / 4) + 16 * (l % 2) : LPR == 16 ? 16 * (l % 8) : 32 * (l % 4);
                vq = R * (K / 2) + 128 * p + off;
                vs = (R * (K / 256) + p) * 16;
            } else {
                const uint32_t hb = acc_index<FMT, LPR>(l, 0);  // slot 0's half-block of the round
                vq = R * K + 16 * hb;
                vs = (R * (K / 32) + hb / 2) * (F16S ? 2 : 4);
            }
        }
        // (the RoPE epilogue's position first, so that waiting for it later
        // does not wait for the weights)
        if constexpr (EPI == kStore) {
            if (g.table) pos = ld_scalar_i32(&g.state->position);
        }
        load_batch(g, wa, 0);
        if constexpr (PRE == 2) load_batch(g, wb, B);
        // The residual is read now, not after the sums: one round trip less
        // at the end of the kernel.
        if constexpr (EPI == kAdd) res = ldg(g.residual + r_row);
    }

    // The RoPE epilogue: the row's rotated value (q and k rows; v rows as
    // they are) given the row's sum y and the pair's other row's sum other,
    // with (c, s) its cos/sin (rope.comp:94-118, vkml_rope_kv_append's
    // arithmetic); then the k and v rows' cache bits stored at the
    // position's cache row.
    __device__ __forceinline__ float rope_store(const GemvArgs& g, uint32_t gr, float y, float other, float2 cs) const {
#pragma clang fp contract(off)
        float v = y;
        if (g.rotate && gr < g.q_rows + g.kv_rows) {
            const bool odd = gr & 1u;
            const float a = odd ? other : y, b = odd ? y : other;
            v = odd ? a * cs.y + b * cs.x : a * cs.x - b * cs.y;
        }
        if (gr >= g.q_rows) {
            const bool is_k = gr < g.q_rows + g.kv_rows;
            const uint32_t kr = gr - g.q_rows - (is_k ? 0u : g.kv_rows);  // row within the kv heads' [kv_heads, hd]
            const uint64_t at = (static_cast<uint64_t>(kr / g.hd) * g.capacity + static_cast<uint32_t>(pos) % g.capacity) * g.hd + kr % g.hd;
            void* cache = is_k ? g.k_cache : g.v_cache;
            if (g.kv_f16) stg(static_cast<uint16_t*>(cache) + at, static_cast<uint16_t>(f32_to_f16_bits(__float_as_uint(v))));
            else stg(static_cast<uint32_t*>(cache) + at, __float_as_uint(v));
        }
        return v;
    }

    __device__ __forceinline__ void finish(const GemvArgs& g, const uint4* s_codes, const float2* s_ss) {
#pragma clang fp contract(off)
        const uint32_t K = g.k;
        float acc[NM][NS];
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int e = 0; e < NS; ++e) acc[m][e] = 0.0f;
        const Q4kField jf = q4k_field((l % 16) / 2);
        // RoPE epilogue: the row's cos/sin, in flight during the sums (the
        // position arrived long before).
        float2 cs = make_float2(0.0f, 0.0f);
        if constexpr (EPI == kStore) {
            if (g.table && g.rotate) {
                const uint32_t gr = g.row0 + r_row;
                if (gr < g.q_rows + g.kv_rows)
                    cs = ldg(reinterpret_cast<const float2*>(g.table + static_cast<uint64_t>(pos) * g.hd + (gr % g.hd & ~1u)));
            }
        }
        const auto sum_batch = [&](const RoundW<FMT, LPR> (&w)[B][NM], uint32_t r0) {
            if constexpr (FULL && LPR == 32) {
                // one slot a lane: the batch's activation reads fit in registers
                RoundA<FMT, LPR> x[B];
#pragma unroll
                for (int i = 0; i < B; ++i) fetch_act<FMT, LPR, true>(r0 + i, l, K, s_codes, s_ss, x[i]);
#pragma unroll
                for (int i = 0; i < B; ++i)
#pragma unroll
                    for (int m = 0; m < NM; ++m) round_terms<FMT, F16S, LPR, true>(w[i][m], x[i], r0 + i, l, K, jf, acc[m]);
            } else {
#pragma unroll
                for (int i = 0; i < B; ++i) {
                    if (r0 + i < rounds) {
                        RoundA<FMT, LPR> x;
                        fetch_act<FMT, LPR, FULL>(r0 + i, l, K, s_codes, s_ss, x);
#pragma unroll
                        for (int m = 0; m < NM; ++m) round_terms<FMT, F16S, LPR, FULL>(w[i][m], x, r0 + i, l, K, jf, acc[m]);
                    }
                }
            }
        };
        if constexpr (PRE == 0) {
            sum_batch(wa, 0);  // every round in flight since start()
        } else if constexpr (PRE == 2) {
            // Both batches are in flight on entry; the last pair of batches
            // is peeled so that no load is issued past the rows' end.
            uint32_t r0 = 0;
            for (; r0 + 2 * B < rounds; r0 += 2 * B) {
                sum_batch(wa, r0);
                load_batch(g, wa, r0 + 2 * B);
                sum_batch(wb, r0 + B);
                load_batch(g, wb, r0 + 3 * B);
            }
            sum_batch(wa, r0);
            sum_batch(wb, r0 + B);
        } else {
            // (the scheduling barriers keep each batch's loads issued before
            // the arithmetic on the previous batch, which would otherwise be
            // hoisted above them together with its wait for the loads)
            for (uint32_t r0 = 0; r0 < rounds; r0 += 2 * B) {
                load_batch(g, wb, r0 + B);
                __builtin_amdgcn_sched_barrier(0);
                sum_batch(wa, r0);
                load_batch(g, wa, r0 + 2 * B);
                __builtin_amdgcn_sched_barrier(0);
                sum_batch(wb, r0 + B);
            }
        }

        float y[NM];
#pragma unroll
        for (int m = 0; m < NM; ++m) y[m] = row_tree<FMT, LPR>(acc[m]);
        // RoPE epilogue: rows 2i and 2i + 1 (the item's rows start even) are
        // LPR lanes apart in one wave; lane 0 of each gets the other's sum.
        float other = 0.0f;
        if constexpr (EPI == kStore) {
            if (g.table) other = __shfl_xor(y[0], LPR);
        }
        float result = 0.0f;
        if (l == 0 && row < g.n) {
            if constexpr (EPI == kStore) {
                result = g.table ? rope_store(g, g.row0 + row, y[0], other, cs) : y[0];
            } else if constexpr (EPI == kAdd) {
                result = res + y[0];  // add(x, attn_out), llama.cpp:374,386
            } else {
                // silu(gate) * up (unary.comp:21-24, then binary.comp's mul)
                const float gate = y[0], up = y[NM - 1];
                result = gate / (1.0f + vk_expf(-gate)) * up;
            }
            if (!COH || g.out) st_f32<COH>(g.out + row, result);
        }
        if constexpr (QOUT) {
            // The item's T / LPR = 32 rows are one Q8_0 block of the output
            // (quantize.comp:100-111): its absmax, scale and codes.
            static_assert(T / LPR == 32, "one Q8_0 block per item");
            __shared__ float s_out[32];
            const uint32_t t = thread_index();
            if (l == 0) s_out[t / LPR] = result;
            __syncthreads();
            if (t < 32) {
                const float v = s_out[t];
                const float absmax = group_max<32>(fabsf(v));
                const float d = absmax / 127.0f;
                const float inv = d > 0.0f ? 1.0f / d : 0.0f;
                st_u8<COH>(g.out_values + item * 32 + t, static_cast<uint8_t>(static_cast<int8_t>(quant_code(v, inv))));
                if (t == 0) st_f32<COH>(g.out_scales + item, d);
            }
            __syncthreads();  // s_out is free for the next item
        }
    }
};

// LDS bytes stage_activation uses for K: the codes, then (code sum, block
// scale) per half-block, then the norm's 257 floats.
__host__ __device__ constexpr uint32_t stage_bytes(uint32_t k, bool norm) { return k + k / 16 * 8 + (norm ? 257 * 4 : 0); }

// The activation's loads (the Q8_0 codes and scales of up to 4 T
// half-blocks; or with NORM, the prologue's loads), issued by a kernel
// before its first weight loads: loads complete in order, so waiting for
// these then does not wait for the weights, which stay in flight while the
// activation is staged.
template <uint32_t T>
struct ActLoads {
    uint4 c[4];
    float sa[4];
};
// NORM: 0, the activation's Q8_0 codes and scales are read; 1, RMSNorm +
// Q8_0 of the f32 row g.x; 2, Q8_0 of g.x alone.
template <uint32_t T, int NORM>
using StageLoads = std::conditional_t<NORM != 0, NormLoads<T>, ActLoads<T>>;

template <uint32_t T, int NORM, bool COH>
__device__ __forceinline__ void stage_load(const GemvArgs& g, StageLoads<T, NORM>& r) {
    if constexpr (NORM != 0) {
        norm_loads<T, COH, NORM == 2>(g.x, g.norm_weight, g.k, r);
    } else {
        const uint32_t halves = g.k / 16, t = thread_index();
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t h = t + i * T;
            r.c[i] = h < halves ? ld_u128<COH>(g.a_values + h) : make_uint4(0, 0, 0, 0);
            r.sa[i] = h < halves ? ld_f32<COH>(g.a_scales + h / 2) : 0.0f;
        }
    }
}

// Stages the activation in LDS (smem, 16-byte aligned) from stage_load's
// registers: with NORM, RMSNorm + Q8_0 of g.x computed here
// (norm_quantize_prologue); otherwise the codes, and per half-block its
// (code sum, block scale), with half-blocks past 4 T loaded here. Ends with
// a barrier.
template <uint32_t T, int NORM, bool COH>
__device__ __forceinline__ void stage_store(const GemvArgs& g, uint4* smem, const StageLoads<T, NORM>& r) {
    const uint32_t K = g.k;
    uint4* s_codes = smem;                                     // K / 16 half-blocks of codes
    float2* s_ss = reinterpret_cast<float2*>(smem + K / 16);   // each half-block's (code sum, block scale)
    const uint32_t halves = K / 16, t = thread_index();
    if constexpr (NORM != 0) {
        float* s_red = reinterpret_cast<float*>(s_ss + K / 16);  // 257 floats
        norm_quantize_prologue<T, NORM == 2>(r, g.eps, K, s_codes, s_ss, s_red);
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t h = t + i * T;
            if (h < halves) {
                s_codes[h] = r.c[i];
                s_ss[h] = make_float2(static_cast<float>(byte_sum(r.c[i])), r.sa[i]);
            }
        }
        for (uint32_t h0 = t + 4 * T; h0 < halves; h0 += 4 * T) {
            uint4 c[4];
            float sa[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t h = h0 + i * T;
                c[i] = h < halves ? ld_u128<COH>(g.a_values + h) : make_uint4(0, 0, 0, 0);
                sa[i] = h < halves ? ld_f32<COH>(g.a_scales + h / 2) : 0.0f;
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t h = h0 + i * T;
                if (h < halves) {
                    s_codes[h] = c[i];
                    s_ss[h] = make_float2(static_cast<float>(byte_sum(c[i])), sa[i]);
                }
            }
        }
    }
    __syncthreads();
}

// stage_load then stage_store.
template <uint32_t T, int NORM, bool COH>
__device__ __forceinline__ void stage_activation(const GemvArgs& g, uint4* smem) {
    StageLoads<T, NORM> r;
    stage_load<T, NORM, COH>(g, r);
    stage_store<T, NORM, COH>(g, smem, r);
}

__device__ __forceinline__ const float2* staged_ss(const uint4* smem, uint32_t k) { return reinterpret_cast<const float2*>(smem + k / 16); }

}  // namespace vkml::gemv
