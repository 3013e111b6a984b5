// k_matmul.hip -- the int8 matrix product for many rows (prefill): the
// reference's shaders/matmul_dot.comp (src/ops/matmul.cpp:246-259), c = a b^T
// with a [M, K] Q8_0 activations (f32 scales) and b [N, K] quantized weights,
// on gfx950's matrix cores.
//
// Order (matmul_dot.comp:134-160). Each output is a sum over K's 32-value
// blocks in order: the block's exact integer dot product of the two codes,
// scaled in f32 and added to the output's accumulator,
//   q8_0 / q4_0: acc += float(sum) * (sa * sb)
//   q4_1 / q4_K: acc += sa * (float(sum) * sb + float(asum) * ob)
// (asum: the block's sum of a's codes; q4_K as its q4_1 form, scale
// f16(d sc) and offset f16(-dmin m) per 32 values, src/io/gguf.cpp:603-617).
// One v_mfma_i32_16x16x32_i8 computes the integer sums of one block for a
// 16 x 16 tile of outputs exactly, so the matrix cores do the dot products
// and the VALU applies the scales per block, in the reference's order.
//
// Mapping. A workgroup of four waves computes a tile of c, each wave 16 RT
// rows by 16 CT columns (RT x CT matrix instructions a block; 64 x 32 for
// large products, smaller tiles for short prompts so every SIMD gets work).
// Lane l of a wave holds, for a 16 x 16 instruction, a's row l % 16 and b's
// column l % 16 at the block's values 8 (l / 16) .. 8 (l / 16) + 7 (one
// 8-byte operand each), and gets the results for rows 4 (l / 16) .. + 3 of
// column l % 16. K runs in chunks of 8 blocks; for each chunk the
// workgroup stages every row's (scale, code sum) and every column's (scale,
// offset) per block in LDS, and the scaling reads four rows' values as one
// 16-byte word. The large-product kernel also stages the chunk's operands
// in LDS, copied with 16-byte loads a chunk ahead in registers (2x the
// kernel that loads each block's 8-byte operands from memory, whose waves
// spent twice their issue time waiting for them); the small tiles load
// operands straight from memory (L2 serves the reuse across workgroups).
// The scaling costs 4 VALU operations per output and block (the offset
// formats' six folded into four, as block_term says), and it bounds the
// kernel: a SIMD issues a wave64 f32 VALU instruction about every 4
// cycles (measured 33.7 T lane-operations a second for fma, 36.8 T for mul,
// 38.7 T for add over the GPU), so 4 operations per output and block cap
// the kernel near 9 T outputs x blocks a second, about 580 TOP/s of the
// int8 products (11.6% of the int8 peak); the matrix instructions are idle
// most of the time.
#include <algorithm>

#include "../../include/vkml_hip.h"
#include "device.hpp"
#include "internal.hpp"

using namespace vkml::dev;

namespace {

constexpr uint32_t kT = 256;      // four waves
typedef int v4i __attribute__((ext_vector_type(4)));

struct MatmulDotArgs {
    const uint8_t* a;     // [M, K] activation codes
    const float* a_scales;  // [M, K / 32]
    const uint8_t* b;     // weight codes (layout per format)
    const void* b_scales;  // per-block scales (q4_K: the 16-byte super-block headers)
    float* out;           // [M, N]
    uint32_t m, n, k;
    const float* residual;  // [M, N] added to each output, or null
};

// out[row, col] = v, or residual[row, col] + v (the binary add that
// follows the o and down projections, the same f32 sum).
__device__ __forceinline__ void store_out(const MatmulDotArgs& p, uint32_t row, uint32_t col, float v) {
    const uint64_t at = static_cast<uint64_t>(row) * p.n + col;
    p.out[at] = p.residual ? p.residual[at] + v : v;
}

__device__ __forceinline__ float f16_at(const void* p, uint64_t i) { return f16_bits_to_float(ldg(static_cast<const uint16_t*>(p) + i)); }

// Four Q4_0 values as signed bytes, the low (shift 0) or high (shift 4)
// nibbles of a word minus 8 (matmul_dot.comp:71-73).
__device__ __forceinline__ uint32_t q4_signed(uint32_t word, uint32_t shift) {
    return (((word >> shift) & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u;
}

// Column n's operand for block blk: its 8 codes at values 8 g .. 8 g + 7 of
// the block, as int8 (q4: codes 0 .. 15, or minus 8 for q4_0).
template <int FMT>
__device__ __forceinline__ long b_codes(const MatmulDotArgs& p, uint32_t n, uint32_t blk, uint32_t g) {
    uint32_t lo, hi;
    if constexpr (FMT == VKML_Q8_0) {
        const uint2 w = ldg(reinterpret_cast<const uint2*>(p.b + static_cast<uint64_t>(n) * p.k + blk * 32 + 8 * g));
        lo = w.x;
        hi = w.y;
    } else if constexpr (FMT == VKML_Q4_K) {
        // sub-block j = blk % 8 of super-block blk / 8: low (j even) or high
        // nibbles of bytes 32 (j / 2) .. of its 128
        const uint32_t j = blk % 8, sb = blk / 8;
        const uint2 w = ldg(reinterpret_cast<const uint2*>(p.b + static_cast<uint64_t>(n) * (p.k / 2) + sb * 128 + 32 * (j / 2) + 8 * g));
        const uint32_t sh = 4 * (j % 2);
        lo = (w.x >> sh) & 0x0F0F0F0Fu;
        hi = (w.y >> sh) & 0x0F0F0F0Fu;
    } else {
        // QuantizedMatrix q4 words: word w' of the block holds values 8 w' .. 8 w' + 7,
        // low nibbles the first four, high the last four
        const uint32_t q = ldg(reinterpret_cast<const uint32_t*>(p.b + static_cast<uint64_t>(n) * (p.k / 2) + blk * 16 + 4 * g));
        if constexpr (FMT == VKML_Q4_0) {
            lo = q4_signed(q, 0);
            hi = q4_signed(q, 4);
        } else {
            lo = q & 0x0F0F0F0Fu;
            hi = (q >> 4) & 0x0F0F0F0Fu;
        }
    }
    return static_cast<long>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Column n's scale and offset for block blk (q8_0 / q4_0: offset unused).
template <int FMT, bool F16S>
__device__ __forceinline__ void b_block_scale(const MatmulDotArgs& p, uint32_t n, uint32_t blk, float& s, float& o) {
    const uint64_t block = static_cast<uint64_t>(n) * (p.k / 32) + blk;
    o = 0.0f;
    if constexpr (FMT == VKML_Q8_0 || FMT == VKML_Q4_0) {
        s = F16S ? f16_at(p.b_scales, block) : ldg(static_cast<const float*>(p.b_scales) + block);
    } else if constexpr (F16S) {
        const uint32_t so = ldg(static_cast<const uint32_t*>(p.b_scales) + block);  // f16 scale | f16 offset << 16
        s = f16_bits_to_float(so & 0xFFFFu);
        o = f16_bits_to_float(so >> 16);
    } else {
        const float2 so = ldg(static_cast<const float2*>(p.b_scales) + block);
        s = so.x;
        o = so.y;
    }
}

// q4_K: sub-block j's scale f16(d sc_j) and offset f16(-dmin m_j) from the
// super-block's 16-byte header (gguf.cpp:603-617).
__device__ __forceinline__ void q4k_block_scale(const uint4& h, uint32_t j, float& s, float& o) {
    const uint32_t b = 8 * (j % 4);
    const uint32_t b1 = (h.y >> b) & 0xFFu, b2 = (h.z >> b) & 0xFFu, b3 = (h.w >> b) & 0xFFu;
    const uint32_t sc = j < 4 ? b1 & 63u : (b3 & 15u) | ((b1 >> 6) << 4);
    const uint32_t mn = j < 4 ? b2 & 63u : (b3 >> 4) | ((b2 >> 6) << 4);
    const _Float16 d = __builtin_bit_cast(_Float16, static_cast<uint16_t>(h.x & 0xFFFFu));
    const _Float16 nd = -__builtin_bit_cast(_Float16, static_cast<uint16_t>(h.x >> 16));
    s = static_cast<float>(d * static_cast<_Float16>(static_cast<uint16_t>(sc)));
    o = static_cast<float>(nd * static_cast<_Float16>(static_cast<uint16_t>(mn)));
}

constexpr uint32_t kChunk = 8;  // blocks of K a chunk (a q4_K super-block)

// The offset formats with f16 scales (q4_K, q4_1 with f16 scales) take the
// reference's six scaling operations, cvt, mul, mul, add, mul, add, as
// four: fma, fma, mul, add, with every result bit for bit the same.
//  - The matrix instruction starts its accumulator at the int32 bits of the
//    f32 1.5 * 2^23, so each block sum comes out as the bits of the f32
//    1.5 * 2^23 + sum, exactly (|sum| <= 32 * 128 * 15 < 2^22). Then
//    fma(that, sb, -1.5 * 2^23 * sb) forms the exact sum * sb and rounds it
//    once: float(sum) * sb, with no conversion. -1.5 * 2^23 * sb is exact
//    because sb is an f16 value (11 significant bits, 13 after the 3).
//  - asum * ob is exact (|asum| <= 32 * 128 = 2^12 has at most 12
//    significant bits, ob is an f16 value, and the smallest nonzero
//    product, 2^-24, is a normal f32), so fma(asum, ob, x) rounds x +
//    asum * ob once, as the reference's add of the rounded product does.
// Signs of zero can differ in the intermediate (an exact zero sum is +0,
// not -0 * sb), but no accumulator starting at +0 ever sees the
// difference: +0 + -0 is +0, and a nonzero accumulator ignores both.
constexpr int32_t kSumBiasBits = 0x4B400000;  // the f32 1.5 * 2^23
constexpr float kSumBias = 12582912.0f;

template <int FMT, bool F16S>
constexpr bool kFoldScaling = FMT == VKML_Q4_K || (FMT == VKML_Q4_1 && F16S);

template <int FMT, bool F16S>
__device__ __forceinline__ v4i sum_start() {
    constexpr int32_t b = kFoldScaling<FMT, F16S> ? kSumBiasBits : 0;
    return v4i{b, b, b, b};
}

// One output's contribution of one block, sa (sum sb + asum ob) or
// sum (sa sb) (matmul_dot.comp:155-160), from the matrix instruction's
// result d (biased where the scaling folds; nsb = -1.5 * 2^23 * sb).
template <int FMT, bool F16S>
__device__ __forceinline__ float block_term(int32_t d, float sa, float asum, float sb, float nsb, float ob) {
#pragma clang fp contract(off)
    if constexpr (kFoldScaling<FMT, F16S>) {
        const float x = __builtin_fmaf(__builtin_bit_cast(float, d), sb, nsb);
        return sa * __builtin_fmaf(asum, ob, x);
    } else if constexpr (FMT == VKML_Q4_1 || FMT == VKML_Q4_K) {
        return sa * (static_cast<float>(d) * sb + asum * ob);
    } else {
        return static_cast<float>(d) * (sa * sb);
    }
}

// One kernel per per-wave tile: RT row tiles of 16 by CT column tiles of
// 16; a workgroup's four waves take 4 CT column tiles side by side, so its
// tile is 16 RT x 64 CT.
template <int FMT, bool F16S, int RT, int CT>
__global__ void __launch_bounds__(kT) k_matmul_dot(MatmulDotArgs p) {
#pragma clang fp contract(off)
    constexpr bool kOffset = FMT == VKML_Q4_1 || FMT == VKML_Q4_K;
    constexpr uint32_t TM = 16 * RT, TN = 64 * CT;
    // Per chunk, double-buffered: rows' scales and code sums, columns'
    // scales and offsets, [block of the chunk][row or column].
    __shared__ __align__(16) float s_sa[2][kChunk][TM];
    __shared__ __align__(16) float s_asum[2][kChunk][kOffset ? TM : 4];
    __shared__ float s_sb[2][kChunk][TN];
    __shared__ float s_ob[2][kChunk][kOffset ? TN : 1];
    const uint32_t t = thread_index(), lane = t % kWave, wave = t / kWave;
    const uint32_t g = lane / 16, li = lane % 16;
    const uint32_t row0 = blockIdx.y * TM, col0 = blockIdx.x * TN;
    const uint32_t blocks = p.k / 32;
    const uint8_t* arow[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r) arow[r] = p.a + static_cast<uint64_t>(min(row0 + 16 * r + li, p.m - 1)) * p.k + 8 * g;
    uint32_t bcol[CT];
#pragma unroll
    for (int c = 0; c < CT; ++c) bcol[c] = min(col0 + 16 * CT * wave + 16 * c + li, p.n - 1);
    float acc[RT][CT][4];
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int c = 0; c < CT; ++c)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[r][c][i] = 0.0f;

    for (uint32_t c0 = 0, buf = 0; c0 < blocks; c0 += kChunk, buf ^= 1) {
        // Stage the chunk's statistics: TM rows x 8 blocks, and TN columns x
        // 8 blocks (a column's four blocks a thread).
#pragma unroll
        for (uint32_t e = t; e < TM * kChunk; e += kT) {
            const uint32_t r = e % TM, b = e / TM, blk = c0 + b;
            if (blk < blocks) {
                const uint32_t row = min(row0 + r, p.m - 1);
                s_sa[buf][b][r] = ldg(p.a_scales + static_cast<uint64_t>(row) * blocks + blk);
                if constexpr (kOffset) {
                    const uint4* codes = reinterpret_cast<const uint4*>(p.a + static_cast<uint64_t>(row) * p.k + blk * 32);
                    s_asum[buf][b][r] = static_cast<float>(byte_sum(ldg(codes)) + byte_sum(ldg(codes + 1)));
                }
            }
        }
#pragma unroll
        for (uint32_t e = t; e < TN * 2; e += kT) {
            const uint32_t cl = e / 2, b0 = 4 * (e % 2), col = min(col0 + cl, p.n - 1);
            if constexpr (FMT == VKML_Q4_K) {
                const uint4 h = ldg(reinterpret_cast<const uint4*>(static_cast<const uint8_t*>(p.b_scales) +
                                                                   (static_cast<uint64_t>(col) * (p.k / 256) + c0 / 8) * 16));
#pragma unroll
                for (uint32_t b = 0; b < 4; ++b) q4k_block_scale(h, b0 + b, s_sb[buf][b0 + b][cl], s_ob[buf][b0 + b][cl]);
            } else {
#pragma unroll
                for (uint32_t b = 0; b < 4; ++b) {
                    if (c0 + b0 + b < blocks) {
                        float s, o;
                        b_block_scale<FMT, F16S>(p, col, c0 + b0 + b, s, o);
                        s_sb[buf][b0 + b][cl] = s;
                        if constexpr (kOffset) s_ob[buf][b0 + b][cl] = o;
                    }
                }
            }
        }
        __syncthreads();  // the chunk's statistics are staged (the other buffer's readers finished a chunk ago)
#pragma unroll
        for (uint32_t b = 0; b < kChunk; ++b) {
            const uint32_t blk = c0 + b;
            if (blk >= blocks) break;
            long av[RT], bv[CT];
#pragma unroll
            for (int r = 0; r < RT; ++r) av[r] = static_cast<long>(__builtin_bit_cast(uint64_t, ldg(reinterpret_cast<const uint2*>(arow[r] + blk * 32))));
#pragma unroll
            for (int c = 0; c < CT; ++c) bv[c] = b_codes<FMT>(p, bcol[c], blk, g);
            float sb[CT], nsb[CT], ob[CT];
#pragma unroll
            for (int c = 0; c < CT; ++c) {
                sb[c] = s_sb[buf][b][16 * CT * wave + 16 * c + li];
                nsb[c] = -kSumBias * sb[c];
                ob[c] = 0.0f;
                if constexpr (kOffset) ob[c] = s_ob[buf][b][16 * CT * wave + 16 * c + li];
            }
#pragma unroll
            for (int r = 0; r < RT; ++r) {
                const float4 sa4 = *reinterpret_cast<const float4*>(&s_sa[buf][b][16 * r + 4 * g]);
                float4 as4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if constexpr (kOffset) as4 = *reinterpret_cast<const float4*>(&s_asum[buf][b][16 * r + 4 * g]);
                const float sa[4] = {sa4.x, sa4.y, sa4.z, sa4.w}, asum[4] = {as4.x, as4.y, as4.z, as4.w};
#pragma unroll
                for (int c = 0; c < CT; ++c) {
                    const v4i d = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[r], bv[c], sum_start<FMT, F16S>(), 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[r][c][i] += block_term<FMT, F16S>(d[i], sa[i], asum[i], sb[c], nsb[c], ob[c]);
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int c = 0; c < CT; ++c) {
            const uint32_t col = col0 + 16 * CT * wave + 16 * c + li;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t row = row0 + 16 * r + 4 * g + i;
                if (row < p.m && col < p.n) store_out(p, row, col, acc[r][c][i]);
            }
        }
}

// The 16 RT x 128 tile with its operands staged in LDS: per 8-block chunk
// the workgroup copies the chunk's A rows (16 RT x 256 bytes) and B columns
// (128 x 128 bytes, 256 for q8_0) with 16-byte loads, a chunk ahead in
// registers, and the matrix instructions read their operands from LDS. Each
// staging thread's A bytes are whole blocks of one row (two at RT = 4, one
// below; at RT = 1 half the threads stage A), so it also sums their codes.
template <int FMT, bool F16S, int RT>
struct StagedChunk {
    static constexpr bool kOffset = FMT == VKML_Q4_1 || FMT == VKML_Q4_K;
    static constexpr uint32_t TM = 16 * RT;                   // rows of the tile
    static constexpr uint32_t kABlocks = RT >= 2 ? RT / 2 : 1;  // a staging thread's A blocks (of one row)
    static constexpr uint32_t kAThreads = TM * kChunk / kABlocks;  // threads that stage A
    static constexpr uint32_t kBBytes = FMT == VKML_Q8_0 ? 256 : 128;  // a column's bytes a chunk
    static constexpr uint32_t kAStride = 272, kBStride = kBBytes + 16;  // padded rows: no bank conflicts
    static constexpr uint32_t kBLoads = kBBytes * 128 / 16 / kT;        // 16-byte B loads a thread
    uint4 a[2 * kABlocks];
    uint4 b[kBLoads];
    float sa[kABlocks];
    uint4 header;
    float s[4], o[4];
};

template <int FMT, bool F16S, int RT>
struct StagedLds {
    static constexpr bool kOffset = FMT == VKML_Q4_1 || FMT == VKML_Q4_K;
    alignas(16) uint8_t a[16 * RT * StagedChunk<FMT, F16S, RT>::kAStride];
    alignas(16) uint8_t b[128 * StagedChunk<FMT, F16S, RT>::kBStride];
    alignas(16) float sa[kChunk][16 * RT];
    alignas(16) float asum[kChunk][kOffset ? 16 * RT : 4];
    float sb[kChunk][128];
    float ob[kChunk][kOffset ? 128 : 1];
};

template <int FMT, bool F16S, int RT>
__device__ __forceinline__ void staged_load(const MatmulDotArgs& p, uint32_t t, uint32_t c0, uint32_t row0, uint32_t col0,
                                            StagedChunk<FMT, F16S, RT>& r) {
    using S = StagedChunk<FMT, F16S, RT>;
    constexpr uint32_t AB = S::kABlocks, kPerRow = kChunk / AB;  // threads a row
    const uint32_t blocks = p.k / 32;
    if (S::kAThreads == kT || t < S::kAThreads) {
        // A: row t / kPerRow, blocks AB (t % kPerRow) .. of the chunk
        const uint32_t row = min(row0 + t / kPerRow, p.m - 1);
#pragma unroll
        for (uint32_t h = 0; h < AB; ++h) {
            const uint32_t b = AB * (t % kPerRow) + h, blk = min(c0 + b, blocks - 1);
            const uint4* src = reinterpret_cast<const uint4*>(p.a + static_cast<uint64_t>(row) * p.k + blk * 32);
            r.a[2 * h] = ldg(src);
            r.a[2 * h + 1] = ldg(src + 1);
            r.sa[h] = ldg(p.a_scales + static_cast<uint64_t>(row) * blocks + blk);
        }
    }
    // B: 16-byte pieces of the columns' chunk bytes, consecutive threads along a column
#pragma unroll
    for (uint32_t u = 0; u < S::kBLoads; ++u) {
        const uint32_t e = t + kT * u, cl = e / (S::kBBytes / 16), piece = e % (S::kBBytes / 16);
        const uint32_t col = min(col0 + cl, p.n - 1);
        const uint8_t* src;
        if constexpr (FMT == VKML_Q8_0) {
            const uint32_t blk = min(c0 + piece / 2, blocks - 1);
            src = p.b + static_cast<uint64_t>(col) * p.k + blk * 32 + 16 * (piece % 2);
        } else if constexpr (FMT == VKML_Q4_K) {
            src = p.b + static_cast<uint64_t>(col) * (p.k / 2) + (c0 / 8) * 128 + 16 * piece;
        } else {
            const uint32_t blk = min(c0 + piece, blocks - 1);
            src = p.b + static_cast<uint64_t>(col) * (p.k / 2) + blk * 16;
        }
        r.b[u] = ldg(reinterpret_cast<const uint4*>(src));
    }
    {
        const uint32_t col = min(col0 + t / 2, p.n - 1), b0 = 4 * (t % 2);
        if constexpr (FMT == VKML_Q4_K) {
            r.header = ldg(reinterpret_cast<const uint4*>(static_cast<const uint8_t*>(p.b_scales) +
                                                          (static_cast<uint64_t>(col) * (p.k / 256) + c0 / 8) * 16));
        } else {
#pragma unroll
            for (uint32_t b = 0; b < 4; ++b) b_block_scale<FMT, F16S>(p, col, min(c0 + b0 + b, blocks - 1), r.s[b], r.o[b]);
        }
    }
}

template <int FMT, bool F16S, int RT>
__device__ __forceinline__ void staged_store(const StagedChunk<FMT, F16S, RT>& r, uint32_t t, StagedLds<FMT, F16S, RT>& l) {
    using S = StagedChunk<FMT, F16S, RT>;
    constexpr bool kOffset = S::kOffset;
    constexpr uint32_t AB = S::kABlocks, kPerRow = kChunk / AB;
    if (S::kAThreads == kT || t < S::kAThreads) {
        const uint32_t row = t / kPerRow;
#pragma unroll
        for (uint32_t i = 0; i < 2 * AB; ++i)
            *reinterpret_cast<uint4*>(l.a + row * S::kAStride + (t % kPerRow) * 32 * AB + 16 * i) = r.a[i];
#pragma unroll
        for (uint32_t h = 0; h < AB; ++h) {
            const uint32_t b = AB * (t % kPerRow) + h;
            l.sa[b][row] = r.sa[h];
            if constexpr (kOffset) l.asum[b][row] = static_cast<float>(byte_sum(r.a[2 * h]) + byte_sum(r.a[2 * h + 1]));
        }
    }
#pragma unroll
    for (uint32_t u = 0; u < S::kBLoads; ++u) {
        const uint32_t e = t + kT * u, cl = e / (S::kBBytes / 16), piece = e % (S::kBBytes / 16);
        *reinterpret_cast<uint4*>(l.b + cl * S::kBStride + 16 * piece) = r.b[u];
    }
    const uint32_t cl = t / 2, b0 = 4 * (t % 2);
#pragma unroll
    for (uint32_t b = 0; b < 4; ++b) {
        float sv = r.s[b], ov = r.o[b];
        if constexpr (FMT == VKML_Q4_K) q4k_block_scale(r.header, b0 + b, sv, ov);
        l.sb[b0 + b][cl] = sv;
        if constexpr (kOffset) l.ob[b0 + b][cl] = ov;
    }
}

// Column cl's operand for block b of the staged chunk (as b_codes).
template <int FMT, bool F16S, int RT>
__device__ __forceinline__ long staged_b(const StagedLds<FMT, F16S, RT>& l, uint32_t cl, uint32_t b, uint32_t g) {
    using S = StagedChunk<FMT, F16S, RT>;
    const uint8_t* col = l.b + cl * S::kBStride;
    uint32_t lo, hi;
    if constexpr (FMT == VKML_Q8_0) {
        const uint2 w = *reinterpret_cast<const uint2*>(col + b * 32 + 8 * g);
        lo = w.x;
        hi = w.y;
    } else if constexpr (FMT == VKML_Q4_K) {
        const uint2 w = *reinterpret_cast<const uint2*>(col + 32 * (b / 2) + 8 * g);
        const uint32_t sh = 4 * (b % 2);
        lo = (w.x >> sh) & 0x0F0F0F0Fu;
        hi = (w.y >> sh) & 0x0F0F0F0Fu;
    } else {
        const uint32_t q = *reinterpret_cast<const uint32_t*>(col + b * 16 + 4 * g);
        if constexpr (FMT == VKML_Q4_0) {
            lo = q4_signed(q, 0);
            hi = q4_signed(q, 4);
        } else {
            lo = q & 0x0F0F0F0Fu;
            hi = (q >> 4) & 0x0F0F0F0Fu;
        }
    }
    return static_cast<long>((static_cast<uint64_t>(hi) << 32) | lo);
}

template <int FMT, bool F16S, int RT>
__global__ void __launch_bounds__(kT) k_matmul_dot_staged(MatmulDotArgs p) {
#pragma clang fp contract(off)
    using S = StagedChunk<FMT, F16S, RT>;
    constexpr bool kOffset = S::kOffset;
    __shared__ StagedLds<FMT, F16S, RT> l;
    const uint32_t t = thread_index(), lane = t % kWave, wave = t / kWave;
    const uint32_t g = lane / 16, li = lane % 16;
    const uint32_t row0 = blockIdx.y * S::TM, col0 = blockIdx.x * 128;
    const uint32_t blocks = p.k / 32;
    float acc[RT][2][4];
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[r][c][i] = 0.0f;
    // A block's matrix instructions (RT x 2 of them) into d.
    const auto sums = [&](uint32_t b, v4i (&d)[RT][2]) {
        long av[RT], bv[2];
#pragma unroll
        for (int r = 0; r < RT; ++r) av[r] = *reinterpret_cast<const long*>(l.a + (16 * r + li) * S::kAStride + b * 32 + 8 * g);
#pragma unroll
        for (int c = 0; c < 2; ++c) bv[c] = staged_b<FMT, F16S, RT>(l, 32 * wave + 16 * c + li, b, g);
#pragma unroll
        for (int r = 0; r < RT; ++r)
#pragma unroll
            for (int c = 0; c < 2; ++c) d[r][c] = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[r], bv[c], sum_start<FMT, F16S>(), 0, 0, 0);
    };
    // A block's scaling of d into the accumulators, in the reference's order.
    const auto scale = [&](uint32_t b, const v4i (&d)[RT][2]) {
        float sb[2], nsb[2], ob[2];
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            sb[c] = l.sb[b][32 * wave + 16 * c + li];
            nsb[c] = -kSumBias * sb[c];
            ob[c] = 0.0f;
            if constexpr (kOffset) ob[c] = l.ob[b][32 * wave + 16 * c + li];
        }
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            const float4 sa4 = *reinterpret_cast<const float4*>(&l.sa[b][16 * r + 4 * g]);
            float4 as4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if constexpr (kOffset) as4 = *reinterpret_cast<const float4*>(&l.asum[b][16 * r + 4 * g]);
            const float sa[4] = {sa4.x, sa4.y, sa4.z, sa4.w}, asum[4] = {as4.x, as4.y, as4.z, as4.w};
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[r][c][i] += block_term<FMT, F16S>(d[r][c][i], sa[i], asum[i], sb[c], nsb[c], ob[c]);
        }
    };
    StagedChunk<FMT, F16S, RT> next;
    staged_load<FMT, F16S, RT>(p, t, 0, row0, col0, next);
    for (uint32_t c0 = 0; c0 < blocks; c0 += kChunk) {
        __syncthreads();  // the last chunk's readers are done
        staged_store<FMT, F16S, RT>(next, t, l);
        __syncthreads();
        if (c0 + kChunk < blocks) staged_load<FMT, F16S, RT>(p, t, c0 + kChunk, row0, col0, next);  // in flight meanwhile
#pragma unroll
        for (uint32_t b = 0; b < kChunk; ++b) {
            if (c0 + b >= blocks) break;
            v4i d[RT][2];
            sums(b, d);
            scale(b, d);
        }
    }
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const uint32_t col = col0 + 32 * wave + 16 * c + li;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t row = row0 + 16 * r + 4 * g + i;
                if (row < p.m && col < p.n) store_out(p, row, col, acc[r][c][i]);
            }
        }
}

template <int FMT, bool F16S, int RT, int CT>
void launch_tiles(const MatmulDotArgs& p) {
    const dim3 grid((p.n + 64 * CT - 1) / (64 * CT), (p.m + 16 * RT - 1) / (16 * RT));
    hipLaunchKernelGGL((k_matmul_dot<FMT, F16S, RT, CT>), grid, dim3(kT), 0, vkml::abi::stream(), p);
}

// The 64 x 128 tile with its operands staged in LDS (2x the direct-load
// kernel at large prompts) wherever it gives every CU about four
// workgroups; below that the 32 x 128 staged tile, wherever it gives the
// SIMDs two waves each; below that the 16 x 128 staged tile, wherever the
// 32-row one would give them half a wave; below that, the largest
// direct-load tile that still gives them about two waves each. (Measured:
// the staged tiles win from 512 of their waves on; a 512-token cfg5
// prompt's projections take 19.1 ms with 32 x 128 tiles against 23.3 ms
// with 64 x 128, a 4096-token prompt's 116-124 ms either way, the 64 x 128
// tile ahead in most runs; cfg3's 512-token q|k|v, o and down, one to one
// and a half 32-row waves a SIMD, take 25.8, 20.6 and 74.0 us with 16-row
// tiles against 29.9, 24.4 and 89.0 us; at 128 rows x 14336 columns the
// 32 x 32 direct tile beats 64 x 32 with half the waves and 32 x 16 with
// twice as many.)
template <int FMT, bool F16S>
void launch(const MatmulDotArgs& p) {
    const auto waves = [&](uint64_t rt, uint64_t ct) { return ((p.m + 16 * rt - 1) / (16 * rt)) * ((p.n + 16 * ct - 1) / (16 * ct)); };
    constexpr uint64_t kEnough = 1792;  // 256 CUs x 4 SIMDs x 1.75
    if (waves(4, 2) >= 4096) {
        const dim3 grid((p.n + 127) / 128, (p.m + 63) / 64);
        hipLaunchKernelGGL((k_matmul_dot_staged<FMT, F16S, 4>), grid, dim3(kT), 0, vkml::abi::stream(), p);
    } else if (waves(2, 2) >= 2048) {
        const dim3 grid((p.n + 127) / 128, (p.m + 31) / 32);
        hipLaunchKernelGGL((k_matmul_dot_staged<FMT, F16S, 2>), grid, dim3(kT), 0, vkml::abi::stream(), p);
    } else if (waves(2, 2) >= 512) {
        const dim3 grid((p.n + 127) / 128, (p.m + 15) / 16);
        hipLaunchKernelGGL((k_matmul_dot_staged<FMT, F16S, 1>), grid, dim3(kT), 0, vkml::abi::stream(), p);
    } else if (waves(2, 2) >= kEnough) launch_tiles<FMT, F16S, 2, 2>(p);
    else if (waves(2, 1) >= kEnough) launch_tiles<FMT, F16S, 2, 1>(p);
    else launch_tiles<FMT, F16S, 1, 1>(p);
}

int matmul_dot_common(const char* what, const vkml_gemv_dot_params* p, const void* a_values, const void* b_values, float* out,
                      const void* b_scales, const float* a_scales, const float* residual) {
    VKML_REQUIRE_INIT();
    const std::string name = what;
    VKML_CHECK_ARG(p, name + ": null params");
    VKML_CHECK_ARG(p->b_type == VKML_Q8_0 || p->b_type == VKML_Q4_0 || p->b_type == VKML_Q4_1 || p->b_type == VKML_Q4_K,
                   name + ": weights must be q8_0, q4_0, q4_1 or q4_K, got type " + std::to_string(p->b_type));
    VKML_CHECK_ARG(p->b_type == VKML_Q4_K || p->scale_type == VKML_F16 || p->scale_type == VKML_F32, name + ": scales must be f16 or f32");
    const uint32_t unit = p->b_type == VKML_Q4_K ? 256 : 32;
    VKML_CHECK_ARG(p->k > 0 && p->k % unit == 0, name + ": k = " + std::to_string(p->k) + " must be a positive multiple of " + std::to_string(unit));
    if (p->m == 0 || p->n == 0) return VKML_OK;
    VKML_CHECK_ARG(a_values && b_values && out && b_scales && a_scales, name + ": null buffer");
    const MatmulDotArgs args{static_cast<const uint8_t*>(a_values), a_scales, static_cast<const uint8_t*>(b_values), b_scales, out,
                             p->m, p->n, p->k, residual};
    vkml::abi::ProfileScope prof(what);
    const bool f16 = p->scale_type == VKML_F16;
    switch (p->b_type) {
        case VKML_Q8_0: f16 ? launch<VKML_Q8_0, true>(args) : launch<VKML_Q8_0, false>(args); break;
        case VKML_Q4_0: f16 ? launch<VKML_Q4_0, true>(args) : launch<VKML_Q4_0, false>(args); break;
        case VKML_Q4_1: f16 ? launch<VKML_Q4_1, true>(args) : launch<VKML_Q4_1, false>(args); break;
        default: launch<VKML_Q4_K, true>(args); break;
    }
    return vkml::abi::check_launch(what);
}

}  // namespace

extern "C" {

int vkml_matmul_dot(const vkml_gemv_dot_params* p, const void* a_values, const void* b_values, float* out, const void* b_scales,
                    const float* a_scales) {
    return matmul_dot_common("matmul_dot", p, a_values, b_values, out, b_scales, a_scales, nullptr);
}

int vkml_matmul_dot_add(const vkml_gemv_dot_params* p, const void* a_values, const void* b_values, float* out, const void* b_scales,
                        const float* a_scales, const float* residual) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(residual || (p && (p->m == 0 || p->n == 0)), "matmul_dot_add: null residual");
    return matmul_dot_common("matmul_dot_add", p, a_values, b_values, out, b_scales, a_scales, residual);
}

}  // extern "C"
