// k_prompt_fast.hip -- a prompt's causal attention on the matrix cores: the
// tolerance form of the reference's chunked q.k^T, softmax and probs.v
// (src/ops/attention.cpp:127-138,205-226), as an option beside the exact
// path (matmul scores, softmax, matmul probs.v in the reference's order).
//
// Not the reference's order of f32 operations: every product is exact (f16
// x f16 in the matrix unit, q and the probabilities split into two f16
// terms) and every sum accumulates in f32, in the matrix unit's order, with
// the softmax taken online over blocks of keys. The results are those of
// f32 attention to within f32 rounding.
//
// A workgroup takes 16 queries of one KV head's four query heads, a wave a
// head, and walks the keys its queries see in blocks of 32:
//   - scores S^T [32 keys x 16 queries] = K . Q^T by
//     v_mfma_f32_16x16x32_f16, K copied into LDS a block ahead by
//     global_load_lds (each row's 16-byte pieces swizzled so that the 16
//     rows of an operand read hit different banks), q (scaled into log2
//     units) as hi + lo f16 terms;
//   - per query (a lane column) the block's max and the running (max, sum),
//     the accumulated output rescaled by 2^(m_old - m_new);
//   - O^T [hd x 16 queries] += V^T . P^T, V loaded a block ahead into
//     registers and written into LDS transposed, [dim][key], so that a
//     lane's operand is two 8-byte reads; P^T straight from the score
//     tile's registers (the accumulator layout of S^T is the B operand's
//     of P^T, keys permuted alike in V^T's A operand). In O^T a query is a
//     lane column, as in S^T, so its rescale needs no exchange between
//     lanes.
// The output is written [query, head, hd]: the o projection's input rows.
#include <algorithm>
#include <string>

#include "attend_fast.hpp"
#include "device.hpp"
#include "internal.hpp"

using namespace vkml::dev;
using vkml::attend::kThreads;
using vkml::attend_fast::f32x4;
using vkml::attend_fast::half8;
using vkml::attend_fast::kLog2e;

namespace {

constexpr uint32_t kQueries = 16;  // queries a workgroup
constexpr uint32_t kBlock = 32;    // keys a block
constexpr uint32_t kHeads = 4;     // query heads a workgroup (a wave each)

struct PromptArgs {
    const float* q;  // [heads, t, hd] f32
    const void* k_cache;
    const void* v_cache;  // [kv_heads, capacity, hd] f16
    float* out;           // [t, heads, hd] f32
    uint32_t heads, kv_heads, group, capacity, t, first;
    float scale, softcap;
};

// A block's tiles in LDS. K row-major, each row's 16-byte pieces swizzled
// (piece p of key row r at p ^ (r % pieces)) so that the 16 rows a score
// operand read takes hit different banks. V transposed, [dim][key] with
// rows padded to 72 bytes, so that a lane's four keys of one dim are one
// 8-byte read and the 16 dims of a read hit different banks.
template <int HD>
struct PromptTiles {
    static constexpr uint32_t kPieces = HD * 2 / 16;  // 16-byte pieces a key row
    static constexpr uint32_t kVtStride = kBlock + 4;  // f16 a V^T row
    alignas(16) uint8_t k[kBlock * HD * 2];
    alignas(16) _Float16 vt[HD * kVtStride];
};

// V of the next block in registers (8 dims of one key a 16-byte piece).
template <int HD>
struct VRegs {
    static constexpr uint32_t kLoads = kBlock * HD * 2 / 16 / kThreads;
    uint4 v[kLoads];
};

// Key block kb's K rows into LDS (global_load_lds, swizzled) and its V rows
// into registers. Keys past `keys` re-read the last.
template <int HD>
__device__ __forceinline__ void load_block(const PromptArgs& a, uint32_t kvh, uint32_t kb, uint32_t keys, PromptTiles<HD>& tl, VRegs<HD>& vr) {
    using T = PromptTiles<HD>;
    constexpr uint32_t RB = HD * 2;
    const uint32_t t = thread_index(), wave_first = t - t % kWave;
    const uint64_t row0 = static_cast<uint64_t>(kvh) * a.capacity;
    const auto* kc = static_cast<const uint8_t*>(a.k_cache);
    const auto* vc = static_cast<const uint8_t*>(a.v_cache);
#pragma unroll
    for (uint32_t i = 0; i < VRegs<HD>::kLoads; ++i) {
        const uint32_t u = i * kThreads + t, rr = u / T::kPieces, piece = u % T::kPieces;
        const uint64_t row = row0 + min(kb * kBlock + rr, keys - 1);
        vkml::attend::load_to_lds16(kc + row * RB + 16 * (piece ^ (rr % T::kPieces)), tl.k + 16 * (i * kThreads + wave_first));
        vr.v[i] = ldg(reinterpret_cast<const uint4*>(vc + row * RB + 16 * piece));
    }
}

// The block's V from registers into its V^T tile.
template <int HD>
__device__ __forceinline__ void store_vt(const VRegs<HD>& vr, PromptTiles<HD>& tl) {
    using T = PromptTiles<HD>;
    const uint32_t t = thread_index();
#pragma unroll
    for (uint32_t i = 0; i < VRegs<HD>::kLoads; ++i) {
        const uint32_t u = i * kThreads + t, key = u / T::kPieces, d0 = 8 * (u % T::kPieces);
        const half8 x = __builtin_bit_cast(half8, vr.v[i]);
#pragma unroll
        for (int e = 0; e < 8; ++e) tl.vt[(d0 + e) * T::kVtStride + key] = x[e];
    }
}

template <int HD>
__global__ void __launch_bounds__(kThreads) k_attend_prompt_fast(PromptArgs a) {
    using T = PromptTiles<HD>;
    __shared__ T s_t[2];
    constexpr int kSteps = HD / 32;
    const uint32_t t = thread_index(), w = t / kWave, l = t % kWave, j = l % 16, g = l / 16;
    // Workgroup L: (KV head, head quad) set L % sets, query tile from the
    // last down. Workgroups are dealt to the 8 XCDs round-robin, so with 8
    // (or a multiple of 8) sets each XCD serves the same KV heads and their
    // K and V stay in its L2 (a KV head's 4096 keys are 2 MiB); the tiles
    // whose queries see the most keys go first.
    const uint32_t quads = a.group / kHeads, sets = a.kv_heads * quads, tiles = (a.t + kQueries - 1) / kQueries;
    const uint32_t set = blockIdx.x % sets, tile = tiles - 1 - blockIdx.x / sets;
    const uint32_t kvh = set / quads, h = kvh * a.group + (set % quads) * kHeads + w;
    const uint32_t q0 = tile * kQueries;
    const uint32_t qi = q0 + j;                                      // the lane's query
    const bool qlive = qi < a.t;
    const uint32_t qpos = a.first + min(qi, a.t - 1);                // its position: keys 0 .. qpos
    const uint32_t keys = a.first + min(q0 + kQueries, a.t);         // keys the workgroup's queries see
    const uint32_t blocks = (keys + kBlock - 1) / kBlock;
    const bool cap = a.softcap > 0.0f;

    VRegs<HD> vr;
    load_block<HD>(a, kvh, 0, keys, s_t[0], vr);
    // q of the lane's query, scaled (in log2 units without a soft cap), as hi + lo f16
    half8 qh[kSteps], ql[kSteps];
    {
        const float qs = cap ? a.scale : a.scale * kLog2e;
        const float* qp = a.q + (static_cast<uint64_t>(h) * a.t + min(qi, a.t - 1)) * HD + 8 * g;
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            const float4 x0 = ldg(reinterpret_cast<const float4*>(qp + 32 * s));
            const float4 x1 = ldg(reinterpret_cast<const float4*>(qp + 32 * s + 4));
            const float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                // The f32 product through an empty asm: both terms come from
                // this one value. Otherwise the compiler folds f16(x qs) into
                // one rounding (v_fma_mixlo_f16) for the residual while the
                // packed operand rounds the f32 product, and where the two
                // differ by an f16 ulp the residual belongs to another high
                // term.
                float v = x[e] * qs;
                asm volatile("" : "+v"(v));
                qh[s][e] = static_cast<_Float16>(v);
                ql[s][e] = static_cast<_Float16>(v - static_cast<float>(qh[s][e]));
            }
        }
    }
    f32x4 o[HD / 16];
#pragma unroll
    for (int dt = 0; dt < HD / 16; ++dt) o[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float m = -__builtin_inff(), lsum = 0.0f;  // the lane's query: running max (log2 units) and sum

    // One block: wait for its loads, put its V into the V^T tile, issue the
    // next block's loads (K into the other tile's LDS, V into registers),
    // then the scores, the online softmax and O^T. Blocks alternate between
    // the two tiles (a pair a trip, so each is named statically).
    const auto block = [&](uint32_t kb, T& cur, T& nxt) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's K copies and V loads of block kb have landed
        store_vt<HD>(vr, cur);
        __syncthreads();  // every wave's; and block kb - 1's tiles are no longer read
        if (kb + 1 < blocks) load_block<HD>(a, kvh, kb + 1, keys, nxt, vr);
        // scores: lane (j, g) holds keys 32 kb + 16 tt + 4 g + e of query j
        f32x4 sacc[2];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            sacc[tt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            const uint32_t rr = 16 * tt + j;
#pragma unroll
            for (int s = 0; s < kSteps; ++s) {
                const uint32_t piece = (4 * s + g) ^ (rr % T::kPieces);
                const half8 kf = *reinterpret_cast<const half8*>(cur.k + rr * (HD * 2) + 16 * piece);
                sacc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qh[s], sacc[tt], 0, 0, 0);
                sacc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, ql[s], sacc[tt], 0, 0, 0);
            }
        }
        float sc[2][4];
        float bm = -__builtin_inff();
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float x = sacc[tt][e];
                if (cap) x = a.softcap * tanhf(fminf(fmaxf(x / a.softcap, -10.0f), 10.0f)) * kLog2e;
                const uint32_t key = kb * kBlock + 16 * tt + 4 * g + e;
                sc[tt][e] = qlive && key <= qpos ? x : -__builtin_inff();
                bm = fmaxf(bm, sc[tt][e]);
            }
        {
            const uint2 a16 = swap_rows<16>(__float_as_uint(bm));
            bm = fmaxf(__uint_as_float(a16.x), __uint_as_float(a16.y));
            const uint2 a32 = swap_rows<32>(__float_as_uint(bm));
            bm = fmaxf(__uint_as_float(a32.x), __uint_as_float(a32.y));
        }
        const float mn = fmaxf(m, bm);
        const bool any = mn != -__builtin_inff();
        const float factor = m == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(m - mn);
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
        lsum = lsum * factor + bs;
        m = mn;
        // O^T: lane (j, g) gives V^T at dim 16 dt + j of keys 4 g .. 4 g + 3
        // and 16 + 4 g .. 16 + 4 g + 3 of the block, the keys its P^T holds
#pragma unroll
        for (int dt = 0; dt < HD / 16; ++dt) {
            const _Float16* row = cur.vt + (16 * dt + j) * T::kVtStride + 4 * g;
            const uint2 lo = *reinterpret_cast<const uint2*>(row), hi = *reinterpret_cast<const uint2*>(row + 16);
            const half8 va = __builtin_bit_cast(half8, make_uint4(lo.x, lo.y, hi.x, hi.y));
#pragma unroll
            for (int e = 0; e < 4; ++e) o[dt][e] *= factor;
            o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, ph, o[dt], 0, 0, 0);
            o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pl, o[dt], 0, 0, 0);
        }
    };
    for (uint32_t kb = 0; kb < blocks; kb += 2) {
        block(kb, s_t[0], s_t[1]);
        if (kb + 1 < blocks) block(kb + 1, s_t[1], s_t[0]);
    }
    // lane (j, g) holds dims 16 dt + 4 g .. + 3 of query j
    if (qlive) {
        const float inv = 1.0f / lsum;
        float* op = a.out + (static_cast<uint64_t>(qi) * a.heads + h) * HD + 4 * g;
#pragma unroll
        for (int dt = 0; dt < HD / 16; ++dt)
            *reinterpret_cast<float4*>(op + 16 * dt) = make_float4(o[dt][0] * inv, o[dt][1] * inv, o[dt][2] * inv, o[dt][3] * inv);
    }
}

const char* check_prompt(const vkml_attend_prompt_params* p) {
    if (!p) return "null params";
    if (p->kv_type != VKML_F16) return "caches must be f16";
    if (p->head_dim != 64 && p->head_dim != 128) return "head_dim must be 64 or 128";
    if (p->kv_heads == 0 || p->heads % p->kv_heads || (p->heads / p->kv_heads) % kHeads)
        return "query heads a KV head must be a multiple of 4";
    if (p->t == 0) return "no queries";
    if (static_cast<uint64_t>(p->first) + p->t > p->capacity) return "the keys do not fit the caches";
    return nullptr;
}

}  // namespace

extern "C" {

int vkml_attend_prompt_fast_supported(const vkml_attend_prompt_params* p) {
    return vkml::abi::initialized() && !check_prompt(p) ? 1 : 0;
}

int vkml_attend_prompt_fast(const vkml_attend_prompt_params* p, const float* q, const void* k_cache, const void* v_cache, float* out) {
    VKML_REQUIRE_INIT();
    if (const char* why = check_prompt(p)) return vkml::abi::fail(VKML_ERROR_INVALID_ARGUMENT, std::string("attend_prompt_fast: ") + why);
    VKML_CHECK_ARG(q && k_cache && v_cache && out, "attend_prompt_fast: null buffer");
    const PromptArgs a{q, k_cache, v_cache, out, p->heads, p->kv_heads, p->heads / p->kv_heads, p->capacity, p->t, p->first,
                       p->scale, p->softcap};
    const dim3 grid((p->t + kQueries - 1) / kQueries * (p->kv_heads * (a.group / kHeads)));
    vkml::abi::ProfileScope prof("attend_prompt_fast");
    if (p->head_dim == 128)
        hipLaunchKernelGGL(k_attend_prompt_fast<128>, grid, dim3(kThreads), 0, vkml::abi::stream(), a);
    else
        hipLaunchKernelGGL(k_attend_prompt_fast<64>, grid, dim3(kThreads), 0, vkml::abi::stream(), a);
    return vkml::abi::check_launch("attend_prompt_fast");
}

}  // extern "C"
