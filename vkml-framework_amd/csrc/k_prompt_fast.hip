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
//     v_mfma_f32_16x16x32_f16, K from memory into registers a block ahead,
//     q (scaled into log2 units) as hi + lo f16 terms;
//   - per query (a lane column) the block's max and the running (max, sum),
//     the accumulated output rescaled by 2^(m_old - m_new);
//   - O^T [hd x 16 queries] += V^T . P^T, V copied into LDS a block ahead by
//     global_load_lds (16-byte pieces swizzled so that the four lane groups
//     of a read hit different banks), P^T straight from the score tile's
//     registers (the accumulator layout of S^T is the B operand's of P^T,
//     keys permuted alike in V^T's A operand). In O^T a query is a lane
//     column, as in S^T, so its rescale needs no exchange between lanes.
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
using vkml::attend_fast::v_offset;

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

template <int HD>
struct KRegs {
    uint4 k[2][HD / 32];  // the block's two 16-key tiles, 8 f16 a lane a step
};

// Key block kb's K fragments (lane (j, g) of tile tt: key 16 tt + j, dims
// 32 s + 8 g ..) and its V rows into LDS buffer `v` (the workgroup's 256
// threads, 16 bytes each an instruction). Keys past `keys` re-read the last.
template <int HD>
__device__ __forceinline__ void load_block(const PromptArgs& a, uint32_t kvh, uint32_t kb, uint32_t keys, KRegs<HD>& r, uint8_t* v) {
    constexpr uint32_t RB = HD * 2;
    const uint32_t t = thread_index(), l = t % kWave, j = l % 16, g = l / 16;
    const uint64_t row0 = static_cast<uint64_t>(kvh) * a.capacity;
    const auto* kc = static_cast<const uint8_t*>(a.k_cache);
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
        const uint64_t row = row0 + min(kb * kBlock + 16 * tt + j, keys - 1);
#pragma unroll
        for (int s = 0; s < HD / 32; ++s) r.k[tt][s] = ldg(reinterpret_cast<const uint4*>(kc + row * RB + 64 * s + 16 * g));
    }
    const auto* vc = static_cast<const uint8_t*>(a.v_cache);
    const uint32_t wave_first = t - l;
#pragma unroll
    for (uint32_t i = 0; i < kBlock * RB / (16 * kThreads); ++i) {
        const uint32_t at = 16 * (i * kThreads + t);  // byte in the block's rows
        const uint32_t rr = at / RB, piece = (at % RB) / 16;
        const uint32_t src_piece = piece ^ (2 * ((rr / 4) % 4));
        const uint64_t row = row0 + min(kb * kBlock + rr, keys - 1);
        vkml::attend::load_to_lds16(vc + row * RB + 16 * src_piece, v + 16 * (i * kThreads + wave_first));
    }
}

template <int HD>
__global__ void __launch_bounds__(kThreads) k_attend_prompt_fast(PromptArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t s_v[2][kBlock * HD * 2];
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

    KRegs<HD> kr[2];
    load_block<HD>(a, kvh, 0, keys, kr[0], s_v[0]);
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

    // One block: wait for its loads, issue the next block's (K into nxt, V
    // into the other LDS buffer), then the scores, the online softmax and
    // O^T. Blocks alternate between kr[0] and kr[1] (a pair a trip, so the
    // registers are named statically).
    const auto block = [&](uint32_t kb, const KRegs<HD>& kc, KRegs<HD>& nxt, const uint8_t* vb, uint8_t* vnext) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's loads of block kb have landed
        __syncthreads();                                   // every wave's; and block kb - 1's V is no longer read
        if (kb + 1 < blocks) load_block<HD>(a, kvh, kb + 1, keys, nxt, vnext);
        // scores: lane (j, g) holds keys 32 kb + 16 tt + 4 g + e of query j
        f32x4 sacc[2];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            sacc[tt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int s = 0; s < kSteps; ++s) {
                const half8 kf = __builtin_bit_cast(half8, kc.k[tt][s]);
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
        // O^T: lane (j, g) gives V^T at dim 16 dt + j of keys 4 g + e (e < 4)
        // and 16 + 4 g + e - 4 (e >= 4) of the block, the keys its P^T holds
        const uint32_t r0 = 4 * g;
#pragma unroll
        for (int dt = 0; dt < HD / 16; ++dt) {
            const uint32_t d = 16 * dt + j;
            half8 va;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t rr = r0 + (e < 4 ? e : 12 + e);
                va[e] = *reinterpret_cast<const _Float16*>(vb + v_offset<HD>(rr, d));
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) o[dt][e] *= factor;
            o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, ph, o[dt], 0, 0, 0);
            o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pl, o[dt], 0, 0, 0);
        }
    };
    for (uint32_t kb = 0; kb < blocks; kb += 2) {
        block(kb, kr[0], kr[1], s_v[0], s_v[1]);
        if (kb + 1 < blocks) block(kb + 1, kr[1], kr[0], s_v[1], s_v[0]);
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
