// k_attend.hip -- decode attention over the KV cache (the reference's
// shaders/attend.comp + attend_merge.comp, src/ops/attention.cpp:54-84):
// the kernels and the C ABI. The device code and its bit-exact order are in
// attend.hpp.
//
// Mapping. Workgroup (chunk, KV head, query head group) as the reference's
// (chunk, head), but numbered so that the query heads sharing a KV head run
// on the same XCD one after another (the dispatcher deals workgroups to the
// 8 XCDs round-robin): the K and V rows come from HBM once and from that
// XCD's L2 for the other heads. A decode step gives several workgroups per
// CU, so one's loads overlap another's arithmetic. The merge is its own
// launch, every load of a head's chunks issued at once, and can quantize its
// output to Q8_0 for the o projection.
//
// Merge + o. In a decode step the merge can share a launch with the o
// projection that consumes it (vkml_attend_step_o): the grid's first
// workgroups merge (two heads each at head_dim 128) and publish the Q8_0
// attention output, and the GEMV's workgroups, which issue their first
// weight loads at once, wait for it. The merge's latency then overlaps the
// GEMV's weight fetch, and the step loses a launch. The wait is on one of
// 16 copies of an arrival counter, to which every merging workgroup adds
// once its write-through stores have completed; it is bounded (a sticky
// error flag past the spin limit, which vkml_attend_o_check reports), and
// the launch is made only when the whole grid is resident at once, so no
// waiting workgroup can hold the slot a merging one needs.
#include <algorithm>

#include "attend.hpp"
#include "device.hpp"
#include "gemv.hpp"
#include "internal.hpp"

using namespace vkml::dev;
using namespace vkml::attend;

namespace {

template <int HD, bool F16, int HPW>
__global__ void __launch_bounds__(kThreads) k_attend_chunk(ChunkArgs a) {
    __shared__ AttendSmem<HD, F16, HPW> sm;
    // Workgroup number -> (chunk, KV head, head group): the head groups of a
    // (chunk, KV head) pair get numbers 8 apart, so the same XCD.
    const uint32_t G = a.group, groups = G / HPW, pairs = a.chunks * a.kv_heads;
    const uint32_t L = blockIdx.x, pair_lo = L % kXcds, rest = L / kXcds;
    if (a.o_sync && L == 0 && threadIdx.x < OSync::kCopies) OSync::counter(a.o_sync, threadIdx.x)[0] = 0u;
    const uint32_t hl = rest % groups, pair = (rest / groups) * kXcds + pair_lo;
    if (pair >= pairs) return;
    const uint32_t chunk = pair / a.kv_heads, kvh = pair % a.kv_heads, head0 = kvh * G + hl * HPW;
    const uint32_t spos = a.state ? static_cast<uint32_t>(ld_scalar_i32(&a.state->position)) : 0u;
    const uint32_t pos = a.step ? (a.state ? spos : a.position) : 0u;
    const uint32_t kv_len = a.step ? pos + 1 : (a.state ? spos + 1u : a.kv_len);
    if (a.window != 0 && kv_len > a.window) a.kv_start = max(a.kv_start, kv_len - a.window);
    if (a.error && L == 0 && threadIdx.x == 0 && kv_len - a.kv_start > a.chunks * kChunk)
        __hip_atomic_store(a.error, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (a.kv_start + chunk * kChunk >= kv_len) {
        // A chunk past the live keys (the grid covers the whole cache, so a
        // replayed graph serves every position): a max of -inf, which the
        // merge skips.
        if (threadIdx.x < HPW) {
            const uint64_t at = static_cast<uint64_t>(head0 + threadIdx.x) * a.chunks + chunk;
            a.stats[at * 2] = -__builtin_inff();
            a.stats[at * 2 + 1] = 0.0f;
        }
        return;
    }
    QLoads<HD, HPW> qv;  // first: the item waits for them before K and V
    attend_q_load<HD, HPW>(a, kvh, hl, pos, qv);
    ChunkLoads<HD, F16> ld;
    attend_chunk_load<HD, F16>(a, chunk, kvh, kv_len, ld, sm.v);
    attend_chunk_item<HD, F16, HPW, false>(a, chunk, kvh, hl, pos, kv_len, qv, ld, sm);
}

constexpr uint32_t kMergeMaxChunks = 1024;  // 131072 keys
// Chunks up to which a decode step's attention, merges and o GEMV run as one
// launch (vkml_attend_step_fused). Its merges are one workgroup per head set
// walking every chunk; the separate launches spread the merge. Measured at
// the 7B shape (32 heads on 8 KV heads, q4_K o), one launch against apart:
// 50 chunks 24.2 / 22.4 us, 66 chunks 27.1 / 28.2, 96 chunks 35.1 / 34.1,
// 131 chunks 44.0 / 37.5, 256 chunks 70.5 / 52.6. Launches are sized in
// power-of-two tiers of chunks, so the bound sits at a tier.
constexpr uint32_t kFusedMaxChunks = 64;

// The merge as its own launch: head blockIdx.x, element threadIdx.x.
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
k_attend_merge(const float* partial, const float* stats, float* out, uint8_t* values, float* scales, uint32_t chunks, uint32_t hd) {
    // (exp(m_c - M), or -1 for a chunk past the live keys; the chunk's sum of weights)
    __shared__ float2 s_rl[kMergeMaxChunks];
    __shared__ float s_wmax[8];
    merge_head<false, 48>(partial, stats, out, values, scales, blockIdx.x, chunks, chunks, hd, threadIdx.x, s_rl, s_wmax);
}

// The merge spread over (head, 32-element slice) workgroups:
// attend_merge.comp:25-38 with merge_head's arithmetic, bit for bit. The
// head's (max, weight sum) pairs are loaded by all 256 threads and M, each
// chunk's factor r_c = exp(m_c - M) and weight product r_c l_c formed once
// into LDS. The slice's partials are loaded 256 chunks a pass by 8 threads
// an element (every load of a pass in flight at once), and those threads
// form the products r_c partial_c (f32 products: the same wherever they
// are rounded) into LDS. Lane e of wave 0 then adds element e's products in
// chunk order, as merge_head's chain does (a chunk past the live keys adds
// +0 * +0 there: nothing), and the slice (one Q8_0 block) is quantized
// across those 32 lanes. Where merge_head's threads each load their
// element's partials in turn and do every operation of the chain, here a
// pass's loads and products come from every thread and the chain is two
// additions a chunk.
constexpr uint32_t kSlice = 32;       // elements a workgroup: one Q8_0 block
constexpr uint32_t kMergePass = 256;  // chunks whose products are in LDS at once

__global__ void __launch_bounds__(256)
k_attend_merge_wide(const float* partial, const float* stats, float* out, uint8_t* values, float* scales, uint32_t chunks, uint32_t hd) {
#pragma clang fp contract(off)
    __shared__ float s_r[kMergeMaxChunks];   // r_c, or -1 for a chunk past the live keys
    __shared__ float s_wp[kMergeMaxChunks];  // r_c l_c (+0 for such a chunk)
    __shared__ float s_p[kMergePass][kSlice];
    __shared__ float s_wmax[4];
    const uint32_t t = threadIdx.x, slices = hd / kSlice;
    const uint32_t h = blockIdx.x / slices, d0 = (blockIdx.x % slices) * kSlice;
    const uint64_t first = static_cast<uint64_t>(h) * chunks;
    const uint64_t* st = reinterpret_cast<const uint64_t*>(stats) + first;
    const float* pc = partial + first * hd + d0;
    const uint32_t e = t % kSlice, g = t / kSlice;  // loader: element e, chunks g, g + 8, ...
    // The first pass's partials, in flight while M and the factors are formed.
    constexpr uint32_t kPer = kMergePass / (256 / kSlice);  // 32 loads a thread a pass
    float p[kPer];
#pragma unroll
    for (uint32_t j = 0; j < kPer; ++j) p[j] = ldg(pc + static_cast<uint64_t>(min(g + 8 * j, chunks - 1)) * hd + e);
    // M = max over the chunks' maxima (exact in any order)
    float m = -__builtin_inff();
    for (uint32_t c = t; c < chunks; c += 256) m = fmaxf(m, __uint_as_float(static_cast<uint32_t>(ldg(st + c))));
    m = wave_max(m);
    if (t % kWave == 0) s_wmax[t / kWave] = m;
    __syncthreads();
    const float top = fmaxf(fmaxf(s_wmax[0], s_wmax[1]), fmaxf(s_wmax[2], s_wmax[3]));
    for (uint32_t c = t; c < chunks; c += 256) {
        const uint64_t ml = ldg(st + c);
        const float mc = __uint_as_float(static_cast<uint32_t>(ml)), lc = __uint_as_float(static_cast<uint32_t>(ml >> 32));
        const float r = mc == -__builtin_inff() ? -1.0f : vk_expf(mc - top);
        const uint32_t keep = r >= 0.0f ? ~0u : 0u;
        const float rr = __uint_as_float(__float_as_uint(r) & keep);
        s_r[c] = r;
        s_wp[c] = rr * __uint_as_float(__float_as_uint(lc) & keep);
    }
    __syncthreads();
    float sum = 0.0f, weight = 0.0f;
    for (uint32_t c0 = 0; c0 < chunks; c0 += kMergePass) {
        if (c0 > 0) {
            __syncthreads();  // the previous pass's chain is done with s_p
#pragma unroll
            for (uint32_t j = 0; j < kPer; ++j) p[j] = ldg(pc + static_cast<uint64_t>(min(c0 + g + 8 * j, chunks - 1)) * hd + e);
        }
#pragma unroll
        for (uint32_t j = 0; j < kPer; ++j) {
            const uint32_t c = min(c0 + g + 8 * j, chunks - 1);
            const float r = s_r[c];
            const uint32_t keep = r >= 0.0f ? ~0u : 0u;
            s_p[g + 8 * j][e] = __uint_as_float(__float_as_uint(r) & keep) * __uint_as_float(__float_as_uint(p[j]) & keep);
        }
        __syncthreads();
        if (t < kSlice) {
            const uint32_t n = min(kMergePass, chunks - c0);
            uint32_t j0 = 0;
            for (; j0 + 8 <= n; j0 += 8) {
                float pv[8], wv[8];
#pragma unroll
                for (uint32_t j = 0; j < 8; ++j) {
                    pv[j] = s_p[j0 + j][e];
                    wv[j] = s_wp[c0 + j0 + j];
                }
#pragma unroll
                for (uint32_t j = 0; j < 8; ++j) {
                    sum += pv[j];
                    weight += wv[j];
                }
            }
            for (; j0 < n; ++j0) {
                sum += s_p[j0][e];
                weight += s_wp[c0 + j0];
            }
        }
    }
    if (t < kSlice) {
        const float o = sum / weight;
        const uint64_t at = static_cast<uint64_t>(h) * hd + d0 + e;
        if (out) out[at] = o;
        if (values) {
            const float absmax = group_max<32>(fabsf(o));
            const float ds = absmax / 127.0f;
            const float inv = ds > 0.0f ? 1.0f / ds : 0.0f;
            values[at] = static_cast<uint8_t>(static_cast<int8_t>(quant_code(o, inv)));
            if (e == 0) scales[at / 32] = ds;
        }
    }
}

template <int HD, bool F16>
void launch_hd(const ChunkArgs& args, uint32_t pair_blocks) {
    hipStream_t s = vkml::abi::stream();
    // Four heads a workgroup (one K and V load for a whole GQA group of 4)
    // where that still leaves two workgroups a compute unit: measured 17%
    // faster at 32K keys, 6% slower at 4K (fewer items to spread).
    if (args.group % 4 == 0 && static_cast<uint64_t>(pair_blocks) * kXcds * (args.group / 4) >= 2ull * vkml::abi::compute_units()) {
        const dim3 grid(pair_blocks * kXcds * (args.group / 4));
        hipLaunchKernelGGL((k_attend_chunk<HD, F16, 4>), grid, dim3(kThreads), 0, s, args);
    } else if (args.group % 2 == 0) {
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
    // Past a few chunks a head, its elements' partial loads are spread over
    // (head, slice) workgroups; few chunks keep one workgroup a head.
    if (chunks > 16)
        hipLaunchKernelGGL(k_attend_merge_wide, dim3(heads * (head_dim / kSlice)), dim3(256), 0, vkml::abi::stream(), partial, stats,
                           out, static_cast<uint8_t*>(values), scales, chunks, head_dim);
    else
        hipLaunchKernelGGL(k_attend_merge, dim3(heads), dim3(head_dim), 0, vkml::abi::stream(), partial, stats, out,
                           static_cast<uint8_t*>(values), scales, chunks, head_dim);
    return VKML_OK;
}

// ---------------------------------------------------------------- merge + o

struct MergeOArgs {
    const float* partial;
    const float* stats;
    float* out;
    uint8_t* values;
    float* scales;
    uint32_t hd, chunks, merge_wgs;
    uint32_t* sync;
    uint32_t wait_cap;  // polls before the GEMV's wait gives up
};

// Workgroups [0, merge_wgs): the merge (kThreads / hd heads each, thread
// element d of head h), its Q8_0 output stored write-through; then the
// arrival on every counter copy. The rest: the o GEMV (32
// lanes a row, + residual) on that output, as k_gemv_dot runs it.
template <int FMT, bool FULL>
__global__ void __launch_bounds__(kThreads) k_merge_o(MergeOArgs m, vkml::gemv::GemvArgs g) {
    extern __shared__ uint4 smem[];
    if (blockIdx.x < m.merge_wgs) {
        const uint32_t hpw = kThreads / m.hd, half = threadIdx.x / m.hd, d = threadIdx.x % m.hd;
        float* f = reinterpret_cast<float*>(smem);
        float2* s_rl = reinterpret_cast<float2*>(f + half * 2 * m.chunks);
        float* s_wmax = f + hpw * 2 * m.chunks + half * (m.hd / kWave);
        merge_head<true, 36>(m.partial, m.stats, m.out, m.values, m.scales, blockIdx.x * hpw + half, m.chunks, m.chunks, m.hd, d, s_rl,
                         s_wmax);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the write-through stores have completed
        __syncthreads();
        if (threadIdx.x < OSync::kCopies)
            __hip_atomic_fetch_add(OSync::counter(m.sync, threadIdx.x), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    const uint32_t wg = blockIdx.x - m.merge_wgs;
    vkml::gemv::GemvRows<FMT, true, 32, vkml::gemv::kAdd, 2, kThreads, false, false, 1, FULL> rows;
    rows.start(g, wg);
    if (!await_merged(m.sync, wg, m.merge_wgs, OSync::error(m.sync), m.wait_cap)) return;
    vkml::gemv::stage_activation<kThreads, false, true>(g, smem);
    rows.finish(g, smem, vkml::gemv::staged_ss(smem, g.k));
}

template <int FMT, bool FULL>
bool launch_merge_o_as(const MergeOArgs& m, const vkml::gemv::GemvArgs& g, uint32_t grid, size_t lds) {
    const void* fn = reinterpret_cast<const void*>(&k_merge_o<FMT, FULL>);
    static int per_cu = -1;  // resident workgroups a CU at this LDS size
    static size_t per_cu_lds = 0;
    if (per_cu < 0 || per_cu_lds != lds) {
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kThreads, lds) != hipSuccess) per_cu = 0;
        per_cu_lds = lds;
    }
    if (static_cast<uint64_t>(per_cu) * vkml::abi::compute_units() < grid) return false;
    hipLaunchKernelGGL((k_merge_o<FMT, FULL>), dim3(grid), dim3(kThreads), lds, vkml::abi::stream(), m, g);
    return true;
}

// The merge + o launch, if the shapes allow it and the grid is resident at
// once; false otherwise (nothing launched).
bool launch_merge_o(const MergeOArgs& m, const vkml::gemv::GemvArgs& g, uint32_t heads, uint32_t b_type, uint32_t scale_type) {
    using namespace vkml::gemv;
    if (b_type != VKML_Q4_K && !(b_type == VKML_Q8_0 && scale_type == VKML_F16)) return false;
    const uint32_t hpw = kThreads / m.hd;
    if (heads % hpw != 0 || g.k != heads * m.hd || g.n == 0) return false;
    const bool q4k = b_type == VKML_Q4_K;
    if ((q4k ? code_bytes<VKML_Q4_K>(g.n, g.k) : code_bytes<VKML_Q8_0>(g.n, g.k)) >= (1ull << 32) ||
        (q4k ? scale_bytes<VKML_Q4_K, true>(g.n, g.k) : scale_bytes<VKML_Q8_0, true>(g.n, g.k)) >= (1ull << 32))
        return false;
    const size_t merge_lds = (static_cast<size_t>(hpw) * 2 * m.chunks + hpw * (m.hd / kWave)) * 4;
    const size_t lds = std::max<size_t>(stage_bytes(g.k, false), merge_lds);
    if (lds > 64 * 1024) return false;
    const uint32_t grid = m.merge_wgs + (g.n + kThreads / 32 - 1) / (kThreads / 32);
    const bool full = g.k % 2048 == 0;  // whole pairs of 2-round batches
    if (q4k) return full ? launch_merge_o_as<VKML_Q4_K, true>(m, g, grid, lds) : launch_merge_o_as<VKML_Q4_K, false>(m, g, grid, lds);
    return full ? launch_merge_o_as<VKML_Q8_0, true>(m, g, grid, lds) : launch_merge_o_as<VKML_Q8_0, false>(m, g, grid, lds);
}

// ------------------------------------------- chunks + merge + o, one launch

struct FusedArgs {
    uint32_t attn_wgs;  // workgroups of the chunk pass (grid padding included), first in the grid
    uint32_t merges;    // sets of chunk items: merging workgroups, one a set
    uint32_t* sync;     // this launch's block: every counter zero at the start
    uint32_t* next;     // the next launch's block, whose o GEMV counters this one zeroes
    uint32_t* error;    // the sticky error flag
    float* out;         // the merged outputs [heads, hd] f32
    uint8_t* values;    // and their Q8_0 codes and f32 scales: the o GEMV's input
    float* scales;
    uint32_t wait_cap;  // polls before the GEMV's wait gives up
};

// Workgroups [0, attn_wgs): the chunk pass, as k_attend_chunk, its partials
// and statistics stored write-through; then each adds one to its set's
// arrival counter, and the set's last to arrive (every other item of the
// set has stored its results) resets the counter, merges the set's HPW
// heads in chunk order (attend_merge.comp's arithmetic, merge_head) with
// the Q8_0 of the outputs stored write-through, and adds one to every copy
// of the o GEMV counter. The rest: the o GEMV + residual, as in k_merge_o,
// waiting (bounded) for all merges. Chunk items never wait, so the GEMV's
// workgroups, fewer than the resident slots, cannot keep an item from
// running, in whatever order workgroups are dispatched.
template <int HD, bool F16, int HPW, int FMT, bool FULL, int DEEP>
__global__ void __launch_bounds__(kThreads) k_attend_fused(ChunkArgs a, FusedArgs f, vkml::gemv::GemvArgs g) {
    extern __shared__ uint4 smem[];
    if (blockIdx.x >= f.attn_wgs) {
        // DEEP (K = 512 DEEP): the rows' every weight load is in flight before the wait
        const uint32_t wg = blockIdx.x - f.attn_wgs;
        vkml::gemv::GemvRows<FMT, true, 32, vkml::gemv::kAdd, DEEP ? DEEP : 2, kThreads, false, false, DEEP ? 0 : 1, FULL> rows;
        rows.start(g, wg);
        if (!await_merged(f.sync, wg, f.merges, f.error, f.wait_cap)) return;
        vkml::gemv::stage_activation<kThreads, false, true>(g, smem);
        rows.finish(g, smem, vkml::gemv::staged_ss(smem, g.k));
        return;
    }
    auto& sm = *reinterpret_cast<AttendSmem<HD, F16, HPW>*>(smem);
    const uint32_t G = a.group, groups = G / HPW, pairs = a.chunks * a.kv_heads;
    const uint32_t L = blockIdx.x, pair_lo = L % kXcds, rest = L / kXcds;
    if (L == 0 && threadIdx.x < OSync::kCopies) OSync::counter(f.next, threadIdx.x)[0] = 0u;
    const uint32_t hl = rest % groups, pair = (rest / groups) * kXcds + pair_lo;
    if (pair >= pairs) return;
    const uint32_t chunk = pair / a.kv_heads, kvh = pair % a.kv_heads, head0 = kvh * G + hl * HPW;
    // Items of chunks that hold keys at any position the launch may see
    // issue their loads before reading the position: q as the q|k|v GEMV
    // left it, K and V over the whole chunk (rows past the live keys, read
    // modulo the capacity, are masked out by the item).
    QLoads<HD, HPW> qv;
    ChunkLoads<HD, F16> ld;
    const bool early = chunk < a.ready;
    if (early) {
        attend_q_load<HD, HPW>(a, kvh, hl, 0, qv);
        attend_chunk_load<HD, F16>(a, chunk, kvh, a.kv_start + (chunk + 1) * kChunk, ld, sm.v);
    }
    const uint32_t pos = static_cast<uint32_t>(ld_scalar_i32(&a.state->position));
    const uint32_t kv_len = pos + 1;
    if (a.window != 0 && kv_len > a.window) a.kv_start = max(a.kv_start, kv_len - a.window);
    // Launched for fewer chunks than the cache holds: keys past them would
    // be left out, so the launch reports it (the results are invalid).
    if (L == 0 && threadIdx.x == 0 && kv_len - a.kv_start > a.chunks * kChunk)
        __hip_atomic_store(f.error, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (a.kv_start + chunk * kChunk >= kv_len) {
        if (threadIdx.x < HPW) {  // past the live keys: a max of -inf, which the merge skips
            const uint64_t at = static_cast<uint64_t>(head0 + threadIdx.x) * a.chunks + chunk;
            st_f32<true>(a.stats + at * 2, -__builtin_inff());
            st_f32<true>(a.stats + at * 2 + 1, 0.0f);
        }
    } else {
        if (!early) {
            attend_q_load<HD, HPW>(a, kvh, hl, pos, qv);
            attend_chunk_load<HD, F16>(a, chunk, kvh, kv_len, ld, sm.v);
        }
        attend_chunk_item<HD, F16, HPW, true>(a, chunk, kvh, hl, pos, kv_len, qv, ld, sm);
    }
    __shared__ uint32_t s_last;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the write-through stores have completed
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t* c = FusedSync::arrive(f.sync, kvh * groups + hl);
        const bool last = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == a.chunks - 1;
        if (last) __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = last;
    }
    __syncthreads();
    if (!s_last) return;
    // The merge, kThreads / HD heads at a time (thread element d of head
    // `half`); threads past the heads of a pass redo its first head without
    // storing, to keep the barriers whole.
    constexpr uint32_t kHalves = kThreads / HD;
    constexpr uint32_t kAtOnce = kHalves < HPW ? kHalves : HPW;
    const uint32_t half = threadIdx.x / HD, d = threadIdx.x % HD;
    float* fl = reinterpret_cast<float*>(smem);
    float2* s_rl = reinterpret_cast<float2*>(fl + half * 2 * a.chunks);
    float* s_wmax = fl + kHalves * 2 * a.chunks + half * (HD / kWave);
    // Chunks past the live keys hold a max of -inf, which the merge skips:
    // it walks the live ones only.
    const uint32_t live = min(a.chunks, (kv_len - a.kv_start + kChunk - 1) / kChunk);
#pragma unroll
    for (uint32_t h0 = 0; h0 < HPW; h0 += kAtOnce) {
        const bool mine = half < kAtOnce;
        if (h0 > 0) __syncthreads();  // the previous pass is done with s_rl
        merge_head<true, 36>(a.partial, a.stats, mine ? f.out : nullptr, mine ? f.values : nullptr, f.scales,
                             head0 + h0 + (mine ? half : 0), a.chunks, live, HD, d, s_rl, s_wmax);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x < OSync::kCopies)
        __hip_atomic_fetch_add(OSync::counter(f.sync, threadIdx.x), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int HD, bool F16, int HPW, int FMT, bool FULL, int DEEP = 0>
bool launch_fused_as(const ChunkArgs& a, const FusedArgs& f, const vkml::gemv::GemvArgs& g, uint32_t gemv_wgs, bool dry) {
    const void* fn = reinterpret_cast<const void*>(&k_attend_fused<HD, F16, HPW, FMT, FULL, DEEP>);
    constexpr uint32_t kHalves = kThreads / HD;
    const size_t merge_lds = (static_cast<size_t>(kHalves) * 2 * a.chunks + kHalves * (HD / kWave)) * 4;
    const size_t lds = std::max({sizeof(AttendSmem<HD, F16, HPW>), merge_lds, static_cast<size_t>(vkml::gemv::stage_bytes(g.k, false))});
    if (lds > 64 * 1024) return false;
    static int per_cu = -1;  // resident workgroups a CU at this LDS size
    static size_t per_cu_lds = 0;
    if (per_cu < 0 || per_cu_lds != lds) {
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kThreads, lds) != hipSuccess) per_cu = 0;
        per_cu_lds = lds;
    }
    // the waiting GEMV workgroups must leave slots for the chunk items
    if (static_cast<uint64_t>(per_cu) * vkml::abi::compute_units() <= gemv_wgs) return false;
    if (dry) return true;
    hipLaunchKernelGGL((k_attend_fused<HD, F16, HPW, FMT, FULL, DEEP>), dim3(f.attn_wgs + gemv_wgs), dim3(kThreads), lds,
                       vkml::abi::stream(), a, f, g);
    return true;
}

template <int HD, bool F16, int HPW>
bool launch_fused_hpw(const ChunkArgs& a, const FusedArgs& f, const vkml::gemv::GemvArgs& g, uint32_t gemv_wgs, bool q4k, bool dry) {
    const bool full = g.k % 2048 == 0;  // whole pairs of 2-round batches
    // o rows of 2048 or 4096 values: every round's weights in flight at once
    if (g.k == 4096)
        return q4k ? launch_fused_as<HD, F16, HPW, VKML_Q4_K, true, 8>(a, f, g, gemv_wgs, dry)
                   : launch_fused_as<HD, F16, HPW, VKML_Q8_0, true, 8>(a, f, g, gemv_wgs, dry);
    if (g.k == 2048)
        return q4k ? launch_fused_as<HD, F16, HPW, VKML_Q4_K, true, 4>(a, f, g, gemv_wgs, dry)
                   : launch_fused_as<HD, F16, HPW, VKML_Q8_0, true, 4>(a, f, g, gemv_wgs, dry);
    if (q4k)
        return full ? launch_fused_as<HD, F16, HPW, VKML_Q4_K, true>(a, f, g, gemv_wgs, dry)
                    : launch_fused_as<HD, F16, HPW, VKML_Q4_K, false>(a, f, g, gemv_wgs, dry);
    return full ? launch_fused_as<HD, F16, HPW, VKML_Q8_0, true>(a, f, g, gemv_wgs, dry)
                : launch_fused_as<HD, F16, HPW, VKML_Q8_0, false>(a, f, g, gemv_wgs, dry);
}

// The one-launch form, if the shapes allow it; false otherwise (nothing launched).
bool launch_fused(uint32_t head_dim, bool f16, const ChunkArgs& a, FusedArgs f, const vkml::gemv::GemvArgs& g, uint32_t b_type,
                  uint32_t scale_type, bool dry = false) {
    using namespace vkml::gemv;
    if (b_type != VKML_Q4_K && !(b_type == VKML_Q8_0 && scale_type == VKML_F16)) return false;
    const bool q4k = b_type == VKML_Q4_K;
    if (g.k != a.heads * head_dim || g.n == 0) return false;
    if ((q4k ? code_bytes<VKML_Q4_K>(g.n, g.k) : code_bytes<VKML_Q8_0>(g.n, g.k)) >= (1ull << 32) ||
        (q4k ? scale_bytes<VKML_Q4_K, true>(g.n, g.k) : scale_bytes<VKML_Q8_0, true>(g.n, g.k)) >= (1ull << 32))
        return false;
    const uint32_t hpw = a.group % 2 == 0 ? 2 : 1;
    f.merges = a.kv_heads * (a.group / hpw);
    if (f.merges > FusedSync::kMaxSets) return false;
    const uint32_t pair_blocks = (a.chunks * a.kv_heads + kXcds - 1) / kXcds;
    f.attn_wgs = pair_blocks * kXcds * (a.group / hpw);
    const uint32_t gemv_wgs = (g.n + kThreads / 32 - 1) / (kThreads / 32);
#define VKML_FUSED(HD)                                                                                             \
    (f16 ? (hpw == 2 ? launch_fused_hpw<HD, true, 2>(a, f, g, gemv_wgs, q4k, dry) : launch_fused_hpw<HD, true, 1>(a, f, g, gemv_wgs, q4k, dry)) \
         : (hpw == 2 ? launch_fused_hpw<HD, false, 2>(a, f, g, gemv_wgs, q4k, dry) : launch_fused_hpw<HD, false, 1>(a, f, g, gemv_wgs, q4k, dry)))
    switch (head_dim) {
        case 64: return VKML_FUSED(64);
        case 128: return VKML_FUSED(128);
        default: return VKML_FUSED(256);
    }
#undef VKML_FUSED
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
    VKML_CHECK_ARG(p->chunks > 0 && p->capacity > 0, "attend: chunks and capacity must be positive");
    // Key position p sits at row p % capacity (a ring, when positions pass
    // the capacity): the keys seen must fit the rows.
    VKML_CHECK_ARG(state ? p->kv_start < p->capacity : p->kv_start < p->kv_len && p->kv_len - p->kv_start <= p->capacity,
                   "attend: keys " + std::to_string(p->kv_start) + ".." + std::to_string(p->kv_len) + " do not fit the cache of " +
                       std::to_string(p->capacity) + " rows");
    // With a decode state, kv_len can reach the capacity: cover every chunk of it.
    const uint64_t keys = state ? p->capacity - p->kv_start : p->kv_len - p->kv_start;
    VKML_CHECK_ARG(static_cast<uint64_t>(p->chunks) * kChunk >= keys,
                   "attend: " + std::to_string(p->chunks) + " chunks of " + std::to_string(kChunk) + " keys do not cover " +
                       std::to_string(keys) + " keys");
    VKML_CHECK_ARG(q && k_cache && v_cache && partial && stats, "attend: null buffer");
    ChunkArgs args{q, nullptr, const_cast<void*>(k_cache), const_cast<void*>(v_cache), partial, stats, state,
                   p->heads, p->kv_heads, p->heads / p->kv_heads, p->capacity, p->kv_start, p->kv_len, 0, p->chunks,
                   0, 0, 0, p->scale, p->softcap, nullptr, 0};
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

}  // extern "C"

namespace {

int check_step(const vkml_attend_step_params* p, const float* qkv, const float* rope_table, const void* k_cache, const void* v_cache,
               const float* partial, const float* stats, const float* out, const void* values, const float* scales,
               const vkml_decode_state* state, const char* what, bool fewer_chunks = false) {
    VKML_REQUIRE_INIT();
    const std::string w(what);
    VKML_CHECK_ARG(p, w + ": null params");
    if (int r = check_heads(p->heads, p->kv_heads, p->head_dim, what)) return r;
    VKML_CHECK_ARG(p->kv_type == VKML_F16 || p->kv_type == VKML_F32, w + ": caches must be f16 or f32");
    VKML_CHECK_ARG(p->capacity > 0 && p->kv_start < p->capacity, w + ": kv_start must lie inside the cache");
    VKML_CHECK_ARG(state || (p->position < p->capacity && p->kv_start <= p->position),
                   w + ": position " + std::to_string(p->position) + " is outside the cache");
    const uint64_t span = p->window ? std::min<uint64_t>(p->window, p->capacity - p->kv_start) : p->capacity - p->kv_start;
    VKML_CHECK_ARG((fewer_chunks ? p->chunks > 0 : static_cast<uint64_t>(p->chunks) * kChunk >= span) && p->chunks <= kMergeMaxChunks,
                   w + ": " + std::to_string(p->chunks) + " chunks do not cover the " + std::to_string(span) + " keys a step can see (or exceed " +
                       std::to_string(kMergeMaxChunks) + ")");
    VKML_CHECK_ARG(qkv && (rope_table || p->prepared) && k_cache && v_cache && partial && stats && out, w + ": null buffer");
    VKML_CHECK_ARG(!p->prepared || state, w + ": a prepared step reads its position from the decode state");
    VKML_CHECK_ARG(!values || scales, w + ": quantized output needs scales");
    return VKML_OK;
}

ChunkArgs step_args(const vkml_attend_step_params* p, const float* qkv, const float* rope_table, void* k_cache, void* v_cache,
                    float* partial, float* stats, const vkml_decode_state* state, uint32_t* o_sync) {
    return ChunkArgs{qkv, rope_table, k_cache, v_cache, partial, stats, state, p->heads, p->kv_heads, p->heads / p->kv_heads,
                     p->capacity, p->kv_start, 0, p->position, p->chunks, 1, p->rope_style, p->rotate, p->scale, p->softcap, o_sync,
                     p->window, p->prepared, p->prepared && !p->window ? std::min(p->ready_chunks, p->chunks) : 0u};
}

}  // namespace

extern "C" {

int vkml_attend_step(const vkml_attend_step_params* p, const float* qkv, const float* rope_table, void* k_cache, void* v_cache,
                     float* partial, float* stats, float* out, void* values, float* scales, const vkml_decode_state* state) {
    if (int r = check_step(p, qkv, rope_table, k_cache, v_cache, partial, stats, out, values, scales, state, "attend_step")) return r;
    const ChunkArgs args = step_args(p, qkv, rope_table, k_cache, v_cache, partial, stats, state, nullptr);
    {
        vkml::abi::ProfileScope prof("attend_step");
        launch_chunks(p->head_dim, p->kv_type == VKML_F16, args);
        if (int r = vkml::abi::check_launch("attend_step")) return r;
    }
    vkml::abi::ProfileScope prof("attend_merge");
    launch_merge(p->heads, p->head_dim, p->chunks, partial, stats, out, values, scales);
    return vkml::abi::check_launch("attend_merge");
}

uint64_t vkml_attend_o_sync_bytes(void) { return static_cast<uint64_t>(OSync::kWords) * 4; }

int vkml_attend_step_o(const vkml_attend_step_params* p, const float* qkv, const float* rope_table, void* k_cache, void* v_cache,
                       float* partial, float* stats, float* out, void* values, float* scales, const vkml_decode_state* state,
                       const vkml_gemv_dot_params* o, const void* o_values, const void* o_scales, float* x, uint32_t* sync) {
    if (int r = check_step(p, qkv, rope_table, k_cache, v_cache, partial, stats, out, values, scales, state, "attend_step_o")) return r;
    VKML_CHECK_ARG(o && values && scales && o_values && o_scales && x && sync, "attend_step_o: null buffer");
    VKML_CHECK_ARG(o->m == 1 && o->k == p->heads * p->head_dim,
                   "attend_step_o: the o projection must take the " + std::to_string(p->heads * p->head_dim) + " attention outputs");
    const MergeOArgs m{partial, stats, out, static_cast<uint8_t*>(values), scales, p->head_dim, p->chunks,
                       p->heads / (kThreads / p->head_dim), sync, vkml::abi::wait_limit()};
    const vkml::gemv::GemvArgs g{static_cast<const uint4*>(values), scales, o_values, o_scales, nullptr, nullptr, x, x, o->n, o->k};
    // The chunk pass clears the merge + o sync words only when that launch follows.
    const bool fusable = o->b_type == VKML_Q4_K || (o->b_type == VKML_Q8_0 && o->scale_type == VKML_F16);
    const ChunkArgs args = step_args(p, qkv, rope_table, k_cache, v_cache, partial, stats, state, fusable ? sync : nullptr);
    {
        vkml::abi::ProfileScope prof("attend_step");
        launch_chunks(p->head_dim, p->kv_type == VKML_F16, args);
        if (int r = vkml::abi::check_launch("attend_step")) return r;
    }
    if (fusable) {
        vkml::abi::ProfileScope prof("attend_merge_o");
        if (launch_merge_o(m, g, p->heads, o->b_type, o->scale_type)) return vkml::abi::check_launch("attend_merge_o");
    }
    {
        vkml::abi::ProfileScope prof("attend_merge");
        launch_merge(p->heads, p->head_dim, p->chunks, partial, stats, out, values, scales);
        if (int r = vkml::abi::check_launch("attend_merge")) return r;
    }
    return vkml_gemv_dot_add(o, values, o_values, x, o_scales, scales, x);
}

uint64_t vkml_attend_fused_sync_bytes(uint32_t blocks) { return static_cast<uint64_t>(FusedSync::kWords) * 4 * blocks; }

int vkml_attend_step_fused(const vkml_attend_step_params* p, const float* qkv, const float* rope_table, void* k_cache, void* v_cache,
                           float* partial, float* stats, float* out, void* values, float* scales, const vkml_decode_state* state,
                           const vkml_gemv_dot_params* o, const void* o_values, const void* o_scales, float* x, uint32_t* sync,
                           uint32_t block, uint32_t blocks) {
    if (int r = check_step(p, qkv, rope_table, k_cache, v_cache, partial, stats, out, values, scales, state, "attend_step_fused", true))
        return r;
    VKML_CHECK_ARG(state, "attend_step_fused: needs the decode state");
    VKML_CHECK_ARG(o && values && scales && o_values && o_scales && x && sync, "attend_step_fused: null buffer");
    VKML_CHECK_ARG(blocks >= 2 && block < blocks, "attend_step_fused: block " + std::to_string(block) + " of " + std::to_string(blocks) +
                                                      " (two blocks at least)");
    VKML_CHECK_ARG(o->m == 1 && o->k == p->heads * p->head_dim,
                   "attend_step_fused: the o projection must take the " + std::to_string(p->heads * p->head_dim) + " attention outputs");
    uint32_t* own = sync + static_cast<uint64_t>(block) * FusedSync::kWords;
    uint32_t* next = sync + static_cast<uint64_t>((block + 1) % blocks) * FusedSync::kWords;
    ChunkArgs args = step_args(p, qkv, rope_table, k_cache, v_cache, partial, stats, state, nullptr);
    const FusedArgs f{0, 0, own, next, sync, out, static_cast<uint8_t*>(values), scales, vkml::abi::wait_limit()};
    const vkml::gemv::GemvArgs g{static_cast<const uint4*>(values), scales, o_values, o_scales, nullptr, nullptr, x, x, o->n, o->k};
    // Past kFusedMaxChunks chunks each head set's merge, one workgroup
    // walking every chunk, outlasts launching it apart (spread over (head,
    // slice) workgroups): those steps take the separate launches below,
    // which report a position past their chunks on the same flag.
    const bool long_merge = p->chunks > kFusedMaxChunks;
    if (!long_merge) {
        vkml::abi::ProfileScope prof("attend_fused");
        if (launch_fused(p->head_dim, p->kv_type == VKML_F16, args, f, g, o->b_type, o->scale_type))
            return vkml::abi::check_launch("attend_step_fused");
        // Shapes the one launch does not take: the chunk pass, the merge and
        // the o GEMV over every chunk of the cache.
        const uint64_t span = p->window ? std::min<uint64_t>(p->window, p->capacity - p->kv_start) : p->capacity - p->kv_start;
        VKML_CHECK_ARG(static_cast<uint64_t>(p->chunks) * kChunk >= span,
                       "attend_step_fused: these weights take separate launches, which need chunks covering the cache");
    }
    // The separate launches; the next block's counters zeroed all the same.
    args.error = sync;
    {
        vkml::abi::ProfileScope prof("attend_step");
        launch_chunks(p->head_dim, p->kv_type == VKML_F16, args);
        if (int r = vkml::abi::check_launch("attend_step")) return r;
    }
    {
        vkml::abi::ProfileScope prof("attend_merge");
        launch_merge(p->heads, p->head_dim, p->chunks, partial, stats, out, values, scales);
        if (int r = vkml::abi::check_launch("attend_merge")) return r;
    }
    if (int r = vkml_fill_u32(next + OSync::kLine, 0u, OSync::kWords - OSync::kLine)) return r;
    return vkml_gemv_dot_add(o, values, o_values, x, o_scales, scales, x);
}

int vkml_attend_step_fused_supported(const vkml_attend_step_params* p, const vkml_gemv_dot_params* o) {
    if (!vkml::abi::initialized() || !p || !o || o->m != 1 || p->kv_heads == 0 || p->heads % p->kv_heads || p->chunks == 0 ||
        p->chunks > kMergeMaxChunks || (p->head_dim != 64 && p->head_dim != 128 && p->head_dim != 256) ||
        (p->kv_type != VKML_F16 && p->kv_type != VKML_F32))
        return 0;
    // (past kFusedMaxChunks a step takes the separate launches: the one
    // launch is asked for the largest count it serves)
    vkml_attend_step_params q = *p;
    q.chunks = std::min(q.chunks, kFusedMaxChunks);
    const ChunkArgs args = step_args(&q, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr);
    const FusedArgs f{0, 0, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 0};
    const vkml::gemv::GemvArgs g{nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, o->n, o->k};
    return launch_fused(p->head_dim, p->kv_type == VKML_F16, args, f, g, o->b_type, o->scale_type, true) ? 1 : 0;
}

int vkml_attend_fused_status(uint32_t* sync, uint32_t blocks, uint32_t* flag_out) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(sync && blocks >= 2 && flag_out, "attend_fused_status: null buffer or fewer than two blocks");
    hipStream_t s = vkml::abi::stream();
    uint32_t flag = 0;
    hipError_t e = hipMemcpyAsync(&flag, sync, 4, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return vkml::abi::hip_fail(e, "attend_fused_status");
    *flag_out = flag;
    if (flag == 0) return VKML_OK;
    // A wait gave up, or a position outran the chunks: every block starts
    // over (flag and counters).
    e = hipMemsetAsync(sync, 0, vkml_attend_fused_sync_bytes(blocks), s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return vkml::abi::hip_fail(e, "attend_fused_status");
    return VKML_OK;
}

int vkml_attend_fused_check(uint32_t* sync, uint32_t blocks) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(sync && blocks >= 2, "attend_fused_check: null buffer or fewer than two blocks");
    uint32_t flag = 0;
    if (int r = vkml_attend_fused_status(sync, blocks, &flag)) return r;
    if (flag == 0) return VKML_OK;
    if (flag == 2)
        return vkml::abi::fail(VKML_ERROR_DEVICE,
                               "attend_step_fused: a position lay past the keys of the launched chunks; the step's results are invalid");
    return vkml::abi::fail(VKML_ERROR_DEVICE,
                           "attend_step_fused: the o GEMV's wait for the merges timed out; the step's results are invalid");
}

}  // extern "C"

// ------------------------------------------------- attend_step, no allocation

// The chunk partials and statistics of vkml_attend_step_noalloc: device
// memory of the library itself, so that a call allocates nothing. Each GPU
// holds its own copy until the process ends; host code never passes the
// array's name to a kernel (that is a host-side stand-in, not the device
// address) but the address hipGetSymbolAddress gives per device.
static __device__ __align__(256) uint8_t scratch[VKML_ATTEND_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
void* g_scratch[kMaxDevices] = {};

// Bytes of the partials [heads, chunks, hd] f32, then the statistics
// [heads, chunks, 2] f32 from the next 256-byte boundary.
uint64_t partial_bytes(const vkml_attend_step_params* p) {
    return (static_cast<uint64_t>(p->heads) * p->chunks * p->head_dim * 4 + 255) / 256 * 256;
}

}  // namespace

namespace vkml::abi {

// Called by vkml_init with the chosen device current: the device address of
// this device's scratch.
int attend_scratch_setup(int device) {
    if (device < 0 || device >= kMaxDevices) return fail(VKML_ERROR_DEVICE, "vkml_init: device index out of range");
    if (g_scratch[device]) return VKML_OK;
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) return hip_fail(e != hipSuccess ? e : hipErrorInvalidSymbol, "vkml_init: scratch address");
    g_scratch[device] = ptr;
    return VKML_OK;
}

}  // namespace vkml::abi

extern "C" {

int vkml_attend_step_noalloc(const vkml_attend_step_params* p, const float* qkv, const float* rope_table, void* k_cache,
                             void* v_cache, float* out, void* values, float* scales, const vkml_decode_state* state) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(p, "attend_step_noalloc: null params");
    const uint64_t need = partial_bytes(p) + static_cast<uint64_t>(p->heads) * p->chunks * 8;
    VKML_CHECK_ARG(need <= VKML_ATTEND_SCRATCH_BYTES,
                   "attend_step_noalloc: " + std::to_string(p->heads) + " heads x " + std::to_string(p->chunks) + " chunks of head_dim " +
                       std::to_string(p->head_dim) + " need " + std::to_string(need) + " bytes of partials and statistics, more than the " +
                       std::to_string(VKML_ATTEND_SCRATCH_BYTES) + " bytes of scratch");
    const int device = vkml::abi::device_index();
    VKML_CHECK_ARG(device >= 0 && device < kMaxDevices && g_scratch[device], "attend_step_noalloc: no scratch on this device");
    auto* base = static_cast<uint8_t*>(g_scratch[device]);
    float* partial = reinterpret_cast<float*>(base);
    float* stats = reinterpret_cast<float*>(base + partial_bytes(p));
    // Every chunk slot of the scratch is written by the chunk pass (live
    // results, or a max of -inf past the live keys) before the merge reads
    // it, so nothing left by an earlier call is read.
    if (int r = check_step(p, qkv, rope_table, k_cache, v_cache, partial, stats, out, values, scales, state, "attend_step_noalloc")) return r;
    const ChunkArgs args = step_args(p, qkv, rope_table, k_cache, v_cache, partial, stats, state, nullptr);
    {
        vkml::abi::ProfileScope prof("attend_step");
        launch_chunks(p->head_dim, p->kv_type == VKML_F16, args);
        if (int r = vkml::abi::check_launch("attend_step_noalloc")) return r;
    }
    vkml::abi::ProfileScope prof("attend_merge");
    launch_merge(p->heads, p->head_dim, p->chunks, partial, stats, out, values, scales);
    return vkml::abi::check_launch("attend_step_noalloc");
}

int vkml_attend_o_status(uint32_t* sync, uint32_t* flag_out) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(sync && flag_out, "attend_o_status: null buffer");
    hipStream_t s = vkml::abi::stream();
    uint32_t flag = 0;
    hipError_t e = hipMemcpyAsync(&flag, sync, 4, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return vkml::abi::hip_fail(e, "attend_o_status");
    *flag_out = flag;
    if (flag == 0) return VKML_OK;
    const uint32_t zero = 0;
    e = hipMemcpyAsync(sync, &zero, 4, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return vkml::abi::hip_fail(e, "attend_o_status");
    return VKML_OK;
}

int vkml_attend_o_check(uint32_t* sync) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(sync, "attend_o_check: null buffer");
    uint32_t flag = 0;
    if (int r = vkml_attend_o_status(sync, &flag)) return r;
    if (flag == 0) return VKML_OK;
    return vkml::abi::fail(VKML_ERROR_DEVICE, "attend_step_o: the o GEMV's wait for the merge timed out; the step's results are invalid");
}

}  // extern "C"
