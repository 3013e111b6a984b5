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
#include <algorithm>

#include "attend.hpp"
#include "device.hpp"
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
    const uint32_t hl = rest % groups, pair = (rest / groups) * kXcds + pair_lo;
    if (pair >= pairs) return;
    const uint32_t chunk = pair / a.kv_heads, kvh = pair % a.kv_heads, head0 = kvh * G + hl * HPW;
    const uint32_t pos = a.step ? (a.state ? static_cast<uint32_t>(a.state->position) : a.position) : 0u;
    const uint32_t kv_len = a.step ? pos + 1 : (a.state ? static_cast<uint32_t>(a.state->position) + 1u : a.kv_len);
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
    attend_chunk_load<HD, F16>(a, chunk, kvh, kv_len, ld);
    attend_chunk_item<HD, F16, HPW, false>(a, chunk, kvh, hl, pos, kv_len, qv, ld, sm);
}

constexpr uint32_t kMergeMaxChunks = 1024;  // 131072 keys

// The merge as its own launch: head blockIdx.x, element threadIdx.x.
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
k_attend_merge(const float* partial, const float* stats, float* out, uint8_t* values, float* scales, uint32_t chunks, uint32_t hd) {
    __shared__ float s_r[kMergeMaxChunks];   // exp(m_c - M), or -1 for a chunk past the live keys
    __shared__ float s_l[kMergeMaxChunks];   // the chunk's sum of weights
    __shared__ float s_wmax[8];
    merge_head<false>(partial, stats, out, values, scales, blockIdx.x, chunks, chunks, hd, threadIdx.x, s_r, s_l, s_wmax);
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
