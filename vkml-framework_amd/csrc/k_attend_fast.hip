// k_attend_fast.hip -- decode attention on the matrix cores (attend_fast.hpp),
// the kernels and their C ABI: the tolerance form of the reference's
// attend.comp + attend_merge.comp (src/ops/attention.cpp:54-84), as an
// option beside the bit-exact kernels of k_attend.hip.
//
// One launch: the items (chunk of 128 keys, KV head) first in the grid,
// numbered so that a KV head's items land on one XCD (workgroups are dealt
// to the 8 XCDs round-robin); the last item of each KV head to arrive merges
// that KV head's heads. In a decode step the launch also carries the o
// projection + residual (vkml_attend_step_fast), whose workgroups issue
// their weight loads at once and wait (bounded) for every merge, as in
// vkml_attend_step_fused; the sync words are that call's blocks.
#include <algorithm>

#include "attend_fast.hpp"
#include "device.hpp"
#include "gemv.hpp"
#include "internal.hpp"

using namespace vkml::dev;
using namespace vkml::attend;
using namespace vkml::attend_fast;

namespace {

struct FastLaunch {
    uint32_t items;  // workgroups of the attention, first in the grid
    uint32_t* sync;  // the o GEMV's counters and error flag (null: no o GEMV)
    uint32_t* next;  // the next launch's block, whose o counters this one zeroes (may be null)
    uint32_t* error;
    uint32_t wait_cap;  // polls before the GEMV's wait gives up
};

constexpr int kNoGemv = -1;

// Waits for the workgroup's stores (written through, so visible to every
// XCD), then adds it to counter c; true on every thread for the workgroup
// that arrives last of `arrivals` (which resets the counter).
__device__ __forceinline__ bool arrive_last(uint32_t* c, uint32_t arrivals) {
    __shared__ uint32_t s_last;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
        const bool last = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == arrivals - 1;
        if (last) __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = last;
    }
    __syncthreads();
    return s_last != 0;
}

template <int HD, int GQ, int FMT, bool FULL, int DEEP, bool RUN>
__global__ void __launch_bounds__(kThreads) k_attend_fast(FastArgs a, FastLaunch f, vkml::gemv::GemvArgs g) {
    extern __shared__ uint4 smem[];
    if constexpr (FMT != kNoGemv) {
        if (blockIdx.x >= f.items) {
            const uint32_t wg = blockIdx.x - f.items;
            vkml::gemv::GemvRows<FMT, true, 32, vkml::gemv::kAdd, DEEP ? DEEP : 2, kThreads, false, false, DEEP ? 0 : 1, FULL> rows;
            rows.start(g, wg);
            if (!await_merged(f.sync, wg, a.kv_heads, f.error, f.wait_cap)) return;
            vkml::gemv::stage_activation<kThreads, false, true>(g, smem);
            rows.finish(g, smem, vkml::gemv::staged_ss(smem, g.k));
            return;
        }
    }
    auto& sm = *reinterpret_cast<FastSmem<HD, GQ>*>(smem);
    const uint32_t L = blockIdx.x, kvh = L % a.kv_heads, chunk = L / a.kv_heads;
    if (f.next && L == 0 && threadIdx.x < OSync::kCopies) OSync::counter(f.next, threadIdx.x)[0] = 0u;
    if constexpr (RUN) {
        // Long contexts: item `chunk` is the run of chunks run * chunk ..,
        // its partial in the slot of the first; one merge level.
        const uint32_t first = chunk * a.run;
        const uint32_t kv_len = a.state ? static_cast<uint32_t>(ld_scalar_i32(&a.state->position)) + 1u : a.kv_len;
        if (f.error && L == 0 && threadIdx.x == 0 && kv_len - a.kv_start > a.chunks * kItemKeys)
            __hip_atomic_store(f.error, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t live = min(a.chunks, (kv_len - a.kv_start + kItemKeys - 1) / kItemKeys);
        if (first < live)
            fast_run<HD, GQ>(a, first, min(a.run, live - first), kvh, kv_len, sm, reinterpret_cast<uint8_t*>(smem) + sizeof(FastSmem<HD, GQ>));
        if (!arrive_last(a.arrive + FusedSync::kArriveStride * kvh, (a.chunks + a.run - 1) / a.run)) return;
        fast_merge<HD, GQ>(a, kvh, 0, (live + a.run - 1) / a.run, a.run, -1, reinterpret_cast<float*>(sm.v));
        if (f.sync) {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            if (threadIdx.x < OSync::kCopies)
                __hip_atomic_fetch_add(OSync::counter(f.sync, threadIdx.x), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        return;
    }
    FastLoads<HD> ld;
    // Chunks whose keys are all live at every position the launch serves
    // load before the position is read.
    const bool early = chunk < a.ready;
    if (early) fast_load<HD>(a, chunk, kvh, kItemKeys, ld, sm.v);
    const uint32_t kv_len = a.state ? static_cast<uint32_t>(ld_scalar_i32(&a.state->position)) + 1u : a.kv_len;
    if (f.error && L == 0 && threadIdx.x == 0 && kv_len - a.kv_start > a.chunks * kItemKeys)
        __hip_atomic_store(f.error, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t key0 = a.kv_start + chunk * kItemKeys;
    if (key0 < kv_len) {
        const uint32_t n = min(kItemKeys, kv_len - key0);
        if (!early) fast_load<HD>(a, chunk, kvh, n, ld, sm.v);
        fast_item<HD, GQ>(a, chunk, kvh, n, ld, sm);
    }
    const uint32_t live = min(a.chunks, (kv_len - a.kv_start + kItemKeys - 1) / kItemKeys);
    float* xch = reinterpret_cast<float*>(sm.v);
    if (a.segs > 1) {
        // First level: the segment's last item merges its live chunks into
        // the slot of the segment's first chunk.
        const uint32_t seg = chunk / kSegment;
        if (!arrive_last(a.arrive + FusedSync::kArriveStride * (a.kv_heads + kvh * a.segs + seg), min(kSegment, a.chunks - seg * kSegment)))
            return;
        if (seg * kSegment < live) {
            fast_merge<HD, GQ>(a, kvh, seg * kSegment, min(kSegment, live - seg * kSegment), 1, static_cast<int32_t>(seg * kSegment), xch);
            __syncthreads();  // the exchange area is read before the next merge writes it
        }
        // Second level: the last segment merges the live segments.
        if (!arrive_last(a.arrive + FusedSync::kArriveStride * kvh, a.segs)) return;
        fast_merge<HD, GQ>(a, kvh, 0, (live + kSegment - 1) / kSegment, kSegment, -1, xch);
    } else {
        if (!arrive_last(a.arrive + FusedSync::kArriveStride * kvh, a.chunks)) return;
        fast_merge<HD, GQ>(a, kvh, 0, live, 1, -1, xch);
    }
    if (f.sync) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (threadIdx.x < OSync::kCopies)
            __hip_atomic_fetch_add(OSync::counter(f.sync, threadIdx.x), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

template <int HD, int GQ>
constexpr size_t item_lds() {
    return sizeof(FastSmem<HD, GQ>);
}

// Resident workgroups a CU holds of kernel fn at lds bytes (cached per kernel).
template <int HD, int GQ, int FMT, bool FULL, int DEEP, bool RUN>
int per_cu(size_t lds) {
    static int n = -1;
    static size_t at = 0;
    if (n < 0 || at != lds) {
        const void* fn = reinterpret_cast<const void*>(&k_attend_fast<HD, GQ, FMT, FULL, DEEP, RUN>);
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, kThreads, lds) != hipSuccess) n = 0;
        at = lds;
    }
    return n;
}

// Launches (or with dry, only checks) the one launch; false where the grid
// could not make progress (the o GEMV's waiting workgroups would fill every
// slot) -- nothing is launched then.
template <int HD, int GQ, int FMT, bool FULL, int DEEP, bool RUN>
bool launch_run(const FastArgs& a, const FastLaunch& f, const vkml::gemv::GemvArgs& g, uint32_t gemv_wgs, bool dry) {
    const size_t item = item_lds<HD, GQ>() + (RUN ? kItemKeys * HD * 2 : 0);  // a run's second V tile
    const size_t lds = std::max<size_t>(item, FMT == kNoGemv ? 0 : vkml::gemv::stage_bytes(g.k, false));
    if (gemv_wgs && static_cast<uint64_t>(per_cu<HD, GQ, FMT, FULL, DEEP, RUN>(lds)) * vkml::abi::compute_units() <= gemv_wgs) return false;
    if (dry) return true;
    hipLaunchKernelGGL((k_attend_fast<HD, GQ, FMT, FULL, DEEP, RUN>), dim3(f.items + gemv_wgs), dim3(kThreads), lds, vkml::abi::stream(), a, f,
                       g);
    return true;
}

// Runs of chunks (a.run > 1) take their own kernel: its second register
// set and V tile would cost the one-chunk items their occupancy.
template <int HD, int GQ, int FMT, bool FULL, int DEEP>
bool launch_as(const FastArgs& a, const FastLaunch& f, const vkml::gemv::GemvArgs& g, uint32_t gemv_wgs, bool dry) {
    return a.run > 1 ? launch_run<HD, GQ, FMT, FULL, DEEP, true>(a, f, g, gemv_wgs, dry) : launch_run<HD, GQ, FMT, FULL, DEEP, false>(a, f, g, gemv_wgs, dry);
}

template <int HD, int GQ>
bool launch_gq(const FastArgs& a, const FastLaunch& f, const vkml::gemv::GemvArgs* g, uint32_t b_type, bool dry) {
    if (!g) return launch_as<HD, GQ, kNoGemv, false, 0>(a, f, vkml::gemv::GemvArgs{}, 0, dry);
    const uint32_t gemv_wgs = (g->n + kThreads / 32 - 1) / (kThreads / 32);
    const bool q4k = b_type == VKML_Q4_K, full = g->k % 2048 == 0;
    // o rows of 2048 or 4096 values: every round's weights in flight at once
    if (g->k == 4096)
        return q4k ? launch_as<HD, GQ, VKML_Q4_K, true, 8>(a, f, *g, gemv_wgs, dry) : launch_as<HD, GQ, VKML_Q8_0, true, 8>(a, f, *g, gemv_wgs, dry);
    if (g->k == 2048)
        return q4k ? launch_as<HD, GQ, VKML_Q4_K, true, 4>(a, f, *g, gemv_wgs, dry) : launch_as<HD, GQ, VKML_Q8_0, true, 4>(a, f, *g, gemv_wgs, dry);
    if (q4k) return full ? launch_as<HD, GQ, VKML_Q4_K, true, 0>(a, f, *g, gemv_wgs, dry) : launch_as<HD, GQ, VKML_Q4_K, false, 0>(a, f, *g, gemv_wgs, dry);
    return full ? launch_as<HD, GQ, VKML_Q8_0, true, 0>(a, f, *g, gemv_wgs, dry) : launch_as<HD, GQ, VKML_Q8_0, false, 0>(a, f, *g, gemv_wgs, dry);
}

// Merge levels for `chunks` chunks of kv_heads KV heads: one up to
// kOneLevel chunks, else segments of kSegment when the counters fit a sync
// block.
uint32_t merge_segments(uint32_t chunks, uint32_t kv_heads) {
    if (chunks <= kOneLevel) return 1;
    const uint32_t segs = (chunks + kSegment - 1) / kSegment;
    return kv_heads * (1 + segs) <= FusedSync::kMaxSets ? segs : 1;
}

// Chunks an item takes. One while the items fit two workgroups a CU (every
// item's loads go out at once); past that, runs that bring the items down
// to about that many, each workgroup streaming its chunks with the next
// one's loads in flight (a grid of one chunk an item would run in rounds
// whose loads all go out, and then all compute, together), and at most
// kOneLevel runs a KV head, so that one merge level takes them.
uint32_t run_length(uint32_t chunks, uint32_t kv_heads) {
    const uint64_t slots = 2ull * vkml::abi::compute_units();
    if (static_cast<uint64_t>(chunks) * kv_heads <= slots) return 1;
    const uint32_t by_slots = static_cast<uint32_t>((static_cast<uint64_t>(chunks) * kv_heads + slots - 1) / slots);
    return std::max(by_slots, (chunks + kOneLevel - 1) / kOneLevel);
}

bool launch_fast(uint32_t hd, const FastArgs& a, const FastLaunch& f, const vkml::gemv::GemvArgs* g, uint32_t b_type, bool dry) {
    const bool wide = a.group > 4;
    if (hd == 128) return wide ? launch_gq<128, 8>(a, f, g, b_type, dry) : launch_gq<128, 4>(a, f, g, b_type, dry);
    return wide ? launch_gq<64, 8>(a, f, g, b_type, dry) : launch_gq<64, 4>(a, f, g, b_type, dry);
}

// The shapes the fast form takes: f16 caches, head_dim 64 or 128, at most 8
// query heads a KV head, and a merge of at most 1024 chunks per head.
int check_fast(uint32_t heads, uint32_t kv_heads, uint32_t head_dim, uint32_t kv_type, uint32_t chunks, const char* what) {
    const std::string w(what);
    VKML_CHECK_ARG(kv_heads > 0 && heads % kv_heads == 0 && heads / kv_heads <= 8,
                   w + ": q's " + std::to_string(heads) + " heads must be a multiple of k and v's " + std::to_string(kv_heads) +
                       ", at most 8 a KV head");
    VKML_CHECK_ARG(head_dim == 64 || head_dim == 128, w + ": head_dim " + std::to_string(head_dim) + " is not 64 or 128");
    VKML_CHECK_ARG(kv_type == VKML_F16, w + ": caches must be f16");
    VKML_CHECK_ARG(chunks > 0 && chunks <= 1024, w + ": chunks must be 1 to 1024");
    VKML_CHECK_ARG(kv_heads <= FusedSync::kMaxSets, w + ": at most " + std::to_string(FusedSync::kMaxSets) + " KV heads");
    return VKML_OK;
}

bool o_fusable(const vkml_gemv_dot_params* o, uint32_t heads, uint32_t hd) {
    using namespace vkml::gemv;
    if (!o || o->m != 1 || o->n == 0 || o->k != heads * hd) return false;
    if (o->b_type != VKML_Q4_K && !(o->b_type == VKML_Q8_0 && o->scale_type == VKML_F16)) return false;
    const bool q4k = o->b_type == VKML_Q4_K;
    return (q4k ? code_bytes<VKML_Q4_K>(o->n, o->k) : code_bytes<VKML_Q8_0>(o->n, o->k)) < (1ull << 32) &&
           (q4k ? scale_bytes<VKML_Q4_K, true>(o->n, o->k) : scale_bytes<VKML_Q8_0, true>(o->n, o->k)) < (1ull << 32);
}

}  // namespace

extern "C" {

int vkml_attend_fast(const vkml_attend_params* p, const float* q, const void* k_cache, const void* v_cache, float* partial,
                     float* stats, float* out, void* values, float* scales, uint32_t* sync, const vkml_decode_state* state) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(p, "attend_fast: null params");
    if (int r = check_fast(p->heads, p->kv_heads, p->head_dim, p->kv_type, p->chunks, "attend_fast")) return r;
    VKML_CHECK_ARG(p->capacity > 0 && (state ? p->kv_start < p->capacity : p->kv_start < p->kv_len && p->kv_len - p->kv_start <= p->capacity),
                   "attend_fast: keys " + std::to_string(p->kv_start) + ".." + std::to_string(p->kv_len) + " do not fit the cache of " +
                       std::to_string(p->capacity) + " rows");
    const uint64_t keys = state ? p->capacity - p->kv_start : p->kv_len - p->kv_start;
    VKML_CHECK_ARG(static_cast<uint64_t>(p->chunks) * kItemKeys >= keys,
                   "attend_fast: " + std::to_string(p->chunks) + " chunks of 128 keys do not cover " + std::to_string(keys) + " keys");
    VKML_CHECK_ARG(q && k_cache && v_cache && partial && stats && sync && (out || values), "attend_fast: null buffer");
    VKML_CHECK_ARG(!values || scales, "attend_fast: quantized output needs scales");
    const uint32_t run = run_length(p->chunks, p->kv_heads);
    const FastArgs a{q, k_cache, v_cache, partial, stats, state, p->heads, p->kv_heads, p->heads / p->kv_heads, p->capacity,
                     p->kv_start, p->kv_len, p->chunks, p->scale, p->softcap, 0, FusedSync::arrive(sync, 0),
                     run > 1 ? 1 : merge_segments(p->chunks, p->kv_heads), run, out, static_cast<uint8_t*>(values), scales};
    const FastLaunch f{(p->chunks + run - 1) / run * p->kv_heads, nullptr, nullptr, nullptr, 0};
    vkml::abi::ProfileScope prof("attend_fast");
    launch_fast(p->head_dim, a, f, nullptr, 0, false);
    return vkml::abi::check_launch("attend_fast");
}

int vkml_attend_step_fast_supported(const vkml_attend_step_params* p, const vkml_gemv_dot_params* o) {
    if (!vkml::abi::initialized() || !p || !o) return 0;
    if (p->kv_type != VKML_F16 || (p->head_dim != 64 && p->head_dim != 128) || p->kv_heads == 0 || p->heads % p->kv_heads ||
        p->heads / p->kv_heads > 8 || p->kv_heads > FusedSync::kMaxSets || p->window || !p->prepared || p->chunks == 0 || p->chunks > 1024)
        return 0;
    if (!o_fusable(o, p->heads, p->head_dim)) return 0;
    const uint32_t run = run_length(p->chunks, p->kv_heads);
    const FastArgs a{nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, p->heads, p->kv_heads, p->heads / p->kv_heads, p->capacity,
                     0, 0, p->chunks, p->scale, p->softcap, 0, nullptr, 1, run, nullptr, nullptr, nullptr};
    const FastLaunch f{(p->chunks + run - 1) / run * p->kv_heads, nullptr, nullptr, nullptr, 0};
    if (run > 1) return launch_fast(p->head_dim, a, f, nullptr, 0, true) ? 1 : 0;  // the o GEMV apart
    const vkml::gemv::GemvArgs g{nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, o->n, o->k};
    return launch_fast(p->head_dim, a, f, &g, o->b_type, true) ? 1 : 0;
}

int vkml_attend_step_fast(const vkml_attend_step_params* p, const float* qkv, void* k_cache, void* v_cache, float* partial,
                          float* stats, float* out, void* values, float* scales, const vkml_decode_state* state,
                          const vkml_gemv_dot_params* o, const void* o_values, const void* o_scales, float* x, uint32_t* sync,
                          uint32_t block, uint32_t blocks) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(p, "attend_step_fast: null params");
    if (int r = check_fast(p->heads, p->kv_heads, p->head_dim, p->kv_type, p->chunks, "attend_step_fast")) return r;
    VKML_CHECK_ARG(p->prepared && !p->window,
                   "attend_step_fast: takes prepared steps (q rotated and the new key and value appended by vkml_gemv_rope) without a window");
    VKML_CHECK_ARG(state, "attend_step_fast: needs the decode state");
    VKML_CHECK_ARG(p->capacity > 0 && p->kv_start < p->capacity, "attend_step_fast: kv_start must lie inside the cache");
    VKML_CHECK_ARG(qkv && k_cache && v_cache && partial && stats && values && scales && o_values && o_scales && x && sync,
                   "attend_step_fast: null buffer");
    VKML_CHECK_ARG(blocks >= 2 && block < blocks,
                   "attend_step_fast: block " + std::to_string(block) + " of " + std::to_string(blocks) + " (two blocks at least)");
    VKML_CHECK_ARG(o_fusable(o, p->heads, p->head_dim),
                   "attend_step_fast: the o projection must take the " + std::to_string(p->heads * p->head_dim) +
                       " attention outputs, with q4_K or q8_0 (f16 scales) weights");
    uint32_t* own = sync + static_cast<uint64_t>(block) * FusedSync::kWords;
    uint32_t* next = sync + static_cast<uint64_t>((block + 1) % blocks) * FusedSync::kWords;
    const uint32_t run = run_length(p->chunks, p->kv_heads);
    const FastArgs a{qkv, k_cache, v_cache, partial, stats, state, p->heads, p->kv_heads, p->heads / p->kv_heads, p->capacity,
                     p->kv_start, 0, p->chunks, p->scale, p->softcap, std::min(p->ready_chunks, p->chunks), FusedSync::arrive(own, 0),
                     run > 1 ? 1 : merge_segments(p->chunks, p->kv_heads), run, out, static_cast<uint8_t*>(values), scales};
    if (run > 1) {
        // Runs of chunks: the attention launch, then the o GEMV + residual
        // apart (the run kernel's second register set and V tile leave too
        // few slots for the GEMV's waiting workgroups). The launch zeroes the
        // next block's o counters and reports a position past its chunks on
        // the same flag.
        const FastLaunch f{(p->chunks + run - 1) / run * p->kv_heads, nullptr, next, sync, 0};
        {
            vkml::abi::ProfileScope prof("attend_fast");
            launch_fast(p->head_dim, a, f, nullptr, 0, false);
            if (int r = vkml::abi::check_launch("attend_step_fast")) return r;
        }
        return vkml_gemv_dot_add(o, values, o_values, x, o_scales, scales, x);
    }
    const FastLaunch f{(p->chunks + run - 1) / run * p->kv_heads, own, next, sync, vkml::abi::wait_limit()};
    const vkml::gemv::GemvArgs g{static_cast<const uint4*>(values), scales, o_values, o_scales, nullptr, nullptr, x, x, o->n, o->k};
    vkml::abi::ProfileScope prof("attend_fast");
    VKML_CHECK_ARG(launch_fast(p->head_dim, a, f, &g, o->b_type, false),
                   "attend_step_fast: the o GEMV's workgroups would fill every slot of the GPU (check vkml_attend_step_fast_supported)");
    return vkml::abi::check_launch("attend_step_fast");
}

}  // extern "C"
