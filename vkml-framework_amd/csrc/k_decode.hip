// k_decode.hip -- the decode step's layers in one persistent launch (the
// layer loop of the reference's src/models/llama.cpp:310-395 for one token).
//
// The separate-launch step runs six kernels a layer; each pays its launch,
// the ramp of its first HBM loads, and a tail. Here a grid of two 256-thread
// workgroups per CU stays resident for every layer and walks the same
// phases, separated by grid barriers:
//   P1 q|k|v GEMV, RMSNorm + Q8_0 of x in the prologue (16 rows an item)
//   P2 attention: (chunk, KV head, four query heads) items, K and V of the
//      first loaded before the barrier; the last item of a head group to
//      finish merges the group's chunks (+ Q8_0)
//   P3 o GEMV + residual into x (16 rows an item)
//   P4 gate|up GEMV, RMSNorm + Q8_0 prologue, SwiGLU + Q8_0 of h (32 rows)
//   P5 down GEMV + residual into x (16 rows an item)
// Between phases every workgroup arrives at the barrier, then issues the
// first weight loads of its next GEMV item (they depend on nothing computed
// at run time), then waits: the weights stream while the barrier resolves.
//
// The device code of every phase is the separate kernels' (gemv.hpp,
// attend.hpp), so the arithmetic -- and every bit of x, the KV caches and the
// intermediate values -- is theirs. What differs is how values cross
// workgroups within the launch. Each XCD has its own L2, which may hold a
// stale copy of a line another XCD has since written. So:
// - a producer stores write-through (agent-scope, sc1 stores) and waits for
//   its stores to complete before it arrives at the barrier;
// - every activation that many workgroups read (x, q|k|v, the attention
//   output's and h's Q8_0 codes) gets a buffer of its own for each value it
//   takes in the launch -- x one per residual add, the others one per layer
//   -- so no buffer is read before it is written or written after it is
//   read, no L2 can hold a stale line of it, and its readers load it through
//   L2 (one XCD's first reader fetches it, the rest hit): no memory channel
//   serves every workgroup's read of the same few lines;
// - the chunk partials, each read once by the workgroup that merges its
//   head pair, are read with agent-scope loads.
// The barrier spreads its arrivals over 16 counters (atomic adds to one
// address serialize); wave 0 polls all 16. Every wait is bounded: past the
// spin limit a workgroup sets the sticky error flag, and every workgroup
// that sees it returns, so the grid always drains.
#include <algorithm>

#include "attend.hpp"
#include "device.hpp"
#include "gemv.hpp"
#include "internal.hpp"

using namespace vkml::dev;
using namespace vkml::gemv;
using namespace vkml::attend;

namespace {

constexpr uint32_t kT = 256;           // threads a workgroup
constexpr uint32_t kPerCu = 2;         // resident workgroups a CU
constexpr uint32_t kHd = 128;          // head_dim of this build of the kernel
constexpr uint32_t kLine = 64;         // words between counters (256 bytes)
constexpr uint32_t kBarCounters = 16;  // barrier arrival counters
constexpr uint32_t kMaxPairs = 64;     // merge counters: one per group of four query heads
constexpr uint32_t kSpinCap = 1u << 20;
// Sync words: [0] sticky error flag; counter i of the barrier at
// kLine * (1 + i); merge counter j at kLine * (1 + kBarCounters + j).
constexpr uint32_t kSyncWords = kLine * (1 + kBarCounters + kMaxPairs);
constexpr uint32_t kMaxFfn = 32768;

// Two batches of weights in flight from before the barrier: with 4 rounds a
// batch, a whole item of a K = 4096 row (8 rounds) at 16 lanes a row. The
// gate|up rows prefetch one batch (of both matrices): two, with the RMSNorm
// prologue's loads, would not fit the registers.
using QkvRows = GemvRows<VKML_Q4_K, true, 16, kStore, 4, kT, false, true, 2>;
using ORows = GemvRows<VKML_Q4_K, true, 16, kAdd, 4, kT, false, true, 2>;
using GateUpRows = GemvRows<VKML_Q4_K, true, 8, kSwiglu, 2, kT, true, true, 1>;
using DownRows = GemvRows<VKML_Q4_K, true, 16, kAdd, 8, kT, false, true, 2>;
constexpr int kHpw = 4;  // query heads an attention item: a KV head's whole group
using AttnSmem = AttendSmem<kHd, true, kHpw>;
using AttnLoads = ChunkLoads<kHd, true>;

constexpr uint32_t kMergeLds = 2 * 2 * 1024 * 4 + 4 * 4;  // s_r, s_l of two heads (1024 chunks), s_wmax
constexpr uint32_t kPool = std::max<uint32_t>({static_cast<uint32_t>(sizeof(AttnSmem)), kMergeLds, stage_bytes(kMaxFfn, false),
                                               stage_bytes(4096, true)});

struct DecodeArgs {
    const vkml_decode_layer* layers;
    uint32_t n_layers, d, heads, kv_heads, ffn, capacity, chunks, style, rotate;
    float eps, scale;
    float* x;          // x before layer 0 and after the last layer
    float* xs;         // the 2 * layers - 1 values x takes in between, d floats each
    float* qkv;        // per layer, qkv_n floats
    uint8_t* ac;       // per layer: the attention output's Q8_0 codes (heads * 128) ...
    float* as;         // ... and scales
    uint8_t* hc;       // per layer: h's Q8_0 codes (ffn) ...
    float* hs;         // ... and scales
    float* partial;
    float* stats;
    const float* rope;
    uint32_t* sync;
    const vkml_decode_state* state;
};

// The work area: the intermediate buffers of every layer, each 256-byte
// aligned, in the order of DecodeArgs.
struct WorkLayout {
    uint64_t xs, qkv, ac, as, hc, hs, bytes;
};
__host__ __device__ constexpr uint64_t align256(uint64_t v) { return (v + 255) / 256 * 256; }
__host__ __device__ inline WorkLayout work_layout(uint32_t layers, uint32_t d, uint32_t heads, uint32_t kv_heads, uint32_t ffn) {
    WorkLayout w{};
    const uint64_t qkv_n = static_cast<uint64_t>(heads + 2 * kv_heads) * kHd, att = static_cast<uint64_t>(heads) * kHd;
    w.xs = 0;
    w.qkv = w.xs + align256(4ull * d) * (2 * layers - 1);
    w.ac = w.qkv + align256(4 * qkv_n) * layers;
    w.as = w.ac + align256(att) * layers;
    w.hc = w.as + align256(att / 32 * 4) * layers;
    w.hs = w.hc + align256(ffn) * layers;
    w.bytes = w.hs + align256(ffn / 32 * 4) * layers;
    return w;
}

// The value x takes after v residual adds (v = 0 .. 2 * layers).
__device__ __forceinline__ float* x_at(const DecodeArgs& a, uint32_t v) {
    if (v == 0 || v == 2 * a.n_layers) return a.x;
    return a.xs + (v - 1) * (align256(4ull * a.d) / 4);
}
__device__ __forceinline__ float* qkv_at(const DecodeArgs& a, uint32_t l) {
    return a.qkv + l * (align256(4ull * (a.heads + 2 * a.kv_heads) * kHd) / 4);
}
__device__ __forceinline__ uint8_t* ac_at(const DecodeArgs& a, uint32_t l) { return a.ac + l * align256(a.heads * kHd); }
__device__ __forceinline__ float* as_at(const DecodeArgs& a, uint32_t l) { return a.as + l * (align256(a.heads * kHd / 32 * 4) / 4); }
__device__ __forceinline__ uint8_t* hc_at(const DecodeArgs& a, uint32_t l) { return a.hc + l * align256(a.ffn); }
__device__ __forceinline__ float* hs_at(const DecodeArgs& a, uint32_t l) { return a.hs + l * (align256(a.ffn / 32 * 4) / 4); }

__device__ __forceinline__ uint32_t* bar_counter(uint32_t* sync, uint32_t i) { return sync + kLine * (1 + i); }
__device__ __forceinline__ uint32_t* merge_counter(uint32_t* sync, uint32_t j) { return sync + kLine * (1 + kBarCounters + j); }

// Arrival: every wave's stores have completed (vmcnt(0): for sc1 stores,
// written where every XCD reads), then one atomic add on this workgroup's
// counter. Called by every thread.
__device__ __forceinline__ void arrive(uint32_t* sync, uint32_t wg) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_fetch_add(bar_counter(sync, wg % kBarCounters), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Waits until barrier number nb (1, 2, ...) has every workgroup's arrival:
// counter i then reads nb times its share of the G workgroups. false if the
// wait gave up (the spin limit, or another workgroup's error). Called by
// every thread; ends with a workgroup barrier.
__device__ __forceinline__ bool await_barrier(uint32_t* sync, uint32_t nb, uint32_t G) {
    __shared__ uint32_t s_ok;
    if (threadIdx.x < kWave) {
        const uint32_t i = threadIdx.x % kBarCounters;
        const uint32_t target = nb * (G / kBarCounters + (i < G % kBarCounters ? 1u : 0u));
        bool ok = true;
        for (uint32_t spins = 0;; ++spins) {
            const uint32_t c = __hip_atomic_load(bar_counter(sync, i), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (__all(c >= target)) break;
            if (spins % 256 == 0 && __hip_atomic_load(sync, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) {
                ok = false;
                break;
            }
            if (spins >= kSpinCap) {
                if (threadIdx.x == 0) __hip_atomic_store(sync, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                ok = false;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        if (threadIdx.x == 0) s_ok = ok ? 1u : 0u;
    }
    __syncthreads();
    return s_ok != 0;
}

// Passes a uniform value through an empty asm the compiler cannot see
// into: what is computed from it is computed inside the phase that uses it,
// instead of once before the layer loop and kept in registers (or spilled)
// across every phase.
template <class V>
__device__ __forceinline__ V opaque(V v) {
    asm volatile("" : "+s"(v));
    return v;
}
__device__ __forceinline__ GemvArgs opaque(GemvArgs g) {
    g.n = opaque(g.n);
    g.k = opaque(g.k);
    return g;
}

__device__ __forceinline__ GemvArgs qkv_args(const DecodeArgs& a, const vkml_decode_layer& L, uint32_t l) {
    GemvArgs g{};
    g.b_values = L.qkv_values;
    g.b_scales = L.qkv_scales;
    g.out = qkv_at(a, l);
    g.n = (a.heads + 2 * a.kv_heads) * kHd;
    g.k = a.d;
    g.x = x_at(a, 2 * l);
    g.norm_weight = L.attn_norm;
    g.eps = a.eps;
    return g;
}
__device__ __forceinline__ GemvArgs o_args(const DecodeArgs& a, const vkml_decode_layer& L, uint32_t l) {
    GemvArgs g{};
    g.a_values = reinterpret_cast<const uint4*>(ac_at(a, l));
    g.a_scales = as_at(a, l);
    g.b_values = L.o_values;
    g.b_scales = L.o_scales;
    g.out = x_at(a, 2 * l + 1);
    g.residual = x_at(a, 2 * l);
    g.n = a.d;
    g.k = a.heads * kHd;
    return g;
}
__device__ __forceinline__ GemvArgs gate_up_args(const DecodeArgs& a, const vkml_decode_layer& L, uint32_t l) {
    GemvArgs g{};
    g.b_values = L.gate_values;
    g.b_scales = L.gate_scales;
    g.b2_values = L.up_values;
    g.b2_scales = L.up_scales;
    g.out = nullptr;  // h is needed only as Q8_0
    g.n = a.ffn;
    g.k = a.d;
    g.x = x_at(a, 2 * l + 1);
    g.norm_weight = L.ffn_norm;
    g.eps = a.eps;
    g.out_values = hc_at(a, l);
    g.out_scales = hs_at(a, l);
    return g;
}
__device__ __forceinline__ GemvArgs down_args(const DecodeArgs& a, const vkml_decode_layer& L, uint32_t l) {
    GemvArgs g{};
    g.a_values = reinterpret_cast<const uint4*>(hc_at(a, l));
    g.a_scales = hs_at(a, l);
    g.b_values = L.down_values;
    g.b_scales = L.down_scales;
    g.out = x_at(a, 2 * l + 2);
    g.residual = x_at(a, 2 * l + 1);
    g.n = a.d;
    g.k = a.ffn;
    return g;
}

template <class Rows>
__device__ __forceinline__ uint32_t items_of(const GemvArgs& g) { return (g.n + Rows::kRows - 1) / Rows::kRows; }

// A GEMV phase: the activation staged once, then the workgroup's items wg,
// wg + G, ...; the first item's loads were issued by the caller
// (rows.start(g, wg)) before the barrier.
template <class Rows, bool NORM>
__device__ __forceinline__ void gemv_phase(const GemvArgs& g, Rows& rows, uint32_t wg, uint32_t G, uint4* pool) {
    const uint32_t items = items_of<Rows>(g);
    if (wg >= items) return;
    stage_activation<kT, NORM, false>(g, pool);
    const float2* s_ss = staged_ss(pool, g.k);
    for (uint32_t it = wg;;) {
        rows.finish(g, pool, s_ss);
        it += G;
        if (it >= items) break;
        rows.start(g, it);
    }
}

// Attention items: (chunk, KV head, group of four query heads), numbered as
// k_attend_chunk numbers its workgroups (a (chunk, KV head) pair's head
// groups 8 apart, on one XCD), live chunks only.
struct AttnItems {
    uint32_t group, groups, kv_len, live, pairs, count;
};
__device__ __forceinline__ AttnItems attn_items(const DecodeArgs& a, uint32_t pos) {
    AttnItems r;
    r.group = a.heads / a.kv_heads;
    r.groups = r.group / kHpw;
    r.kv_len = pos + 1;
    r.live = (r.kv_len + kChunk - 1) / kChunk;
    r.pairs = r.live * a.kv_heads;
    r.count = (r.pairs + kXcds - 1) / kXcds * kXcds * r.groups;
    return r;
}
// Item it -> (chunk, KV head, head group); false for a number past the live chunks.
__device__ __forceinline__ bool attn_item(const DecodeArgs& a, const AttnItems& n, uint32_t it, uint32_t& chunk, uint32_t& kvh,
                                          uint32_t& hl) {
    const uint32_t pair_lo = it % kXcds, rest = it / kXcds;
    hl = rest % n.groups;
    const uint32_t pair = (rest / n.groups) * kXcds + pair_lo;
    chunk = pair / a.kv_heads;
    kvh = pair % a.kv_heads;
    return pair < n.pairs;
}
__device__ __forceinline__ ChunkArgs chunk_args(const DecodeArgs& a, const vkml_decode_layer& L, uint32_t l) {
    return ChunkArgs{qkv_at(a, l), a.rope, L.k_cache, L.v_cache, a.partial, a.stats, nullptr, opaque(a.heads), opaque(a.kv_heads),
                     a.heads / a.kv_heads, opaque(a.capacity), 0, 0, 0, opaque(a.chunks), 1, a.style, a.rotate, a.scale, 0.0f,
                     nullptr};
}

// The attention phase. The workgroup's first item's K and V were loaded by
// the caller (ld) before the barrier; later items load their own. After an
// item, its arrival on its head group's counter; the group's last item
// merges the group's heads (two at a time: threads 0-127 one head, 128-255
// the next) and resets the counter for the next layer.
__device__ __forceinline__ void attention_phase(const DecodeArgs& a, const vkml_decode_layer& L, uint32_t l, uint32_t pos,
                                                uint32_t wg, uint32_t G, uint8_t* pool, AttnLoads& ld) {
    const AttnItems n = attn_items(a, pos);
    const ChunkArgs ca = chunk_args(a, L, l);
    AttnSmem& sm = *reinterpret_cast<AttnSmem*>(pool);
    __shared__ uint32_t s_last;
    for (uint32_t it = wg; it < n.count; it += G) {
        uint32_t chunk, kvh, hl;
        if (!attn_item(a, n, it, chunk, kvh, hl)) continue;
        if (it != wg) attend_chunk_load<kHd, true>(ca, chunk, kvh, n.kv_len, ld);
        QLoads<kHd, kHpw> qv;  // q comes from this launch's q|k|v phase: loaded after the barrier
        attend_q_load<kHd, kHpw>(ca, kvh, hl, pos, qv);
        attend_chunk_item<kHd, true, kHpw, true, 16>(ca, chunk, kvh, hl, pos, n.kv_len, qv, ld, sm);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        const uint32_t j = kvh * n.groups + hl;
        if (threadIdx.x == 0) {
            const uint32_t before = __hip_atomic_fetch_add(merge_counter(a.sync, j), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_last = before + 1 == n.live ? 1u : 0u;
        }
        __syncthreads();
        if (s_last) {
            const uint32_t half = threadIdx.x / kHd, d = threadIdx.x % kHd;
            float* s_r = reinterpret_cast<float*>(pool) + half * 2 * 1024;
            float* s_l = s_r + 1024;
            float* s_wmax = reinterpret_cast<float*>(pool) + 4 * 1024 + half * 2;
#pragma unroll
            for (int hp = 0; hp < kHpw; hp += 2) {
                merge_head<true, 16>(a.partial, a.stats, nullptr, ac_at(a, l), as_at(a, l), kvh * n.group + hl * kHpw + hp + half,
                                     a.chunks, n.live, kHd, d, s_r, s_l, s_wmax);
                __syncthreads();
            }
            if (threadIdx.x == 0) __hip_atomic_store(merge_counter(a.sync, j), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();  // the pool is free for the next item
    }
}

__global__ void __launch_bounds__(kT) __attribute__((amdgpu_waves_per_eu(kPerCu))) k_decode_layers(DecodeArgs a) {
    __shared__ __align__(16) uint8_t pool[kPool];
    uint4* pool4 = reinterpret_cast<uint4*>(pool);
    const uint32_t G = gridDim.x, wg = blockIdx.x;
    const uint32_t pos = static_cast<uint32_t>(a.state->position);
    uint32_t nb = 0;
    // Each phase's rows are started before the barrier that precedes the
    // phase. start() is unconditional (a workgroup without an item of the
    // phase loads clamped rows and never uses them), and each phase's rows
    // are local to it, so no row registers stay live outside their phase.
    // Each phase reads the layer's pointers itself (through a laundered
    // index), so they are not all held in scalar registers across the layer.
    for (uint32_t layer = 0; layer < a.n_layers; ++layer) {
        {
            const vkml_decode_layer& L = a.layers[opaque(layer)];
            // x of layer 0 comes from the previous launch (the embedding).
            QkvRows rows;
            if (layer > 0) arrive(a.sync, wg);
            const GemvArgs gq = opaque(qkv_args(a, L, layer));
            rows.start(gq, wg);
            if (layer > 0 && !await_barrier(a.sync, ++nb, G)) return;
            gemv_phase<QkvRows, true>(gq, rows, wg, G, pool4);
        }

        {
            // The first item's K and V load while the barrier resolves.
            const vkml_decode_layer& L = a.layers[opaque(layer)];
            AttnLoads ld;
            arrive(a.sync, wg);
            const uint32_t p = opaque(pos);
            const AttnItems n = attn_items(a, p);
            uint32_t chunk, kvh, hl;
            if (wg < n.count && attn_item(a, n, wg, chunk, kvh, hl))
                attend_chunk_load<kHd, true>(chunk_args(a, L, layer), chunk, kvh, n.kv_len, ld);
            if (!await_barrier(a.sync, ++nb, G)) return;
            attention_phase(a, L, layer, p, wg, G, pool, ld);
        }

        {
            const vkml_decode_layer& L = a.layers[opaque(layer)];
            ORows rows;
            arrive(a.sync, wg);
            const GemvArgs go = opaque(o_args(a, L, layer));
            rows.start(go, wg);
            if (!await_barrier(a.sync, ++nb, G)) return;
            gemv_phase<ORows, false>(go, rows, wg, G, pool4);
        }
        {
            const vkml_decode_layer& L = a.layers[opaque(layer)];
            GateUpRows rows;
            arrive(a.sync, wg);
            const GemvArgs gg = opaque(gate_up_args(a, L, layer));
            rows.start(gg, wg);
            if (!await_barrier(a.sync, ++nb, G)) return;
            gemv_phase<GateUpRows, true>(gg, rows, wg, G, pool4);
        }
        {
            const vkml_decode_layer& L = a.layers[opaque(layer)];
            DownRows rows;
            arrive(a.sync, wg);
            const GemvArgs gd = opaque(down_args(a, L, layer));
            rows.start(gd, wg);
            if (!await_barrier(a.sync, ++nb, G)) return;
            gemv_phase<DownRows, false>(gd, rows, wg, G, pool4);
        }
    }
}

// Zeroes the barrier and merge counters (the words after the error flag).
__global__ void k_sync_reset(uint32_t* sync) {
    for (uint32_t i = kLine + blockIdx.x * blockDim.x + threadIdx.x; i < kSyncWords; i += gridDim.x * blockDim.x) sync[i] = 0;
}

uint32_t grid_size() {
    static int cached_device = -1;
    static uint32_t cached = 0;
    if (cached_device != vkml::abi::device_index()) {
        int per_cu = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_decode_layers, kT, 0) != hipSuccess) per_cu = 0;
        cached = std::min<uint32_t>(static_cast<uint32_t>(std::max(per_cu, 0)), kPerCu) * vkml::abi::compute_units();
        cached -= cached % kXcds;
        cached_device = vkml::abi::device_index();
    }
    return cached;
}

}  // namespace

extern "C" {

uint64_t vkml_decode_sync_bytes(const vkml_decode_layers_params*) { return static_cast<uint64_t>(kSyncWords) * 4; }

uint64_t vkml_decode_work_bytes(const vkml_decode_layers_params* p) {
    if (!p || p->layers == 0) return 0;
    return work_layout(p->layers, p->hidden, p->heads, p->kv_heads, p->ffn).bytes;
}

int vkml_decode_layers(const vkml_decode_layers_params* p, const vkml_decode_layer* layers, const vkml_decode_buffers* b,
                       const vkml_decode_state* state) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(p && b, "decode_layers: null params");
    VKML_CHECK_ARG(p->layers > 0, "decode_layers: no layers");
    VKML_CHECK_ARG(p->weight_type == VKML_Q4_K, "decode_layers: weights must be q4_K");
    VKML_CHECK_ARG(p->kv_type == VKML_F16, "decode_layers: the KV caches must be f16");
    VKML_CHECK_ARG(p->head_dim == kHd, "decode_layers: head_dim must be 128");
    VKML_CHECK_ARG(p->kv_heads > 0 && p->heads % p->kv_heads == 0 && (p->heads / p->kv_heads) % kHpw == 0,
                   "decode_layers: each KV head needs a multiple of 4 query heads");
    VKML_CHECK_ARG(p->heads / kHpw <= kMaxPairs, "decode_layers: too many query heads");
    VKML_CHECK_ARG(p->hidden % 256 == 0 && p->hidden > 0 && p->hidden <= 4096, "decode_layers: hidden must be a multiple of 256 up to 4096");
    VKML_CHECK_ARG(p->heads * kHd % 256 == 0 && p->heads * kHd <= kMaxK, "decode_layers: heads * head_dim must be a multiple of 256");
    VKML_CHECK_ARG(p->ffn % 256 == 0 && p->ffn > 0 && p->ffn <= kMaxFfn, "decode_layers: ffn must be a multiple of 256 up to 32768");
    VKML_CHECK_ARG(p->capacity > 0 && static_cast<uint64_t>(p->chunks) * kChunk >= p->capacity && p->chunks <= 1024,
                   "decode_layers: chunks must cover the cache (at most 1024)");
    VKML_CHECK_ARG(layers && state && b->x && b->partial && b->stats && b->work && b->rope_table && b->sync,
                   "decode_layers: null buffer");
    const uint32_t G = grid_size();
    VKML_CHECK_ARG(G > 0, "decode_layers: the kernel does not fit on this device");
    const WorkLayout w = work_layout(p->layers, p->hidden, p->heads, p->kv_heads, p->ffn);
    uint8_t* work = static_cast<uint8_t*>(b->work);
    DecodeArgs a{layers, p->layers, p->hidden, p->heads, p->kv_heads, p->ffn, p->capacity, p->chunks, p->rope_style, p->rotate,
                 p->eps, p->scale, b->x, reinterpret_cast<float*>(work + w.xs), reinterpret_cast<float*>(work + w.qkv),
                 work + w.ac, reinterpret_cast<float*>(work + w.as), work + w.hc, reinterpret_cast<float*>(work + w.hs),
                 b->partial, b->stats, b->rope_table, b->sync, state};
    vkml::abi::ProfileScope prof("decode_layers");
    hipStream_t s = vkml::abi::stream();
    hipLaunchKernelGGL(k_sync_reset, dim3(4), dim3(256), 0, s, b->sync);
    hipLaunchKernelGGL(k_decode_layers, dim3(G), dim3(kT), 0, s, a);
    return vkml::abi::check_launch("decode_layers");
}

int vkml_decode_layers_check(uint32_t* sync) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(sync, "decode_layers_check: null buffer");
    hipStream_t s = vkml::abi::stream();
    uint32_t flag = 0;
    hipError_t e = hipMemcpyAsync(&flag, sync, 4, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return vkml::abi::hip_fail(e, "decode_layers_check");
    if (flag == 0) return VKML_OK;
    const uint32_t zero = 0;
    e = hipMemcpyAsync(sync, &zero, 4, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return vkml::abi::hip_fail(e, "decode_layers_check");
    return vkml::abi::fail(VKML_ERROR_DEVICE, "decode_layers: a grid barrier timed out (the grid was not resident at once); "
                                              "the step's results are invalid");
}

}  // extern "C"
