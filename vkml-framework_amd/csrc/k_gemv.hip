// k_gemv.hip -- quantized matrix-vector products for decoding (the
// reference's shaders/gemv_dot.comp and gemv.comp), written for gfx950.
//
// The int8 path's device code (mapping, bit-exact order) is in gemv.hpp;
// here are its kernels, their launch shapes and the C ABI. 16 lanes a row
// are used when 8 would leave SIMDs idle (the N = 4096 projections of a 7B
// model: 4096 rows x 16 lanes is one wave per SIMD).
#include <algorithm>

#include "device.hpp"
#include "gemv.hpp"
#include "internal.hpp"

using namespace vkml::dev;
using namespace vkml::gemv;

namespace {

template <int FMT, bool F16S, int LPR, int EPI, int B, uint32_t T, int NORM, bool QOUT, bool FULL, int PRE = 1>
__global__ void __launch_bounds__(T) k_gemv_dot(GemvArgs g) {
    extern __shared__ uint4 smem[];
    GemvRows<FMT, F16S, LPR, EPI, B, T, QOUT, false, PRE, FULL> rows;
    if constexpr (PRE == 0) {
        // Every weight load of the row is issued at once: the activation's
        // loads go first, so that staging waits for them alone.
        StageLoads<T, NORM> act;
        stage_load<T, NORM, false>(g, act);
        rows.start(g, blockIdx.x);
        stage_store<T, NORM, false>(g, smem, act);
    } else if constexpr (NORM != 0) {
        // (the norm prologue's loads after the weights': measured faster)
        rows.start(g, blockIdx.x);  // the first batch of weights is in flight while the activation is staged
        stage_activation<T, NORM, false>(g, smem);
    } else {
        StageLoads<T, false> act;
        stage_load<T, false, false>(g, act);  // first: staging waits for these alone
        rows.start(g, blockIdx.x);            // the first batch of weights is in flight while the activation is staged
        stage_store<T, false, false>(g, smem, act);
    }
    rows.finish(g, smem, staged_ss(smem, g.k));
}

// Rows of up to 4096 values at 32 lanes a row: every round of the row is
// one batch, all in flight at once (T threads, T / 32 rows a workgroup).
template <int FMT, bool F16S, int EPI, int NORM, bool QOUT, uint32_t T>
int launch_deep(const GemvArgs& g, const char* label) {
    const dim3 grid((g.n + T / 32 - 1) / (T / 32));
    const size_t lds = stage_bytes(g.k, NORM != 0);
    if (g.k <= 2048) {
        if (g.k == 2048)
            hipLaunchKernelGGL((k_gemv_dot<FMT, F16S, 32, EPI, 4, T, NORM, QOUT, true, 0>), grid, dim3(T), lds, vkml::abi::stream(), g);
        else
            hipLaunchKernelGGL((k_gemv_dot<FMT, F16S, 32, EPI, 4, T, NORM, QOUT, false, 0>), grid, dim3(T), lds, vkml::abi::stream(), g);
    } else {
        if (g.k == 4096)
            hipLaunchKernelGGL((k_gemv_dot<FMT, F16S, 32, EPI, 8, T, NORM, QOUT, true, 0>), grid, dim3(T), lds, vkml::abi::stream(), g);
        else
            hipLaunchKernelGGL((k_gemv_dot<FMT, F16S, 32, EPI, 8, T, NORM, QOUT, false, 0>), grid, dim3(T), lds, vkml::abi::stream(), g);
    }
    return vkml::abi::check_launch(label);
}

// The batch pipeline (B rounds a batch, two batches in flight), T threads.
template <int FMT, bool F16S, int LPR, int EPI, int NORM, bool QOUT, uint32_t T>
int launch_batched(const GemvArgs& g, const char* label) {
    constexpr int B = LPR == 16 ? 4 : 2;  // rounds per batch (2 measured best at 32 lanes)
    const dim3 grid((g.n + T / LPR - 1) / (T / LPR));
    const size_t lds = stage_bytes(g.k, NORM != 0);
    // Whole pairs of whole batches (K a multiple of 1024 B) need no per-lane
    // tail check and no per-round test (q4_K and q8_0 kernels are built both
    // ways).
    constexpr bool kWhole = FMT == VKML_Q4_K || FMT == VKML_Q8_0;
    if (kWhole && g.k % (1024 * B) == 0)
        hipLaunchKernelGGL((k_gemv_dot<FMT, F16S, LPR, EPI, B, T, NORM, QOUT, kWhole>), grid, dim3(T), lds, vkml::abi::stream(), g);
    else
        hipLaunchKernelGGL((k_gemv_dot<FMT, F16S, LPR, EPI, B, T, NORM, QOUT, false>), grid, dim3(T), lds, vkml::abi::stream(), g);
    return vkml::abi::check_launch(label);
}

template <int FMT, bool F16S, int LPR, int EPI, int NORM, bool QOUT>
int launch(const GemvArgs& g, const char* label) {
    // (512 threads with the norm prologue at 32 lanes: half the workgroups
    // redo RMSNorm + Q8_0 of x, each over twice the threads)
    constexpr uint32_t T = QOUT ? 32 * LPR : LPR == 32 ? (NORM != 0 ? 512 : 256) : 128;
    vkml::abi::ProfileScope prof(label);
    const uint32_t cus = vkml::abi::compute_units();
    constexpr bool kWhole = FMT == VKML_Q4_K || FMT == VKML_Q8_0;
    if constexpr (kWhole && LPR == 32) {
        if (g.k <= 4096) {
            // With the norm prologue, which every workgroup computes over the
            // whole row: 24 rows a workgroup where that makes one workgroup a
            // compute unit (the N = 6144 q|k|v projection of a 7B model).
            if constexpr (NORM != 0) {
                if ((g.n + 15) / 16 > cus && (g.n + 23) / 24 <= cus) {
                    // q4_K rows of 4096 with the store epilogue (a decode
                    // step's q|k|v): 16 lanes a row over 384 threads, the
                    // same 24 rows a workgroup. 32 lanes load each 16-byte
                    // code group twice (lanes l and l ^ 2), 16 lanes once, so
                    // a compute unit queues half the code loads (measured:
                    // 606.6 against 605.3 tokens/s at cfg5).
                    if constexpr (FMT == VKML_Q4_K && EPI == kStore) {
                        if (g.k == 4096) {
                            hipLaunchKernelGGL((k_gemv_dot<FMT, F16S, 16, EPI, 8, 384, NORM, QOUT, true, 0>), dim3((g.n + 23) / 24),
                                               dim3(384), stage_bytes(g.k, true), vkml::abi::stream(), g);
                            return vkml::abi::check_launch(label);
                        }
                    }
                    return launch_deep<FMT, F16S, EPI, NORM, QOUT, 768>(g, label);
                }
            }
            return launch_deep<FMT, F16S, EPI, NORM, QOUT, T>(g, label);
        }
    }
    return launch_batched<FMT, F16S, LPR, EPI, NORM, QOUT, T>(g, label);
}

template <int FMT, bool F16S, int EPI, int NORM, bool QOUT>
int dispatch(const GemvArgs& g, const char* label) {
    // 8 lanes a row unless that leaves fewer than one wave per SIMD; 32
    // (q4_K, q8_0) when 16 would leave fewer than two, so that one wave's
    // arithmetic overlaps another's loads (the N = 4096 and 6144 projections
    // of a 7B model: measured 13-18% faster than 16 lanes).
    const uint64_t simds = 4ull * std::max<uint32_t>(vkml::abi::compute_units(), 1);
    if constexpr (FMT == VKML_Q4_K || FMT == VKML_Q8_0) {
        // (their buffer loads address a matrix under 4 GiB)
        if (code_bytes<FMT>(g.n, g.k) >= (1ull << 32) || scale_bytes<FMT, F16S>(g.n, g.k) >= (1ull << 32))
            return vkml::abi::fail(VKML_ERROR_UNSUPPORTED, std::string(label) + ": a matrix of 4 GiB or more");
        if constexpr (!QOUT) {
            if ((g.n + 3) / 4 < 2 * simds) return launch<FMT, F16S, 32, EPI, NORM, QOUT>(g, label);
        }
    }
    if ((g.n + 7) / 8 < simds) return launch<FMT, F16S, 16, EPI, NORM, QOUT>(g, label);
    return launch<FMT, F16S, 8, EPI, NORM, QOUT>(g, label);
}

template <int EPI, int NORM = 0, bool QOUT = false>
int dispatch_format(uint32_t b_type, uint32_t scale_type, const GemvArgs& g, const char* label) {
    const bool f16 = scale_type == VKML_F16;
    switch (b_type) {
        case VKML_Q8_0: return f16 ? dispatch<VKML_Q8_0, true, EPI, NORM, QOUT>(g, label) : dispatch<VKML_Q8_0, false, EPI, NORM, QOUT>(g, label);
        case VKML_Q4_0: return f16 ? dispatch<VKML_Q4_0, true, EPI, NORM, QOUT>(g, label) : dispatch<VKML_Q4_0, false, EPI, NORM, QOUT>(g, label);
        case VKML_Q4_1: return f16 ? dispatch<VKML_Q4_1, true, EPI, NORM, QOUT>(g, label) : dispatch<VKML_Q4_1, false, EPI, NORM, QOUT>(g, label);
        case VKML_Q4_K: return dispatch<VKML_Q4_K, true, EPI, NORM, QOUT>(g, label);
        default: return vkml::abi::fail(VKML_ERROR_UNSUPPORTED, std::string(label) + ": no int8 kernel for weight type " + std::to_string(b_type));
    }
}

int check_dot_params(const vkml_gemv_dot_params* p, const char* what, bool any_k = false) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(p, std::string(what) + ": null params");
    VKML_CHECK_ARG(p->b_type == VKML_Q8_0 || p->b_type == VKML_Q4_0 || p->b_type == VKML_Q4_1 || p->b_type == VKML_Q4_K,
                   std::string(what) + ": weights must be q8_0, q4_0, q4_1 or q4_K, got type " + std::to_string(p->b_type));
    VKML_CHECK_ARG(p->b_type == VKML_Q4_K || p->scale_type == VKML_F16 || p->scale_type == VKML_F32,
                   std::string(what) + ": scales must be f16 or f32");
    const uint32_t unit = p->b_type == VKML_Q4_K ? 256 : 32;
    VKML_CHECK_ARG(p->k > 0 && p->k % unit == 0 && (any_k || p->k <= kMaxK),
                   std::string(what) + ": k = " + std::to_string(p->k) + " must be a positive multiple of " +
                       std::to_string(unit) + (any_k ? std::string() : " up to " + std::to_string(kMaxK)));
    return VKML_OK;
}

// ---------------------------------------------------------------- several rows

// gemv_dot for 2 .. 8 activation rows in one launch (gemv_dot.comp handles
// its M rows in one dispatch): each round of a weight row is loaded once and
// applied to every activation row, each row with its own accumulators in
// the single-row kernel's order (the same lanes, terms and halving tree).
// LPR lanes an output row (32 for q8_0 and q4_K, 16 for q4_0 and q4_1);
// the activation codes are read from memory (the workgroup's rows share
// them in L1), the next round's weights in flight during this one.
template <int FMT, bool F16S, int LPR, bool FULL>
__global__ void __launch_bounds__(256) k_gemv_dot_rows(GemvArgs g, uint32_t m) {
    constexpr int NS = Plan<FMT, LPR>::NS;
    constexpr uint32_t kRows = 256 / LPR;
    const uint32_t t = thread_index(), l = t % LPR, grp = t / LPR;
    const uint32_t out_row = blockIdx.x * kRows + grp, row = min(out_row, g.n - 1);
    const uint32_t K = g.k, halves = K / 16, rounds = (halves + 31) / 32;
    const Q4kField jf = q4k_field((l % 16) / 2);
    float acc[8][NS];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int e = 0; e < NS; ++e) acc[i][e] = 0.0f;
    RoundW<FMT, LPR> w;
    load_round<FMT, F16S, LPR>(g.b_values, g.b_scales, K, row, 0, l, w);
    for (uint32_t r = 0; r < rounds; ++r) {
        RoundW<FMT, LPR> next;
        load_round<FMT, F16S, LPR>(g.b_values, g.b_scales, K, row, min(r + 1, rounds - 1), l, next);
#pragma unroll
        for (uint32_t i = 0; i < 8; ++i) {
            if (i >= m) break;
            RoundA<FMT, LPR> x;
#pragma unroll
            for (int e = 0; e < NS; ++e) {
                const uint32_t hb = min(32 * r + acc_index<FMT, LPR>(l, e), halves - 1);
                x.a[e] = ldg(g.a_values + static_cast<uint64_t>(i) * halves + hb);
                x.ss[e] = make_float2(static_cast<float>(byte_sum(x.a[e])), ldg(g.a_scales + static_cast<uint64_t>(i) * (K / 32) + hb / 2));
            }
            round_terms<FMT, F16S, LPR, FULL>(w, x, r, l, K, jf, acc[i]);
        }
        w = next;
    }
#pragma unroll
    for (uint32_t i = 0; i < 8; ++i) {
        if (i >= m) break;
        const float v = row_tree<FMT, LPR>(acc[i]);
        // + residual (one activation row): add(x, y), llama.cpp:374,386
        if (l == 0 && out_row < g.n) g.out[static_cast<uint64_t>(i) * g.n + out_row] = g.residual ? ldg(g.residual + out_row) + v : v;
    }
}

template <int FMT, bool F16S>
int launch_rows(const GemvArgs& g, uint32_t m) {
    constexpr int LPR = FMT == VKML_Q8_0 || FMT == VKML_Q4_K ? 32 : 16;
    const dim3 grid((g.n + 256 / LPR - 1) / (256 / LPR));
    vkml::abi::ProfileScope prof("gemv_dot");
    if (g.k % 512 == 0) hipLaunchKernelGGL((k_gemv_dot_rows<FMT, F16S, LPR, true>), grid, dim3(256), 0, vkml::abi::stream(), g, m);
    else hipLaunchKernelGGL((k_gemv_dot_rows<FMT, F16S, LPR, false>), grid, dim3(256), 0, vkml::abi::stream(), g, m);
    return vkml::abi::check_launch("gemv_dot");
}

int dispatch_rows(uint32_t fmt, uint32_t st, const GemvArgs& g, uint32_t m) {
    const bool f16 = st == VKML_F16;
    switch (fmt) {
        case VKML_Q8_0: return f16 ? launch_rows<VKML_Q8_0, true>(g, m) : launch_rows<VKML_Q8_0, false>(g, m);
        case VKML_Q4_0: return f16 ? launch_rows<VKML_Q4_0, true>(g, m) : launch_rows<VKML_Q4_0, false>(g, m);
        case VKML_Q4_1: return f16 ? launch_rows<VKML_Q4_1, true>(g, m) : launch_rows<VKML_Q4_1, false>(g, m);
        default: return launch_rows<VKML_Q4_K, true>(g, m);
    }
}

// ---------------------------------------------------------------- float path

// gemv.comp's order: 32 lanes per output, lane l taking the 4-element
// groups l, l + 32, ... of its row (dot(a4, w) summed left to right), then
// the halving tree over the 32 lanes (gemv.comp:117-212). Two rows a wave.
// Batch blockIdx.y multiplies its a by float b's batch y / b_group.
template <int BT>
__global__ void __launch_bounds__(256) k_gemv_float(const float* a, uint32_t m, const void* b, const void* bs, uint32_t st,
                                                    float* out, uint32_t n, uint32_t k, uint32_t b_group, uint64_t b_stride) {
#pragma clang fp contract(off)
    const uint32_t z = blockIdx.y;
    a += static_cast<uint64_t>(z) * m * k;
    out += static_cast<uint64_t>(z) * m * n;
    if constexpr (BT <= VKML_BF16) {
        const uint64_t off = static_cast<uint64_t>(z / b_group) * b_stride * (BT == VKML_F32 ? 4 : 2);
        b = static_cast<const uint8_t*>(b) + off;
    }
    const uint32_t lane = threadIdx.x % 32;
    const uint32_t row = blockIdx.x * (blockDim.x / 32) + threadIdx.x / 32;
    const uint32_t r = min(row, n - 1);
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    const auto w_at = [&](uint64_t col) -> float {
        if constexpr (BT == VKML_F32) return static_cast<const float*>(b)[static_cast<uint64_t>(r) * k + col];
        else return weight_value(BT, st, b, bs, k, r, col);
    };
    if (k % 4 == 0) {
        for (uint32_t i = lane; i < k / 4; i += 32) {
            const float w0 = w_at(4 * i), w1 = w_at(4 * i + 1), w2 = w_at(4 * i + 2), w3 = w_at(4 * i + 3);
#pragma unroll
            for (uint32_t q = 0; q < 8; ++q) {
                if (q < m) {
                    const float* ar = a + static_cast<uint64_t>(q) * k + 4 * i;
                    acc[q] += ar[0] * w0 + ar[1] * w1 + ar[2] * w2 + ar[3] * w3;
                }
            }
        }
    } else {
        for (uint32_t col = lane; col < k; col += 32) {
            const float w = w_at(col);
#pragma unroll
            for (uint32_t q = 0; q < 8; ++q)
                if (q < m) acc[q] += a[static_cast<uint64_t>(q) * k + col] * w;
        }
    }
#pragma unroll
    for (uint32_t q = 0; q < 8; ++q) {
        if (q >= m) break;
        const float v = tree_to_first<32>(acc[q]);  // strides 16 .. 1 toward the row's lane 0
        if (lane == 0 && row < n) out[static_cast<uint64_t>(q) * n + row] = v;
    }
}

}  // namespace

extern "C" {

int vkml_gemv_dot(const vkml_gemv_dot_params* p, const void* a_values, const void* b_values, float* out,
                  const void* b_scales, const float* a_scales) {
    if (int r = check_dot_params(p, "gemv_dot", true)) return r;
    VKML_CHECK_ARG(p->m >= 1 && p->m <= 8, "gemv_dot: m must be 1 to 8, got " + std::to_string(p->m));
    if (p->n == 0) return VKML_OK;
    VKML_CHECK_ARG(a_values && b_values && out && b_scales && a_scales, "gemv_dot: null buffer");
    if (p->m > 1 || p->k > kMaxK) {
        const GemvArgs g{static_cast<const uint4*>(a_values), a_scales, b_values, b_scales, nullptr, nullptr, out, nullptr, p->n, p->k};
        return dispatch_rows(p->b_type, p->scale_type, g, p->m);
    }
    const GemvArgs g{static_cast<const uint4*>(a_values), a_scales, b_values, b_scales, nullptr, nullptr, out, nullptr, p->n, p->k};
    return dispatch_format<kStore>(p->b_type, p->scale_type, g, "gemv_dot");
}

int vkml_gemv_dot_add(const vkml_gemv_dot_params* p, const void* a_values, const void* b_values, float* out,
                      const void* b_scales, const float* a_scales, const float* residual) {
    if (int r = check_dot_params(p, "gemv_dot_add", true)) return r;
    VKML_CHECK_ARG(p->m == 1, "gemv_dot_add: m must be 1");
    if (p->n == 0) return VKML_OK;
    VKML_CHECK_ARG(a_values && b_values && out && b_scales && a_scales && residual, "gemv_dot_add: null buffer");
    GemvArgs g{static_cast<const uint4*>(a_values), a_scales, b_values, b_scales, nullptr, nullptr, out, residual, p->n, p->k};
    if (p->k > kMaxK) return dispatch_rows(p->b_type, p->scale_type, g, 1);  // the activation read from memory
    return dispatch_format<kAdd>(p->b_type, p->scale_type, g, "gemv_dot_add");
}

int vkml_gemv_dot_swiglu(const vkml_gemv_dot_params* p, const void* a_values, const float* a_scales,
                         const void* gate_values, const void* gate_scales, const void* up_values,
                         const void* up_scales, float* h) {
    if (int r = check_dot_params(p, "gemv_dot_swiglu")) return r;
    VKML_CHECK_ARG(p->m == 1, "gemv_dot_swiglu: m must be 1");
    if (p->n == 0) return VKML_OK;
    VKML_CHECK_ARG(a_values && a_scales && gate_values && gate_scales && up_values && up_scales && h,
                   "gemv_dot_swiglu: null buffer");
    GemvArgs g{static_cast<const uint4*>(a_values), a_scales, gate_values, gate_scales, up_values, up_scales, h, nullptr, p->n, p->k};
    return dispatch_format<kSwiglu>(p->b_type, p->scale_type, g, "gemv_dot_swiglu");
}

int vkml_gemv_fused(const vkml_gemv_fused_params* p, const void* a, const float* a_scales, const float* norm_weight,
                    const void* b_values, const void* b_scales, const void* b2_values, const void* b2_scales,
                    const float* residual, float* out, void* out_values, float* out_scales) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(p, "gemv_fused: null params");
    const vkml_gemv_dot_params dp{1, p->n, p->k, p->b_type, p->scale_type};
    if (int r = check_dot_params(&dp, "gemv_fused")) return r;
    VKML_CHECK_ARG(p->epilogue <= 2, "gemv_fused: epilogue must be 0 (store), 1 (+ residual) or 2 (SwiGLU)");
    VKML_CHECK_ARG(!p->quantize_out || p->epilogue == 2, "gemv_fused: quantize_out needs the SwiGLU epilogue");
    VKML_CHECK_ARG(!p->quantize_out || p->n % 32 == 0, "gemv_fused: quantize_out needs n a multiple of 32");
    VKML_CHECK_ARG(p->norm <= 2, "gemv_fused: norm must be 0 (quantized input), 1 (RMSNorm + Q8_0) or 2 (Q8_0)");
    VKML_CHECK_ARG(!p->norm || p->k <= 4096, "gemv_fused: the RMSNorm / Q8_0 prologue takes k up to 4096");
    VKML_CHECK_ARG(!(p->norm && p->epilogue == 1), "gemv_fused: the RMSNorm / Q8_0 prologue goes with the store or SwiGLU epilogue");
    VKML_CHECK_ARG(p->norm != 2 || p->epilogue == 0, "gemv_fused: the plain Q8_0 prologue (norm 2) goes with the store epilogue");
    if (p->n == 0) return VKML_OK;
    VKML_CHECK_ARG(a && b_values && b_scales && out, "gemv_fused: null buffer");
    VKML_CHECK_ARG(p->norm == 1 ? norm_weight != nullptr : p->norm == 2 || a_scales != nullptr,
                   "gemv_fused: the input needs its norm weight or scales");
    VKML_CHECK_ARG(p->epilogue != 1 || residual, "gemv_fused: the residual epilogue needs the residual");
    VKML_CHECK_ARG(p->epilogue != 2 || (b2_values && b2_scales), "gemv_fused: SwiGLU needs the up matrix");
    VKML_CHECK_ARG(!p->quantize_out || (out_values && out_scales), "gemv_fused: quantize_out needs its buffers");
    GemvArgs g{p->norm ? nullptr : static_cast<const uint4*>(a), a_scales, b_values, b_scales, b2_values, b2_scales, out, residual,
               p->n, p->k, p->norm ? static_cast<const float*>(a) : nullptr, p->norm == 1 ? norm_weight : nullptr, p->eps,
               static_cast<uint8_t*>(out_values), out_scales};
    const char* label = "gemv_fused";
    switch (p->epilogue) {
        case 0: return p->norm == 1 ? dispatch_format<kStore, 1>(p->b_type, p->scale_type, g, label)
                       : p->norm == 2 ? dispatch_format<kStore, 2>(p->b_type, p->scale_type, g, label)
                                      : dispatch_format<kStore>(p->b_type, p->scale_type, g, label);
        case 1: return dispatch_format<kAdd>(p->b_type, p->scale_type, g, label);
        default:
            if (p->norm) {
                return p->quantize_out ? dispatch_format<kSwiglu, true, true>(p->b_type, p->scale_type, g, label)
                                       : dispatch_format<kSwiglu, true, false>(p->b_type, p->scale_type, g, label);
            }
            return p->quantize_out ? dispatch_format<kSwiglu, false, true>(p->b_type, p->scale_type, g, label)
                                   : dispatch_format<kSwiglu>(p->b_type, p->scale_type, g, label);
    }
}

int vkml_gemv_rope(const vkml_gemv_rope_params* p, const float* x, const float* norm_weight, const void* b_values,
                   const void* b_scales, float* qkv, const float* rope_table, const vkml_decode_state* state, void* k_cache,
                   void* v_cache) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(p, "gemv_rope: null params");
    const vkml_gemv_dot_params dp{1, p->n, p->k, p->b_type, p->scale_type};
    if (int r = check_dot_params(&dp, "gemv_rope")) return r;
    VKML_CHECK_ARG(p->k <= 4096, "gemv_rope: the RMSNorm + Q8_0 prologue takes k up to 4096");
    VKML_CHECK_ARG(p->head_dim > 0 && p->head_dim % 2 == 0 && p->heads > 0 && p->kv_heads > 0 && p->capacity > 0,
                   "gemv_rope: heads, kv_heads, capacity and an even head_dim must be positive");
    VKML_CHECK_ARG(p->kv_type == VKML_F16 || p->kv_type == VKML_F32, "gemv_rope: caches must be f16 or f32");
    const uint64_t q_rows = static_cast<uint64_t>(p->heads) * p->head_dim, kv_rows = static_cast<uint64_t>(p->kv_heads) * p->head_dim;
    // Pairs of rows share a workgroup when the first row is even.
    VKML_CHECK_ARG(p->row0 % 2 == 0 && p->n % 2 == 0 && p->row0 + static_cast<uint64_t>(p->n) <= q_rows + 2 * kv_rows,
                   "gemv_rope: rows " + std::to_string(p->row0) + " .. " + std::to_string(p->row0 + p->n) + " must be even-aligned rows of the " +
                       std::to_string(q_rows + 2 * kv_rows) + " of [q | k | v]");
    if (p->n == 0) return VKML_OK;
    VKML_CHECK_ARG(x && norm_weight && b_values && b_scales && qkv && state && k_cache && v_cache && (rope_table || !p->rotate),
                   "gemv_rope: null buffer");
    GemvArgs g{nullptr, nullptr, b_values, b_scales, nullptr, nullptr, qkv + p->row0, nullptr, p->n, p->k, x, norm_weight, p->eps,
               nullptr, nullptr};
    // (a non-null table selects the epilogue; with rotate = 0 it is not read)
    g.table = rope_table ? rope_table : x;
    g.state = state;
    g.k_cache = k_cache;
    g.v_cache = v_cache;
    g.row0 = p->row0;
    g.q_rows = static_cast<uint32_t>(q_rows);
    g.kv_rows = static_cast<uint32_t>(kv_rows);
    g.hd = p->head_dim;
    g.capacity = p->capacity;
    g.kv_f16 = p->kv_type == VKML_F16;
    g.rotate = p->rotate;
    return dispatch_format<kStore, 1>(p->b_type, p->scale_type, g, "gemv_rope");
}

int vkml_gemv(const vkml_gemv_params* p, const float* a, const void* b, float* out, const void* b_scales) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(p, "gemv: null params");
    VKML_CHECK_ARG(p->m >= 1 && p->m <= 8, "gemv: m must be 1 to 8, got " + std::to_string(p->m));
    VKML_CHECK_ARG(p->b_type <= VKML_Q4_K, "gemv: unknown weight type " + std::to_string(p->b_type));
    const uint32_t batches = std::max(p->batches, 1u), group = std::max(p->b_group, 1u);
    VKML_CHECK_ARG(batches <= 65535, "gemv: too many batches");
    if (p->b_type >= VKML_Q8_0) {
        const uint32_t unit = p->b_type == VKML_Q4_K ? 256 : 32;
        VKML_CHECK_ARG(p->k % unit == 0, "gemv: k = " + std::to_string(p->k) + " is not whole blocks of " + std::to_string(unit));
        VKML_CHECK_ARG(b_scales, "gemv: quantized weights need scales");
        VKML_CHECK_ARG(batches == 1, "gemv: batches need a float b");
    }
    if (p->n == 0) return VKML_OK;
    VKML_CHECK_ARG(a && b && out, "gemv: null buffer");
    const dim3 grid((p->n + 7) / 8, batches);
    vkml::abi::ProfileScope prof("gemv");
    hipStream_t s = vkml::abi::stream();
    const uint64_t bst = p->b_stride;
#define VKML_GEMV_LAUNCH(T) \
    hipLaunchKernelGGL(k_gemv_float<T>, grid, dim3(256), 0, s, a, p->m, b, b_scales, p->scale_type, out, p->n, p->k, group, bst)
    switch (p->b_type) {
        case VKML_F32: VKML_GEMV_LAUNCH(VKML_F32); break;
        case VKML_F16: VKML_GEMV_LAUNCH(VKML_F16); break;
        case VKML_BF16: VKML_GEMV_LAUNCH(VKML_BF16); break;
        case VKML_Q8_0: VKML_GEMV_LAUNCH(VKML_Q8_0); break;
        case VKML_Q4_0: VKML_GEMV_LAUNCH(VKML_Q4_0); break;
        case VKML_Q4_1: VKML_GEMV_LAUNCH(VKML_Q4_1); break;
        default: VKML_GEMV_LAUNCH(VKML_Q4_K); break;
    }
#undef VKML_GEMV_LAUNCH
    return vkml::abi::check_launch("gemv");
}

}  // extern "C"
