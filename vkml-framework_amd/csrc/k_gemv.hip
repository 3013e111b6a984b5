// k_gemv.hip -- quantized matrix-vector products for decoding (the
// reference's shaders/gemv_dot.comp and gemv.comp), written for gfx950.
//
// Bit-exact by construction. The reference sums each output over 32
// accumulators: accumulator l takes the terms of half-blocks (16 values) l,
// l + 32, l + 64, ... in that order, each term an exact int8 dot product
// scaled in f32 (gemv_dot.comp:349-363), and the 32 are added in a halving
// tree (:370-375). Every f32 operation here happens in that order, so the
// outputs are the reference's bits, and the Q8_0 codes the next layer
// quantizes from them are too.
//
// The 32 accumulators of a row live in 8 lanes, 4 each: lane j takes the
// 64-value tasks c = j, j + 8, ..., whose half-blocks 4c .. 4c + 3 are
// exactly accumulators 4j .. 4j + 3. So each lane still streams its weights
// with 128-bit loads (32 B of 4-bit codes, or 64 B of q8_0, plus the task's
// scales or q4_K's 16-byte header), a wave64 covers 8 rows, and the tree's
// strides 16, 8 and 4 are lane exchanges within the 8-lane group, 2 and 1
// additions within a lane. The activation vector is staged once per
// workgroup in LDS with each half-block's code sum. No MFMA: these are
// matrix-vector products, bound by HBM.
#include <algorithm>

#include "device.hpp"
#include "internal.hpp"

using namespace vkml::dev;

namespace {

constexpr uint32_t kMaxK = 32768;  // LDS staging: K + K / 16 * 4 + K / 32 * 4 bytes

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
};

// One row's weights for one 64-value task.
struct Wt {
    uint4 q[4];
    uint4 s;
};

template <int FMT, bool F16S>
__device__ __forceinline__ void load_task(const void* bv, const void* bs, uint32_t K, uint32_t row, uint32_t t, Wt& w) {
    const uint64_t r = row;
    if constexpr (FMT == VKML_Q8_0) {
        const uint4* q = static_cast<const uint4*>(bv) + r * (K / 16) + 4 * t;
        w.q[0] = q[0]; w.q[1] = q[1]; w.q[2] = q[2]; w.q[3] = q[3];
        if constexpr (F16S) w.s.x = static_cast<const uint32_t*>(bs)[r * (K / 64) + t];
        else { const uint2 s = static_cast<const uint2*>(bs)[r * (K / 64) + t]; w.s.x = s.x; w.s.y = s.y; }
    } else {
        const uint4* q = static_cast<const uint4*>(bv) + r * (K / 32) + 2 * t;
        w.q[0] = q[0]; w.q[1] = q[1];
        if constexpr (FMT == VKML_Q4_K) {
            w.s = static_cast<const uint4*>(bs)[r * (K / 256) + t / 4];
        } else if constexpr (FMT == VKML_Q4_1) {
            if constexpr (F16S) { const uint2 s = static_cast<const uint2*>(bs)[r * (K / 64) + t]; w.s.x = s.x; w.s.y = s.y; }
            else w.s = static_cast<const uint4*>(bs)[r * (K / 64) + t];
        } else {
            if constexpr (F16S) w.s.x = static_cast<const uint32_t*>(bs)[r * (K / 64) + t];
            else { const uint2 s = static_cast<const uint2*>(bs)[r * (K / 64) + t]; w.s.x = s.x; w.s.y = s.y; }
        }
    }
}

constexpr uint32_t kLow = 0x0F0F0F0Fu;

// The exact dot product of one half-block: 16 weight codes as bytes (four
// words) with 16 activation codes (gemv_dot.comp:352-353).
__device__ __forceinline__ int half_dot(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3, uint4 a) {
    return dot4(w3, a.w, dot4(w2, a.z, dot4(w1, a.y, dot4(w0, a.x, 0))));
}

// Adds the task's four half-block terms to acc[0..3] with the reference's
// expressions (gemv_dot.comp:354-362): q8_0/q4_0 float(d) * (scale * sa);
// q4_1 (and q4_K, whose sub-blocks are q4_1's) sa * (float(d) * scale +
// float(sum) * offset). S holds each half-block's activation code sum, sa
// the two blocks' activation scales.
template <int FMT, bool F16S>
__device__ __forceinline__ void task_terms(const Wt& w, uint32_t t, const uint4 (&a)[4], float4 S, float2 sa, float (&acc)[4]) {
#pragma clang fp contract(off)
    int d[4];
    float s0, s1, o0 = 0.0f, o1 = 0.0f;
    if constexpr (FMT == VKML_Q8_0) {
#pragma unroll
        for (int h = 0; h < 4; ++h) d[h] = half_dot(w.q[h].x, w.q[h].y, w.q[h].z, w.q[h].w, a[h]);
        if constexpr (F16S) { s0 = f16_bits_to_float(w.s.x & 0xFFFFu); s1 = f16_bits_to_float(w.s.x >> 16); }
        else { s0 = __uint_as_float(w.s.x); s1 = __uint_as_float(w.s.y); }
    } else if constexpr (FMT == VKML_Q4_K) {
        // Bytes 32c .. 32c + 31 of the super-block's codes: low nibbles are
        // sub-block 2c, high nibbles sub-block 2c + 1, each in value order.
        const uint4 q0 = w.q[0], q1 = w.q[1];
        d[0] = half_dot(q0.x & kLow, q0.y & kLow, q0.z & kLow, q0.w & kLow, a[0]);
        d[1] = half_dot(q1.x & kLow, q1.y & kLow, q1.z & kLow, q1.w & kLow, a[1]);
        d[2] = half_dot((q0.x >> 4) & kLow, (q0.y >> 4) & kLow, (q0.z >> 4) & kLow, (q0.w >> 4) & kLow, a[2]);
        d[3] = half_dot((q1.x >> 4) & kLow, (q1.y >> 4) & kLow, (q1.z >> 4) & kLow, (q1.w >> 4) & kLow, a[3]);
        q4k_scales(w.s, t & 3u, s0, o0, s1, o1);
    } else {
        // QuantizedMatrix q4 words: byte j holds value j (low) and j + 4 (high).
        const uint4 q0 = w.q[0], q1 = w.q[1];
        d[0] = half_dot(q0.x & kLow, (q0.x >> 4) & kLow, q0.y & kLow, (q0.y >> 4) & kLow, a[0]);
        d[1] = half_dot(q0.z & kLow, (q0.z >> 4) & kLow, q0.w & kLow, (q0.w >> 4) & kLow, a[1]);
        d[2] = half_dot(q1.x & kLow, (q1.x >> 4) & kLow, q1.y & kLow, (q1.y >> 4) & kLow, a[2]);
        d[3] = half_dot(q1.z & kLow, (q1.z >> 4) & kLow, q1.w & kLow, (q1.w >> 4) & kLow, a[3]);
        if constexpr (FMT == VKML_Q4_1) {
            if constexpr (F16S) {
                s0 = f16_bits_to_float(w.s.x & 0xFFFFu); o0 = f16_bits_to_float(w.s.x >> 16);
                s1 = f16_bits_to_float(w.s.y & 0xFFFFu); o1 = f16_bits_to_float(w.s.y >> 16);
            } else {
                s0 = __uint_as_float(w.s.x); o0 = __uint_as_float(w.s.y); s1 = __uint_as_float(w.s.z); o1 = __uint_as_float(w.s.w);
            }
        } else {
            if constexpr (F16S) { s0 = f16_bits_to_float(w.s.x & 0xFFFFu); s1 = f16_bits_to_float(w.s.x >> 16); }
            else { s0 = __uint_as_float(w.s.x); s1 = __uint_as_float(w.s.y); }
            // q4_0 codes are q + 8: the reference's signed bytes q4_bytes give
            // the same exact sum, d - 8 * sum(a).
            d[0] -= 8 * static_cast<int>(S.x); d[1] -= 8 * static_cast<int>(S.y);
            d[2] -= 8 * static_cast<int>(S.z); d[3] -= 8 * static_cast<int>(S.w);
        }
    }
    const float sum[4] = {S.x, S.y, S.z, S.w};
#pragma unroll
    for (int h = 0; h < 4; ++h) {
        const float scale = h < 2 ? s0 : s1, a_scale = h < 2 ? sa.x : sa.y;
        if constexpr (FMT == VKML_Q4_1 || FMT == VKML_Q4_K) {
            const float offset = h < 2 ? o0 : o1;
            acc[h] += a_scale * (static_cast<float>(d[h]) * scale + sum[h] * offset);
        } else {
            acc[h] += static_cast<float>(d[h]) * (scale * a_scale);
        }
    }
}

// The halving tree over the 32 accumulators of the 8-lane group; the row's
// sum ends in lane 0 of the group (gemv_dot.comp:370-375).
__device__ __forceinline__ float tree32(float (&acc)[4]) {
#pragma clang fp contract(off)
#pragma unroll
    for (int off = 4; off >= 1; off >>= 1)
#pragma unroll
        for (int h = 0; h < 4; ++h) acc[h] += __shfl_xor(acc[h], off, kWave);
    acc[0] += acc[2];
    acc[1] += acc[3];
    return acc[0] + acc[1];
}

enum { kStore = 0, kAdd = 1, kSwiglu = 2 };

template <int FMT, bool F16S, int EPI>
__global__ void __launch_bounds__(256) k_gemv_dot(GemvArgs g) {
#pragma clang fp contract(off)
    extern __shared__ uint4 smem[];
    const uint32_t K = g.k;
    uint4* s_codes = smem;                                   // K / 16 half-blocks of codes
    float* s_sum = reinterpret_cast<float*>(smem + K / 16);  // each half-block's code sum
    float* s_sa = s_sum + K / 16;                            // each block's activation scale
    for (uint32_t h = threadIdx.x; h < K / 16; h += blockDim.x) {
        const uint4 c = g.a_values[h];
        s_codes[h] = c;
        s_sum[h] = static_cast<float>(byte_sum(c));
        if (h % 2 == 0) s_sa[h / 2] = g.a_scales[h / 2];
    }
    __syncthreads();
    const uint32_t lane8 = threadIdx.x % 8;
    const uint32_t row = blockIdx.x * (blockDim.x / 8) + threadIdx.x / 8;
    const uint32_t r = min(row, g.n - 1);
    constexpr int NM = EPI == kSwiglu ? 2 : 1;
    constexpr int U = (FMT == VKML_Q8_0 || NM == 2) ? 2 : 4;  // tasks in flight per lane
    float acc[NM][4];
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int h = 0; h < 4; ++h) acc[m][h] = 0.0f;
    const uint32_t tasks = K / 64;
    const float4* sum4 = reinterpret_cast<const float4*>(s_sum);
    const float2* sa2 = reinterpret_cast<const float2*>(s_sa);
    for (uint32_t t0 = lane8; t0 < tasks; t0 += 8 * U) {
        Wt w[U][NM];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t t = t0 + 8 * u;
            if (t < tasks) {
                load_task<FMT, F16S>(g.b_values, g.b_scales, K, r, t, w[u][0]);
                if constexpr (NM == 2) load_task<FMT, F16S>(g.b2_values, g.b2_scales, K, r, t, w[u][NM - 1]);
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t t = t0 + 8 * u;
            if (t < tasks) {
                const uint4 a[4] = {s_codes[4 * t], s_codes[4 * t + 1], s_codes[4 * t + 2], s_codes[4 * t + 3]};
                const float4 S = sum4[t];
                const float2 sa = sa2[t];
#pragma unroll
                for (int m = 0; m < NM; ++m) task_terms<FMT, F16S>(w[u][m], t, a, S, sa, acc[m]);
            }
        }
    }
    float y[NM];
#pragma unroll
    for (int m = 0; m < NM; ++m) y[m] = tree32(acc[m]);
    if (lane8 == 0 && row < g.n) {
        if constexpr (EPI == kStore) {
            g.out[row] = y[0];
        } else if constexpr (EPI == kAdd) {
            g.out[row] = g.residual[row] + y[0];  // add(x, attn_out), llama.cpp:374,386
        } else {
            // silu(gate) * up (unary.comp:21-24, then binary.comp's mul)
            const float gate = y[0], up = y[NM - 1];
            g.out[row] = gate / (1.0f + vk_expf(-gate)) * up;
        }
    }
}

template <int FMT, bool F16S, int EPI>
int dispatch(const GemvArgs& g, const char* label) {
    // Rows per workgroup (8 per wave): enough workgroups to cover the CUs twice.
    const uint32_t cus = std::max<uint32_t>(vkml::abi::compute_units(), 1);
    uint32_t threads = 256;
    while (threads > 64 && (g.n + threads / 8 - 1) / (threads / 8) < 2 * cus) threads /= 2;
    const dim3 grid((g.n + threads / 8 - 1) / (threads / 8));
    const size_t lds = g.k + g.k / 16 * 4 + g.k / 32 * 4;
    vkml::abi::ProfileScope prof(label);
    hipLaunchKernelGGL((k_gemv_dot<FMT, F16S, EPI>), grid, dim3(threads), lds, vkml::abi::stream(), g);
    return vkml::abi::check_launch(label);
}

template <int EPI>
int dispatch_format(uint32_t b_type, uint32_t scale_type, const GemvArgs& g, const char* label) {
    const bool f16 = scale_type == VKML_F16;
    switch (b_type) {
        case VKML_Q8_0: return f16 ? dispatch<VKML_Q8_0, true, EPI>(g, label) : dispatch<VKML_Q8_0, false, EPI>(g, label);
        case VKML_Q4_0: return f16 ? dispatch<VKML_Q4_0, true, EPI>(g, label) : dispatch<VKML_Q4_0, false, EPI>(g, label);
        case VKML_Q4_1: return f16 ? dispatch<VKML_Q4_1, true, EPI>(g, label) : dispatch<VKML_Q4_1, false, EPI>(g, label);
        case VKML_Q4_K: return dispatch<VKML_Q4_K, true, EPI>(g, label);
        default: return vkml::abi::fail(VKML_ERROR_UNSUPPORTED, std::string(label) + ": no int8 kernel for weight type " + std::to_string(b_type));
    }
}

int check_dot_params(const vkml_gemv_dot_params* p, const char* what) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(p, std::string(what) + ": null params");
    VKML_CHECK_ARG(p->b_type == VKML_Q8_0 || p->b_type == VKML_Q4_0 || p->b_type == VKML_Q4_1 || p->b_type == VKML_Q4_K,
                   std::string(what) + ": weights must be q8_0, q4_0, q4_1 or q4_K, got type " + std::to_string(p->b_type));
    VKML_CHECK_ARG(p->b_type == VKML_Q4_K || p->scale_type == VKML_F16 || p->scale_type == VKML_F32,
                   std::string(what) + ": scales must be f16 or f32");
    const uint32_t unit = p->b_type == VKML_Q4_K ? 256 : 64;
    VKML_CHECK_ARG(p->k > 0 && p->k % unit == 0 && p->k <= kMaxK,
                   std::string(what) + ": k = " + std::to_string(p->k) + " must be a positive multiple of " +
                       std::to_string(unit) + " up to " + std::to_string(kMaxK));
    return VKML_OK;
}

// ---------------------------------------------------------------- float path

// gemv.comp's order: 32 lanes per output, lane l taking the 4-element
// groups l, l + 32, ... of its row (dot(a4, w) summed left to right), then
// the halving tree over the 32 lanes (gemv.comp:117-212). Two rows a wave.
template <int BT>
__global__ void __launch_bounds__(256) k_gemv_float(const float* a, uint32_t m, const void* b, const void* bs, uint32_t st,
                                                    float* out, uint32_t n, uint32_t k) {
#pragma clang fp contract(off)
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
        float v = acc[q];
#pragma unroll
        for (int off = 16; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
        if (lane == 0 && row < n) out[static_cast<uint64_t>(q) * n + row] = v;
    }
}

}  // namespace

extern "C" {

int vkml_gemv_dot(const vkml_gemv_dot_params* p, const void* a_values, const void* b_values, float* out,
                  const void* b_scales, const float* a_scales) {
    if (int r = check_dot_params(p, "gemv_dot")) return r;
    VKML_CHECK_ARG(p->m >= 1 && p->m <= 8, "gemv_dot: m must be 1 to 8, got " + std::to_string(p->m));
    if (p->n == 0) return VKML_OK;
    VKML_CHECK_ARG(a_values && b_values && out && b_scales && a_scales, "gemv_dot: null buffer");
    for (uint32_t r = 0; r < p->m; ++r) {
        GemvArgs g{reinterpret_cast<const uint4*>(static_cast<const uint8_t*>(a_values) + static_cast<uint64_t>(r) * p->k),
                   a_scales + static_cast<uint64_t>(r) * (p->k / 32), b_values, b_scales, nullptr, nullptr,
                   out + static_cast<uint64_t>(r) * p->n, nullptr, p->n, p->k};
        if (int e = dispatch_format<kStore>(p->b_type, p->scale_type, g, "gemv_dot")) return e;
    }
    return VKML_OK;
}

int vkml_gemv_dot_add(const vkml_gemv_dot_params* p, const void* a_values, const void* b_values, float* out,
                      const void* b_scales, const float* a_scales, const float* residual) {
    if (int r = check_dot_params(p, "gemv_dot_add")) return r;
    VKML_CHECK_ARG(p->m == 1, "gemv_dot_add: m must be 1");
    if (p->n == 0) return VKML_OK;
    VKML_CHECK_ARG(a_values && b_values && out && b_scales && a_scales && residual, "gemv_dot_add: null buffer");
    GemvArgs g{static_cast<const uint4*>(a_values), a_scales, b_values, b_scales, nullptr, nullptr, out, residual, p->n, p->k};
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

int vkml_gemv(const vkml_gemv_params* p, const float* a, const void* b, float* out, const void* b_scales) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(p, "gemv: null params");
    VKML_CHECK_ARG(p->m >= 1 && p->m <= 8, "gemv: m must be 1 to 8, got " + std::to_string(p->m));
    VKML_CHECK_ARG(p->b_type <= VKML_Q4_K, "gemv: unknown weight type " + std::to_string(p->b_type));
    if (p->b_type >= VKML_Q8_0) {
        const uint32_t unit = p->b_type == VKML_Q4_K ? 256 : 32;
        VKML_CHECK_ARG(p->k % unit == 0, "gemv: k = " + std::to_string(p->k) + " is not whole blocks of " + std::to_string(unit));
        VKML_CHECK_ARG(b_scales, "gemv: quantized weights need scales");
    }
    if (p->n == 0) return VKML_OK;
    VKML_CHECK_ARG(a && b && out, "gemv: null buffer");
    const dim3 grid((p->n + 7) / 8);
    vkml::abi::ProfileScope prof("gemv");
    hipStream_t s = vkml::abi::stream();
    switch (p->b_type) {
        case VKML_F32: hipLaunchKernelGGL(k_gemv_float<VKML_F32>, grid, dim3(256), 0, s, a, p->m, b, b_scales, p->scale_type, out, p->n, p->k); break;
        case VKML_F16: hipLaunchKernelGGL(k_gemv_float<VKML_F16>, grid, dim3(256), 0, s, a, p->m, b, b_scales, p->scale_type, out, p->n, p->k); break;
        case VKML_BF16: hipLaunchKernelGGL(k_gemv_float<VKML_BF16>, grid, dim3(256), 0, s, a, p->m, b, b_scales, p->scale_type, out, p->n, p->k); break;
        case VKML_Q8_0: hipLaunchKernelGGL(k_gemv_float<VKML_Q8_0>, grid, dim3(256), 0, s, a, p->m, b, b_scales, p->scale_type, out, p->n, p->k); break;
        case VKML_Q4_0: hipLaunchKernelGGL(k_gemv_float<VKML_Q4_0>, grid, dim3(256), 0, s, a, p->m, b, b_scales, p->scale_type, out, p->n, p->k); break;
        case VKML_Q4_1: hipLaunchKernelGGL(k_gemv_float<VKML_Q4_1>, grid, dim3(256), 0, s, a, p->m, b, b_scales, p->scale_type, out, p->n, p->k); break;
        default: hipLaunchKernelGGL(k_gemv_float<VKML_Q4_K>, grid, dim3(256), 0, s, a, p->m, b, b_scales, p->scale_type, out, p->n, p->k); break;
    }
    return vkml::abi::check_launch("gemv");
}

}  // extern "C"
