// k_gemv.hip -- quantized matrix-vector products for decoding (the
// reference's shaders/gemv_dot.comp and gemv.comp), written for gfx950.
//
// int8 path (vkml_gemv_dot*): each workgroup stages the Q8_0 activation
// vector once in LDS (codes plus, per 32-value block, its f32 scale and the
// sum of its codes), then each wave64 computes RPW rows. A row is cut into
// 64-value tasks; lane l takes tasks l, l + 64, ...: per task it loads the
// weights with 128-bit loads (64 B of q8_0 codes, or 32 B of 4-bit codes)
// plus the task's scales (an f16 pair, (scale, offset) pairs, or q4_K's
// 16-byte super-block header), multiplies with v_dot4_i32_i8 against the
// staged activations, and scales each 32-value block's exact integer sum in
// f32 as the reference's matmul_dot.comp does (acc += sa * (D * s + S * o)
// for q4_1/q4_K, D * (s * sa) for q8_0). A wave reduction then sums the
// lanes, and the epilogue stores, adds the residual, or applies SwiGLU.
// There is no MFMA here: these are matrix-vector products, bound by HBM.
#include <algorithm>

#include "device.hpp"
#include "internal.hpp"

using namespace vkml::dev;

namespace {

constexpr uint32_t kMaxK = 32768;  // LDS staging: K + K / 4 bytes
constexpr int kThreads = 256;

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

// Low (shift 0) or high (shift 4) nibbles of a 32-value block of
// QuantizedMatrix q4 words (byte j: value j, high nibble value j + 4) dotted
// with the block's 32 activation codes a0, a1.
__device__ __forceinline__ int q4_block_dot(uint4 q, uint4 a0, uint4 a1) {
    int d = dot4(q.x & kLow, a0.x, 0);
    d = dot4((q.x >> 4) & kLow, a0.y, d);
    d = dot4(q.y & kLow, a0.z, d);
    d = dot4((q.y >> 4) & kLow, a0.w, d);
    d = dot4(q.z & kLow, a1.x, d);
    d = dot4((q.z >> 4) & kLow, a1.y, d);
    d = dot4(q.w & kLow, a1.z, d);
    d = dot4((q.w >> 4) & kLow, a1.w, d);
    return d;
}

template <int FMT, bool F16S>
__device__ __forceinline__ float task_dot(const Wt& w, uint32_t t, const uint4 (&a)[4], float4 bi) {
    // bi: (sa0, S0, sa1, S1) for the task's two activation blocks.
    if constexpr (FMT == VKML_Q8_0) {
        int d0 = dot4(w.q[0].x, a[0].x, 0); d0 = dot4(w.q[0].y, a[0].y, d0); d0 = dot4(w.q[0].z, a[0].z, d0); d0 = dot4(w.q[0].w, a[0].w, d0);
        d0 = dot4(w.q[1].x, a[1].x, d0); d0 = dot4(w.q[1].y, a[1].y, d0); d0 = dot4(w.q[1].z, a[1].z, d0); d0 = dot4(w.q[1].w, a[1].w, d0);
        int d1 = dot4(w.q[2].x, a[2].x, 0); d1 = dot4(w.q[2].y, a[2].y, d1); d1 = dot4(w.q[2].z, a[2].z, d1); d1 = dot4(w.q[2].w, a[2].w, d1);
        d1 = dot4(w.q[3].x, a[3].x, d1); d1 = dot4(w.q[3].y, a[3].y, d1); d1 = dot4(w.q[3].z, a[3].z, d1); d1 = dot4(w.q[3].w, a[3].w, d1);
        float s0, s1;
        if constexpr (F16S) { s0 = f16_bits_to_float(w.s.x & 0xFFFFu); s1 = f16_bits_to_float(w.s.x >> 16); }
        else { s0 = __uint_as_float(w.s.x); s1 = __uint_as_float(w.s.y); }
        return static_cast<float>(d0) * (s0 * bi.x) + static_cast<float>(d1) * (s1 * bi.z);
    } else if constexpr (FMT == VKML_Q4_K) {
        // Bytes 32c..32c+31 of the super-block's codes: low nibbles are
        // sub-block 2c, high nibbles sub-block 2c + 1, each in value order.
        int d0 = dot4(w.q[0].x & kLow, a[0].x, 0); d0 = dot4(w.q[0].y & kLow, a[0].y, d0);
        d0 = dot4(w.q[0].z & kLow, a[0].z, d0); d0 = dot4(w.q[0].w & kLow, a[0].w, d0);
        d0 = dot4(w.q[1].x & kLow, a[1].x, d0); d0 = dot4(w.q[1].y & kLow, a[1].y, d0);
        d0 = dot4(w.q[1].z & kLow, a[1].z, d0); d0 = dot4(w.q[1].w & kLow, a[1].w, d0);
        int d1 = dot4((w.q[0].x >> 4) & kLow, a[2].x, 0); d1 = dot4((w.q[0].y >> 4) & kLow, a[2].y, d1);
        d1 = dot4((w.q[0].z >> 4) & kLow, a[2].z, d1); d1 = dot4((w.q[0].w >> 4) & kLow, a[2].w, d1);
        d1 = dot4((w.q[1].x >> 4) & kLow, a[3].x, d1); d1 = dot4((w.q[1].y >> 4) & kLow, a[3].y, d1);
        d1 = dot4((w.q[1].z >> 4) & kLow, a[3].z, d1); d1 = dot4((w.q[1].w >> 4) & kLow, a[3].w, d1);
        float s0, o0, s1, o1;
        q4k_scales(w.s, t & 3u, s0, o0, s1, o1);
        return bi.x * (static_cast<float>(d0) * s0 + bi.y * o0) + bi.z * (static_cast<float>(d1) * s1 + bi.w * o1);
    } else {
        const int d0 = q4_block_dot(w.q[0], a[0], a[1]);
        const int d1 = q4_block_dot(w.q[1], a[2], a[3]);
        if constexpr (FMT == VKML_Q4_1) {
            float s0, o0, s1, o1;
            if constexpr (F16S) {
                s0 = f16_bits_to_float(w.s.x & 0xFFFFu); o0 = f16_bits_to_float(w.s.x >> 16);
                s1 = f16_bits_to_float(w.s.y & 0xFFFFu); o1 = f16_bits_to_float(w.s.y >> 16);
            } else {
                s0 = __uint_as_float(w.s.x); o0 = __uint_as_float(w.s.y); s1 = __uint_as_float(w.s.z); o1 = __uint_as_float(w.s.w);
            }
            return bi.x * (static_cast<float>(d0) * s0 + bi.y * o0) + bi.z * (static_cast<float>(d1) * s1 + bi.w * o1);
        } else {  // q4_0: codes are q + 8
            float s0, s1;
            if constexpr (F16S) { s0 = f16_bits_to_float(w.s.x & 0xFFFFu); s1 = f16_bits_to_float(w.s.x >> 16); }
            else { s0 = __uint_as_float(w.s.x); s1 = __uint_as_float(w.s.y); }
            const int e0 = d0 - 8 * static_cast<int>(bi.y), e1 = d1 - 8 * static_cast<int>(bi.w);
            return static_cast<float>(e0) * (s0 * bi.x) + static_cast<float>(e1) * (s1 * bi.z);
        }
    }
}

enum { kStore = 0, kAdd = 1, kSwiglu = 2 };

template <int FMT, bool F16S, int RPW, int EPI>
__global__ void __launch_bounds__(kThreads) k_gemv_dot(GemvArgs g) {
    extern __shared__ uint4 smem[];
    const uint32_t K = g.k;
    uint4* s_codes = smem;
    float2* s_info = reinterpret_cast<float2*>(smem + K / 16);
    for (uint32_t b = threadIdx.x; b < K / 32; b += kThreads) {
        const uint4 c0 = g.a_values[2 * b], c1 = g.a_values[2 * b + 1];
        s_codes[2 * b] = c0;
        s_codes[2 * b + 1] = c1;
        s_info[b] = make_float2(g.a_scales[b], static_cast<float>(byte_sum(c0) + byte_sum(c1)));
    }
    __syncthreads();
    const uint32_t wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const uint32_t row0 = (blockIdx.x * (kThreads / kWave) + wave) * RPW;
    if (row0 >= g.n) return;
    constexpr int NM = EPI == kSwiglu ? 2 : 1;
    float acc[NM][RPW];
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int r = 0; r < RPW; ++r) acc[m][r] = 0.0f;
    const uint32_t tasks = K / 64;
    const float4* info4 = reinterpret_cast<const float4*>(s_info);
    for (uint32_t t = lane; t < tasks; t += kWave) {
        Wt w[NM][RPW];
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const uint32_t row = min(row0 + r, g.n - 1);
            load_task<FMT, F16S>(g.b_values, g.b_scales, K, row, t, w[0][r]);
            if constexpr (EPI == kSwiglu) load_task<FMT, F16S>(g.b2_values, g.b2_scales, K, row, t, w[NM - 1][r]);
        }
        const uint4 a[4] = {s_codes[4 * t], s_codes[4 * t + 1], s_codes[4 * t + 2], s_codes[4 * t + 3]};
        const float4 bi = info4[t];
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int r = 0; r < RPW; ++r) acc[m][r] += task_dot<FMT, F16S>(w[m][r], t, a, bi);
    }
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int r = 0; r < RPW; ++r) acc[m][r] = wave_sum(acc[m][r]);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const uint32_t row = row0 + r;
            if (row >= g.n) break;
            if constexpr (EPI == kStore) {
                g.out[row] = acc[0][r];
            } else if constexpr (EPI == kAdd) {
                g.out[row] = g.residual[row] + acc[0][r];
            } else {
                const float gate = acc[0][r], up = acc[NM - 1][r];
                g.out[row] = gate / (1.0f + expf(-gate)) * up;
            }
        }
    }
}

template <int FMT, bool F16S, int EPI>
int dispatch_rpw(const GemvArgs& g, const char* label) {
    // Rows per wave: enough workgroups to cover the CUs a few times over.
    const uint32_t cus = std::max<uint32_t>(vkml::abi::compute_units(), 1);
    int rpw = 4;
    while (rpw > 1 && (g.n + 4u * rpw - 1) / (4u * rpw) < 2 * cus) rpw /= 2;
    const uint32_t rows_per_block = 4u * rpw;
    const dim3 grid((g.n + rows_per_block - 1) / rows_per_block);
    const size_t lds = g.k + g.k / 32 * 8;
    vkml::abi::ProfileScope prof(label);
    switch (rpw) {
        case 4: hipLaunchKernelGGL((k_gemv_dot<FMT, F16S, 4, EPI>), grid, dim3(kThreads), lds, vkml::abi::stream(), g); break;
        case 2: hipLaunchKernelGGL((k_gemv_dot<FMT, F16S, 2, EPI>), grid, dim3(kThreads), lds, vkml::abi::stream(), g); break;
        default: hipLaunchKernelGGL((k_gemv_dot<FMT, F16S, 1, EPI>), grid, dim3(kThreads), lds, vkml::abi::stream(), g); break;
    }
    return vkml::abi::check_launch(label);
}

template <int EPI>
int dispatch_format(uint32_t b_type, uint32_t scale_type, const GemvArgs& g, const char* label) {
    const bool f16 = scale_type == VKML_F16;
    switch (b_type) {
        case VKML_Q8_0: return f16 ? dispatch_rpw<VKML_Q8_0, true, EPI>(g, label) : dispatch_rpw<VKML_Q8_0, false, EPI>(g, label);
        case VKML_Q4_0: return f16 ? dispatch_rpw<VKML_Q4_0, true, EPI>(g, label) : dispatch_rpw<VKML_Q4_0, false, EPI>(g, label);
        case VKML_Q4_1: return f16 ? dispatch_rpw<VKML_Q4_1, true, EPI>(g, label) : dispatch_rpw<VKML_Q4_1, false, EPI>(g, label);
        case VKML_Q4_K: return dispatch_rpw<VKML_Q4_K, true, EPI>(g, label);
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

template <int BT>
__global__ void __launch_bounds__(256) k_gemv_float(const float* a, uint32_t m, const void* b, const void* bs,
                                                    uint32_t st, float* out, uint32_t n, uint32_t k) {
    const uint32_t wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const uint32_t row = blockIdx.x * 4 + wave;
    if (row >= n) return;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (uint32_t col = lane; col < k; col += kWave) {
        const float w = BT == VKML_F32 ? static_cast<const float*>(b)[static_cast<uint64_t>(row) * k + col]
                                       : weight_value(BT, st, b, bs, k, row, col);
#pragma unroll
        for (uint32_t r = 0; r < 8; ++r)
            if (r < m) acc[r] += a[static_cast<uint64_t>(r) * k + col] * w;
    }
#pragma unroll
    for (uint32_t r = 0; r < 8; ++r) {
        if (r >= m) break;
        const float s = wave_sum(acc[r]);
        if (lane == 0) out[static_cast<uint64_t>(r) * n + row] = s;
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
    const dim3 grid((p->n + 3) / 4);
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
