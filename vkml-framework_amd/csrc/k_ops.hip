// k_ops.hip -- the decode path's small kernels and the rest of the op set:
// quantize/dequantize, RMSNorm (+ fused activation quantize), RoPE (+ fused
// cast and KV append), cast, row copies, permute, elementwise, embeddings,
// argmax, softmax and a tiled f32 matmul, plus the decode-state helpers.
// Where the result is integer or bit-level (codes, scales, casts, copies,
// argmax) it is exactly the reference's; products and sums that the
// reference writes separately are rounded separately here (plain operators
// under contract(off) below: HIP's __fmul_rn/__fadd_rn are ordinary header
// functions whose products the backend would still fuse).
#include <algorithm>
#include <cmath>

#include "device.hpp"
#include "internal.hpp"

// Bit-exact results need every product and sum the reference writes apart to
// be rounded apart: no multiply-add fusion in this file.
#pragma clang fp contract(off)

using namespace vkml::dev;
using vkml::abi::ProfileScope;

namespace {

hipStream_t S() { return vkml::abi::stream(); }

uint32_t blocks_for(uint64_t n, uint32_t threads = 256, uint32_t cap = 65535) {
    return static_cast<uint32_t>(std::max<uint64_t>(1, std::min<uint64_t>((n + threads - 1) / threads, cap)));
}

__device__ __forceinline__ float load_src(const void* x, uint64_t e, uint32_t type) {
    if (type == VKML_F32) return static_cast<const float*>(x)[e];
    return half_to_float(static_cast<const uint16_t*>(x)[e], type);
}

// ---------------------------------------------------------------- quantize

// shaders/quantize.comp:153-247 for one block: codes into q, scale (and
// offset) as kept (rounded to f16 with f16 scales), their f16 bits in bits.
__device__ void quantize_block(const void* x, uint32_t src_type, uint32_t quant, bool f16, uint64_t b,
                               uint32_t* q, float& d_out, float& m_out, uint32_t& bits_d, uint32_t& bits_m) {
    const uint64_t base = b * 32;
    const auto kept = [&](float v, uint32_t& bits) -> float {
        if (!f16) {
            bits = 0;
            return v;
        }
        bits = f32_to_f16_bits(__float_as_uint(v));
        return f16_bits_to_float(bits);
    };
    bits_m = 0;
    if (quant == VKML_Q4_1) {
        float lo = load_src(x, base, src_type), hi = lo;
        for (int i = 1; i < 32; ++i) {
            const float v = load_src(x, base + i, src_type);
            lo = fminf(lo, v);
            hi = fmaxf(hi, v);
        }
        const float m = kept(lo, bits_m);
        const float d = kept((hi - lo) / 15.0f, bits_d);
        const float inv = d > 0.0f ? 1.0f / d : 0.0f;
        for (int w = 0; w < 4; ++w) {
            uint32_t word = 0;
            for (uint32_t j = 0; j < 8; ++j) {
                const float code = fminf(fmaxf(__builtin_rintf((load_src(x, base + 8 * w + j, src_type) - m) * inv), 0.0f), 15.0f);
                word |= static_cast<uint32_t>(code) << q4_shift(j);
            }
            q[w] = word;
        }
        d_out = d;
        m_out = m;
        return;
    }
    if (quant == VKML_Q4_0) {
        float m = 0.0f;
        for (int i = 0; i < 32; ++i) {
            const float v = load_src(x, base + i, src_type);
            if (fabsf(v) > fabsf(m)) m = v;
        }
        const float d = kept(m / -8.0f, bits_d);
        const float inv = d != 0.0f ? 1.0f / d : 0.0f;
        for (int w = 0; w < 4; ++w) {
            uint32_t word = 0;
            for (uint32_t j = 0; j < 8; ++j) {
                const int v = static_cast<int>(fminf(fmaxf(__builtin_rintf(load_src(x, base + 8 * w + j, src_type) * inv), -8.0f), 7.0f));
                word |= static_cast<uint32_t>(v + 8) << q4_shift(j);
            }
            q[w] = word;
        }
        d_out = d;
        m_out = 0.0f;
        return;
    }
    float absmax = 0.0f;
    for (int i = 0; i < 32; ++i) absmax = fmaxf(absmax, fabsf(load_src(x, base + i, src_type)));
    const float d = kept(absmax / 127.0f, bits_d);
    const float inv = d > 0.0f ? 1.0f / d : 0.0f;
    for (int w = 0; w < 8; ++w) {
        uint32_t word = 0;
        for (int j = 0; j < 4; ++j) word |= (static_cast<uint32_t>(quant_code(load_src(x, base + 4 * w + j, src_type), inv)) & 0xFFu) << (8 * j);
        q[w] = word;
    }
    d_out = d;
    m_out = 0.0f;
}

__global__ void k_quantize(vkml_quantize_params p, const void* x, uint32_t* values, void* scales) {
    const bool f16 = p.scale_type == VKML_F16;
    const uint32_t per_word = p.quant == VKML_Q8_0 ? 8 : 4;
    for (uint64_t b = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; b < p.blocks;
         b += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
        float d, m;
        uint32_t bd, bm;
        quantize_block(x, p.src_type, p.quant, f16, b, values + b * per_word, d, m, bd, bm);
        if (!f16) {
            float* s = static_cast<float*>(scales);
            if (p.quant == VKML_Q4_1) {
                s[2 * b] = d;
                s[2 * b + 1] = m;
            } else {
                s[b] = d;
            }
        } else {
            uint16_t* s = static_cast<uint16_t*>(scales);
            if (p.quant == VKML_Q4_1) {
                s[2 * b] = static_cast<uint16_t>(bd);
                s[2 * b + 1] = static_cast<uint16_t>(bm);
            } else {
                s[b] = static_cast<uint16_t>(bd);
            }
        }
    }
}

// Float4 i of a Q8_0 row with f32 scales, 8 lanes per block of 32 (every
// lane of the group takes part in the absmax, live or not): the block's
// scale absmax / 127, the four codes packed into word i.
__device__ __forceinline__ void store_q8_lane(float4 v, bool live, uint64_t i, uint32_t* values, float* scales) {
    const float absmax = group_max<8>(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    const float d = absmax / 127.0f;
    const float inv = d > 0.0f ? 1.0f / d : 0.0f;
    if (!live) return;
    values[i] = (static_cast<uint32_t>(quant_code(v.x, inv)) & 0xFFu) | ((static_cast<uint32_t>(quant_code(v.y, inv)) & 0xFFu) << 8) |
                ((static_cast<uint32_t>(quant_code(v.z, inv)) & 0xFFu) << 16) | (static_cast<uint32_t>(quant_code(v.w, inv)) << 24);
    if (i % 8 == 0) scales[i / 8] = d;
}

// Activations to Q8_0 with f32 scales.
__global__ void k_quantize_act(uint32_t blocks, const float4* x, uint32_t* values, float* scales) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;  // float4 index
    const bool live = i < static_cast<uint64_t>(blocks) * 8;
    store_q8_lane(live ? x[i] : make_float4(0, 0, 0, 0), live, i, values, scales);
}

// silu(gate) * up, then its Q8_0 form: the f32 operations of k_unary's silu
// and k_binary's mul, the codes and scales of k_quantize_act.
__device__ __forceinline__ float swiglu(float g, float u) { return g / (1.0f + vk_expf(-g)) * u; }

__global__ void k_swiglu_quantize(uint32_t blocks, const float4* gate, const float4* up, uint32_t* values, float* scales) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;  // float4 index
    const bool live = i < static_cast<uint64_t>(blocks) * 8;
    float4 h = make_float4(0, 0, 0, 0);
    if (live) {
        const float4 g = gate[i], u = up[i];
        h = make_float4(swiglu(g.x, u.x), swiglu(g.y, u.y), swiglu(g.z, u.z), swiglu(g.w, u.w));
    }
    store_q8_lane(h, live, i, values, scales);
}

__global__ void k_dequantize(vkml_dequantize_params p, const void* values, const void* scales, float* out) {
    for (uint64_t e = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < p.count;
         e += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
        out[e] = weight_value(p.quant, p.scale_type, values, scales, p.cols, e / p.cols, e % p.cols);
    }
}

// ---------------------------------------------------------------- norms

// The reference's workgroup reduction at its width of 256 (rms_norm.comp:19-33,
// softmax.comp's reduce_sum): every invocation's value, then the halving
// tree, strides 128 and 64 through LDS and 32 .. 1 within wave 0. Every
// thread gets the result. scratch: 257 floats of LDS.
constexpr uint32_t kRowThreads = 256;

__device__ float tree256_sum(float v, float* scratch) {
    const uint32_t t = threadIdx.x;
    scratch[t] = v;
    __syncthreads();
    if (t < 64) {
        const float s = tree_to_first<64>((scratch[t] + scratch[t + 128]) + (scratch[t + 64] + scratch[t + 192]));
        if (t == 0) scratch[256] = s;
    }
    __syncthreads();
    const float r = scratch[256];
    __syncthreads();
    return r;
}

// Invocation t's sum of x[c]^2 over c = t, t + 256, ... in that order
// (rms_norm.comp:38), its loads issued eight at a time.
__device__ __forceinline__ float strided_sum_sq(const float* xr, uint32_t cols) {
    float s = 0.0f;
    for (uint32_t c0 = threadIdx.x; c0 < cols; c0 += 8 * kRowThreads) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t c = c0 + j * kRowThreads;
            v[j] = c < cols ? xr[c] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (c0 + j * kRowThreads < cols) s += v[j] * v[j];
    }
    return s;
}

// rms_norm.comp:35-49: invocation t sums x[c]^2 over c = t, t + 256, ...;
// scale = 1 / sqrt(sum / cols + eps); out = x * scale * w.
__global__ void __launch_bounds__(kRowThreads) k_rms_norm(vkml_rms_norm_params p, const float* x, const float* w, float* out) {
    __shared__ float scratch[kRowThreads + 1];
    for (uint32_t row = blockIdx.x; row < p.rows; row += gridDim.x) {
        const float* xr = x + static_cast<uint64_t>(row) * p.cols;
        const float s = tree256_sum(strided_sum_sq(xr, p.cols), scratch);
        const float scale = 1.0f / sqrtf(s / static_cast<float>(p.cols) + p.eps);
#pragma unroll 4
        for (uint32_t c = threadIdx.x; c < p.cols; c += kRowThreads)
            out[static_cast<uint64_t>(row) * p.cols + c] = xr[c] * scale * w[c];
    }
}

// rms_norm followed by quantize.comp's Q8_0 with f32 scales (:100-111): the
// sum in the reference's order, then each thread normalizes float4s of the
// row and the 8 lanes of a 32-value block quantize it together.
__global__ void __launch_bounds__(kRowThreads) k_rms_norm_quantize(vkml_rms_norm_params p, const float* x, const float4* w,
                                                                   float4* out, uint32_t* values, float* scales) {
    __shared__ float scratch[kRowThreads + 1];
    const uint32_t row = blockIdx.x, n4 = p.cols / 4;
    const float* xr = x + static_cast<uint64_t>(row) * p.cols;
    const float s = tree256_sum(strided_sum_sq(xr, p.cols), scratch);
    const float scale = 1.0f / sqrtf(s / static_cast<float>(p.cols) + p.eps);
    const float4* xr4 = reinterpret_cast<const float4*>(xr);
#pragma unroll 4
    for (uint32_t i = threadIdx.x; i < n4; i += kRowThreads) {
        // n4 is a multiple of 8, so the 8 lanes of a block are live together.
        const float4 v = xr4[i], wv = w[i];
        const float4 y = make_float4(v.x * scale * wv.x, v.y * scale * wv.y, v.z * scale * wv.z, v.w * scale * wv.w);
        const uint64_t at = static_cast<uint64_t>(row) * n4 + i;
        if (out) out[at] = y;
        const float absmax = group_max<8>(fmaxf(fmaxf(fabsf(y.x), fabsf(y.y)), fmaxf(fabsf(y.z), fabsf(y.w))));
        const float d = absmax / 127.0f;
        const float inv = d > 0.0f ? 1.0f / d : 0.0f;
        values[at] = (static_cast<uint32_t>(quant_code(y.x, inv)) & 0xFFu) | ((static_cast<uint32_t>(quant_code(y.y, inv)) & 0xFFu) << 8) |
                     ((static_cast<uint32_t>(quant_code(y.z, inv)) & 0xFFu) << 16) | (static_cast<uint32_t>(quant_code(y.w, inv)) << 24);
        if (i % 8 == 0) scales[at / 8] = d;
    }
}

// shaders/softmax.comp:85-124, with its order: strided per-invocation max
// and sum of exp over 256 invocations (over key positions first .. visible,
// column p % ring for a ring), the halving tree, then exp(score - m) *
// (1 / s) in each visible column and 0 elsewhere.
__global__ void __launch_bounds__(kRowThreads) k_softmax(vkml_softmax_params p, const float* x, float* out) {
    __shared__ float scratch[kRowThreads + 1];
    __shared__ float s_max[16];
    const bool ring = p.causal && p.ring != 0;
    for (uint32_t row = blockIdx.x; row < p.rows; row += gridDim.x) {
        const float* xr = x + static_cast<uint64_t>(row) * p.cols;
        uint32_t visible = p.cols, first = 0;
        if (p.causal) {
            visible = row % p.q_len + p.offset + 1;
            if (!ring) visible = min(p.cols, visible);
            if (p.window != 0 && visible > p.window) first = visible - p.window;
        }
        const auto col = [&](uint32_t c) { return ring ? c % p.ring : c; };
        const auto score = [&](uint32_t c) {  // c: a column
            const float s = p.scale * xr[c];
            return p.softcap > 0.0f ? p.softcap * tanhf(fminf(fmaxf(s / p.softcap, -10.0f), 10.0f)) : s;
        };
        float m = -__builtin_inff();
        for (uint32_t c = first + threadIdx.x; c < visible; c += kRowThreads) m = fmaxf(m, score(col(c)));
        m = block_max(m, s_max);
        float s = 0.0f;
        for (uint32_t c = first + threadIdx.x; c < visible; c += kRowThreads) s += vk_expf(score(col(c)) - m);
        s = tree256_sum(s, scratch);
        const float inv = 1.0f / s;
        // column c holds a visible key if it lies within visible - first
        // columns of first's, going round the ring
        const uint32_t first_col = col(first);
        for (uint32_t c = threadIdx.x; c < p.cols; c += kRowThreads) {
            const bool seen = ring ? (c >= first_col ? c - first_col : c + p.ring - first_col) < visible - first : (c >= first && c < visible);
            out[static_cast<uint64_t>(row) * p.cols + c] = seen ? vk_expf(score(c) - m) * inv : 0.0f;
        }
        __syncthreads();
    }
}

// k_softmax for rows of at most 256 * NV columns, in the same order with
// the same operations: a thread's scores (columns first + t, + 256, ...)
// are loaded once, all at once, into registers, and each exp is evaluated
// once and kept for the output, instead of reading the row three times and
// evaluating each exp twice.
template <uint32_t NV>
__global__ void __launch_bounds__(kRowThreads) k_softmax_held(vkml_softmax_params p, const float* x, float* out) {
    __shared__ float scratch[kRowThreads + 1];
    __shared__ float s_max[16];
    for (uint32_t row = blockIdx.x; row < p.rows; row += gridDim.x) {
        const float* xr = x + static_cast<uint64_t>(row) * p.cols;
        float* orow = out + static_cast<uint64_t>(row) * p.cols;
        uint32_t visible = p.cols, first = 0;
        if (p.causal) {
            visible = min(p.cols, row % p.q_len + p.offset + 1);
            if (p.window != 0 && visible > p.window) first = visible - p.window;
        }
        float v[NV];
#pragma unroll
        for (uint32_t i = 0; i < NV; ++i) {
            const uint32_t c = first + threadIdx.x + kRowThreads * i;
            v[i] = c < visible ? xr[c] : 0.0f;
        }
        float m = -__builtin_inff();
#pragma unroll
        for (uint32_t i = 0; i < NV; ++i) {
            if (first + threadIdx.x + kRowThreads * i < visible) {
                float s = p.scale * v[i];
                if (p.softcap > 0.0f) s = p.softcap * tanhf(fminf(fmaxf(s / p.softcap, -10.0f), 10.0f));
                v[i] = s;
                m = fmaxf(m, s);
            }
        }
        m = block_max(m, s_max);
        float s = 0.0f;
#pragma unroll
        for (uint32_t i = 0; i < NV; ++i) {
            if (first + threadIdx.x + kRowThreads * i < visible) {
                v[i] = vk_expf(v[i] - m);
                s += v[i];
            }
        }
        s = tree256_sum(s, scratch);
        const float inv = 1.0f / s;
#pragma unroll
        for (uint32_t i = 0; i < NV; ++i) {
            const uint32_t c = first + threadIdx.x + kRowThreads * i;
            if (c < visible) orow[c] = v[i] * inv;
        }
        for (uint32_t c = threadIdx.x; c < first; c += kRowThreads) orow[c] = 0.0f;
        for (uint32_t c = visible + threadIdx.x; c < p.cols; c += kRowThreads) orow[c] = 0.0f;
        __syncthreads();
    }
}

// ---------------------------------------------------------------- argmax

// (value, column) of the winner of two candidates: larger, or equal and
// earlier; column -1 means none (all NaN so far). shaders/argmax.comp:145-148.
__device__ __forceinline__ void better(float& v, int& c, float ov, int oc) {
    if (oc >= 0 && (c < 0 || ov > v || (ov == v && oc < c))) {
        v = ov;
        c = oc;
    }
}

// The wave's best (value, column) toward lane 0: strides 32 .. 1, lane j
// comparing itself with lane j + o (its butterfly partner j ^ o), so lane 0
// ends with what a shuffle-xor reduction gives it.
__device__ __forceinline__ void argmax_to_first(float& best, int& col) {
    better(best, col, lane_down<32>(best), lane_down_i<32>(col));
    better(best, col, lane_down<16>(best), lane_down_i<16>(col));
    better(best, col, lane_down<8>(best), lane_down_i<8>(col));
    better(best, col, lane_down<4>(best), lane_down_i<4>(col));
    better(best, col, lane_down<2>(best), lane_down_i<2>(col));
    better(best, col, lane_down<1>(best), lane_down_i<1>(col));
}

__device__ __forceinline__ void consider(float& best, int& col, float v, uint32_t c) {
    if (!__builtin_isnan(v) && (col < 0 || v > best)) {
        best = v;
        col = static_cast<int>(c);
    }
}

// Each thread visits its columns in increasing order (a float4 per step
// when the row is 16-byte aligned, four steps' loads at a time), so ties
// keep the earliest; the reduction breaks ties the same way.
__device__ int block_argmax(const float* x, uint32_t cols) {
    __shared__ float s_v[16];
    __shared__ int s_c[16];
    float best = 0.0f;
    int col = -1;
    if (cols % 4 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0) {
        const float4* x4 = reinterpret_cast<const float4*>(x);
        const uint32_t n4 = cols / 4;
        for (uint32_t i0 = threadIdx.x; i0 < n4; i0 += 4 * blockDim.x) {
            float4 v[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t i = i0 + j * blockDim.x;
                v[j] = i < n4 ? x4[i] : make_float4(0, 0, 0, 0);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t i = i0 + j * blockDim.x;
                if (i < n4) {
                    consider(best, col, v[j].x, 4 * i);
                    consider(best, col, v[j].y, 4 * i + 1);
                    consider(best, col, v[j].z, 4 * i + 2);
                    consider(best, col, v[j].w, 4 * i + 3);
                }
            }
        }
    } else {
        for (uint32_t c = threadIdx.x; c < cols; c += blockDim.x) consider(best, col, x[c], c);
    }
    argmax_to_first(best, col);
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    __syncthreads();
    if (lane == 0) {
        s_v[wave] = best;
        s_c[wave] = col;
    }
    __syncthreads();
    if (wave == 0) {
        const int waves = blockDim.x / kWave;
        best = lane < waves ? s_v[lane] : 0.0f;
        col = lane < waves ? s_c[lane] : -1;
        argmax_to_first(best, col);
    }
    return col < 0 ? 0 : col;  // valid in thread 0
}

__global__ void __launch_bounds__(1024) k_argmax(uint32_t rows, uint32_t cols, const float* x, int32_t* out) {
    for (uint32_t row = blockIdx.x; row < rows; row += gridDim.x) {
        const int c = block_argmax(x + static_cast<uint64_t>(row) * cols, cols);
        if (threadIdx.x == 0) out[row] = c;
        __syncthreads();
    }
}

__global__ void __launch_bounds__(1024) k_step_finish(uint32_t vocab, const float* logits, vkml_decode_state* st, int32_t* log,
                                                      uint32_t cap) {
    int tok = 0;
    if (logits) tok = block_argmax(logits, vocab);
    if (threadIdx.x == 0) {
        if (logits) {
            st->token = tok;
            if (log && static_cast<uint32_t>(st->steps) < cap) log[st->steps] = tok;
            st->steps += 1;
        }
        st->position += 1;
    }
}

__global__ void k_state_set(vkml_decode_state* st, int32_t token, int32_t position, int32_t steps) {
    st->token = token;
    st->position = position;
    st->steps = steps;
    st->reserved = 0;
}

// ---------------------------------------------------------------- rope

__global__ void k_rope(vkml_rope_params p, const float* x, const float* table, float* out) {
    const uint32_t rest = p.dim - 2 * p.half_dim;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < static_cast<uint64_t>(p.pairs) + p.copies;
         i += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
        if (i >= p.pairs) {
            const uint64_t q = i - p.pairs;
            const uint64_t at = (q / rest) * p.dim + 2 * p.half_dim + q % rest;
            out[at] = x[at];
            continue;
        }
        const uint64_t row = i / p.half_dim, k = i % p.half_dim;
        const uint64_t pos = p.start_pos + (row / p.heads) % p.seq;
        const uint64_t base = row * p.dim;
        const uint64_t ia = base + (p.style == 0 ? 2 * k : k);
        const uint64_t ib = base + (p.style == 0 ? 2 * k + 1 : k + p.half_dim);
        const float c = table[(pos * p.half_dim + k) * 2], s = table[(pos * p.half_dim + k) * 2 + 1];
        const float a = x[ia], b = x[ib];
        out[ia] = a * c - b * s;
        out[ib] = a * s + b * c;
    }
}

__device__ __forceinline__ void store_cache(void* cache, uint32_t type, uint64_t at, float v) {
    if (type == VKML_F16) static_cast<uint16_t*>(cache)[at] = static_cast<uint16_t>(f32_to_f16_bits(__float_as_uint(v)));
    else static_cast<float*>(cache)[at] = v;
}

// One thread per (token, pair): q pairs, then k pairs (rotated, cast,
// appended), then v pairs. Token t's row of q | k | v starts row_stride
// floats after token t - 1's; q goes heads first, [heads, tokens, head_dim].
__global__ void k_rope_kv_append(vkml_rope_kv_params p, uint32_t tokens, uint32_t row_stride, const float* qkv, const float* table,
                                 float* q_out, void* k_cache, void* v_cache, const vkml_decode_state* st) {
    const uint32_t half = p.head_dim / 2;
    const uint32_t q_pairs = p.heads * half, kv_pairs = p.kv_heads * half, per = q_pairs + 2 * kv_pairs;
    const uint32_t q_dim = p.heads * p.head_dim, kv_dim = p.kv_heads * p.head_dim;
    const uint32_t pos0 = st ? static_cast<uint32_t>(st->position) : p.position;
    const uint64_t total = static_cast<uint64_t>(tokens) * per;
    for (uint64_t g = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; g < total;
         g += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
        const uint32_t t = static_cast<uint32_t>(g / per), i = static_cast<uint32_t>(g % per);
        const uint32_t pos = pos0 + t;
        const uint64_t cache_row = pos % p.capacity;
        const float* row = qkv + static_cast<uint64_t>(t) * row_stride;
        if (i < q_pairs + kv_pairs) {
            const bool is_q = i < q_pairs;
            const uint32_t j = is_q ? i : i - q_pairs;
            const uint32_t head = j / half, k = j % half;
            const uint32_t ia = p.style == 0 ? 2 * k : k, ib = p.style == 0 ? 2 * k + 1 : k + half;
            const float* src = row + (is_q ? 0 : q_dim) + head * p.head_dim;
            float a = src[ia], b = src[ib];
            if (p.rotate) {
                const float c = table[(static_cast<uint64_t>(pos) * half + k) * 2], s = table[(static_cast<uint64_t>(pos) * half + k) * 2 + 1];
                const float ra = a * c - b * s;
                const float rb = a * s + b * c;
                a = ra;
                b = rb;
            }
            if (is_q) {
                float* dst = q_out + (static_cast<uint64_t>(head) * tokens + t) * p.head_dim;
                dst[ia] = a;
                dst[ib] = b;
            } else {
                const uint64_t at = (static_cast<uint64_t>(head) * p.capacity + cache_row) * p.head_dim;
                store_cache(k_cache, p.kv_type, at + ia, a);
                store_cache(k_cache, p.kv_type, at + ib, b);
            }
        } else {
            const uint32_t j = i - q_pairs - kv_pairs;
            const uint32_t head = j / half, e = 2 * (j % half);
            const float* v = row + q_dim + kv_dim + head * p.head_dim;
            const uint64_t at = (static_cast<uint64_t>(head) * p.capacity + cache_row) * p.head_dim;
            store_cache(v_cache, p.kv_type, at + e, v[e]);
            store_cache(v_cache, p.kv_type, at + e + 1, v[e + 1]);
        }
    }
}

// ---------------------------------------------------------------- copies

__global__ void k_cast(uint32_t count, uint32_t src, uint32_t dst, const void* x, void* out) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += stride) {
        if (dst == VKML_F32) {
            static_cast<float*>(out)[i] = load_src(x, i, src);
        } else {
            const uint32_t bits = static_cast<const uint32_t*>(x)[i];
            static_cast<uint16_t*>(out)[i] = static_cast<uint16_t>(dst == VKML_F16 ? f32_to_f16_bits(bits) : f32_to_bf16_bits(bits));
        }
    }
}

__global__ void k_copy_rows(vkml_copy_rows_params p, const uint32_t* src, uint32_t* dst) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < p.count; i += stride) {
        const uint64_t batch = i / p.block, at = i % p.block;
        dst[batch * p.dst_stride + p.dst_start + at] = src[batch * p.src_stride + p.src_start + at];
    }
}

__global__ void k_permute(vkml_permute_params p, const uint32_t* x, uint32_t* out) {
    uint64_t in_stride[6];
    uint64_t s = 1;
    for (int d = static_cast<int>(p.rank) - 1; d >= 0; --d) {
        in_stride[d] = s;
        s *= p.in_shape[d];
    }
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < p.count; i += stride) {
        uint64_t rem = i, src = 0;
        for (int d = static_cast<int>(p.rank) - 1; d >= 0; --d) {
            const uint32_t size = p.in_shape[p.dims[d]];
            src += (rem % size) * in_stride[p.dims[d]];
            rem /= size;
        }
        out[i] = x[src];
    }
}

__global__ void k_binary(uint32_t op, uint32_t count, uint32_t b_count, const float* a, const float* b, float* out) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += stride) {
        const float x = a[i], y = b[i % b_count];
        out[i] = op == 0 ? x + y : op == 1 ? x - y : op == 2 ? x * y : x / y;
    }
}

__global__ void k_unary(uint32_t op, uint32_t count, float param, const float* x, float* out) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += stride) {
        const float v = x[i];
        float r;
        if (op == 0) {
            r = v / (1.0f + vk_expf(-v));
        } else if (op == 1) {
            const float inner = fminf(fmaxf(0.7978845608f * (v + 0.044715f * v * v * v), -10.0f), 10.0f);
            r = 0.5f * v * (1.0f + tanhf(inner));
        } else {
            r = param * tanhf(fminf(fmaxf(v / param, -10.0f), 10.0f));
        }
        out[i] = r;
    }
}

__global__ void k_embedding(vkml_embedding_params p, const void* values, const void* scales, const int32_t* ids,
                            const vkml_decode_state* st, float* out) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < p.count; i += stride) {
        const int32_t id = st ? st->token : ids[i / p.dim];
        const uint64_t col = i % p.dim;
        out[i] = (id >= 0 && static_cast<uint32_t>(id) < p.vocab)
                     ? weight_value(p.table_type, p.scale_type, values, scales, p.dim, static_cast<uint64_t>(id), col)
                     : 0.0f;
    }
}

// ---------------------------------------------------------------- matmul

// matmul.comp's order: every output sums a[m][k] * b(k, n) in k order, a
// product and an add at a time (matmul.comp:131-140). A 256-thread
// workgroup computes a 64 x 64 block of c, each thread the 4 x 4 outputs at
// rows 4 ty.., columns 4 tx..; K steps by 16 through LDS, both tiles stored
// k-major so a thread reads its 4 rows and 4 columns as one 16-byte word
// each. b is f32/f16/bf16, or (transposed, one batch) a quantized matrix
// widened as gemv's weights are.
// Four consecutive elements of a float b (f32, or f16/bf16 bits) at element e
// (a multiple of 4, the row's base aligned), widened to f32.
template <uint32_t BTYPE>
__device__ __forceinline__ float4 load_b4(const void* b, uint64_t e) {
    if constexpr (BTYPE == VKML_F32) {
        return *reinterpret_cast<const float4*>(static_cast<const float*>(b) + e);
    } else {
        const uint2 w = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(b) + e);
        return make_float4(half_to_float(w.x & 0xFFFFu, BTYPE), half_to_float(w.x >> 16, BTYPE), half_to_float(w.y & 0xFFFFu, BTYPE),
                           half_to_float(w.y >> 16, BTYPE));
    }
}

// VEC (float b, rows of a and of b whole vec4s, aligned): each thread loads
// a's and b's tile elements as one vec4 each instead of four scalars.
template <bool BT, uint32_t BTYPE, bool VEC = false>
__global__ void __launch_bounds__(256) k_matmul(vkml_matmul_params p, const float* a, const void* b, const void* bs, float* c) {
    // Rows of 68: stores that run along k hit 16 different banks.
    __shared__ __align__(16) float ta[16][68], tb[16][68];
    const uint32_t tid = threadIdx.x, tx = tid % 16, ty = tid / 16;
    const uint32_t row0 = blockIdx.y * 64, col0 = blockIdx.x * 64, z = blockIdx.z;
    // Under a causal mask the tile's last row sees keys up to row0 + 63 +
    // offset: scores past it are never read, and a's entries past it are 0.
    const uint64_t last_key = static_cast<uint64_t>(row0) + 63 + p.causal_offset;
    if (BT && p.causal && col0 > last_key) return;
    const uint32_t k_end = (!BT && p.causal) ? static_cast<uint32_t>(min<uint64_t>(p.k, last_key + 1)) : p.k;
    const float* az = a + static_cast<uint64_t>(z) * p.m * p.k;
    const uint64_t b_off = static_cast<uint64_t>(z / p.b_group) * p.b_stride;
    const auto b_at = [&](uint32_t n, uint32_t k) -> float {
        if constexpr (BTYPE >= VKML_Q8_0) {
            return weight_value(BTYPE, p.scale_type, b, bs, p.k, n, k);
        } else {
            const uint64_t e = b_off + (BT ? static_cast<uint64_t>(n) * p.k + k : static_cast<uint64_t>(k) * p.n + n);
            return load_src(b, e, BTYPE);
        }
    };
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;
    for (uint32_t k0 = 0; k0 < k_end; k0 += 16) {
        // Out-of-range elements are zeros, which add nothing.
        if constexpr (VEC) {
            {  // a: row tid / 4, k0 + 4 (tid % 4) ..
                const uint32_t r = tid / 4, kq = tid % 4, row = row0 + r, k = k0 + 4 * kq;
                float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if (row < p.m && k < p.k) v = *reinterpret_cast<const float4*>(az + static_cast<uint64_t>(row) * p.k + k);
                ta[4 * kq][r] = v.x;
                ta[4 * kq + 1][r] = v.y;
                ta[4 * kq + 2][r] = v.z;
                ta[4 * kq + 3][r] = v.w;
            }
            if constexpr (BT) {  // b [n, k]: column tid / 4, k0 + 4 (tid % 4) ..
                const uint32_t col = tid / 4, kq = tid % 4, n = col0 + col, kg = k0 + 4 * kq;
                float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if (n < p.n && kg < p.k) v = load_b4<BTYPE>(b, b_off + static_cast<uint64_t>(n) * p.k + kg);
                tb[4 * kq][col] = v.x;
                tb[4 * kq + 1][col] = v.y;
                tb[4 * kq + 2][col] = v.z;
                tb[4 * kq + 3][col] = v.w;
            } else {  // b [k, n]: k0 + tid / 16, columns 4 (tid % 16) ..
                const uint32_t kb = tid / 16, cq = tid % 16, n = col0 + 4 * cq, kg = k0 + kb;
                float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if (n < p.n && kg < p.k) v = load_b4<BTYPE>(b, b_off + static_cast<uint64_t>(kg) * p.n + n);
                *reinterpret_cast<float4*>(&tb[kb][4 * cq]) = v;
            }
        } else {
#pragma unroll
        for (uint32_t u = 0; u < 4; ++u) {
            const uint32_t e = tid + 256 * u;
            const uint32_t r = e / 16, kk = e % 16, row = row0 + r, k = k0 + kk;
            ta[kk][r] = (row < p.m && k < p.k) ? az[static_cast<uint64_t>(row) * p.k + k] : 0.0f;
            uint32_t col, kb;
            if (BT) {  // b is [n, k]: run along k
                col = e / 16;
                kb = e % 16;
            } else {  // b is [k, n]: run along n
                kb = e / 64;
                col = e % 64;
            }
            const uint32_t n = col0 + col, kg = k0 + kb;
            tb[kb][col] = (n < p.n && kg < p.k) ? b_at(n, kg) : 0.0f;
        }
        }
        __syncthreads();
#pragma unroll
        for (uint32_t kk = 0; kk < 16; ++kk) {
            const float4 av = *reinterpret_cast<const float4*>(&ta[kk][4 * ty]);
            const float4 bv = *reinterpret_cast<const float4*>(&tb[kk][4 * tx]);
            const float ar[4] = {av.x, av.y, av.z, av.w}, br[4] = {bv.x, bv.y, bv.z, bv.w};
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] += ar[i] * br[j];
        }
        __syncthreads();
    }
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i) {
        const uint32_t row = row0 + 4 * ty + i;
        if (row >= p.m) continue;
        float* cr = c + (static_cast<uint64_t>(z) * p.m + row) * p.n;
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
            const uint32_t col = col0 + 4 * tx + j;
            if (col < p.n) cr[col] = acc[i][j];
        }
    }
}

}  // namespace

extern "C" {

int vkml_quantize(const vkml_quantize_params* p, const void* x, void* values, void* scales) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(p, "quantize: null params");
    VKML_CHECK_ARG(p->src_type <= VKML_BF16, "quantize: source must be f32, f16 or bf16");
    VKML_CHECK_ARG(p->quant == VKML_Q8_0 || p->quant == VKML_Q4_0 || p->quant == VKML_Q4_1, "quantize: format must be q8_0, q4_0 or q4_1");
    VKML_CHECK_ARG(p->scale_type == VKML_F32 || p->scale_type == VKML_F16, "quantize: scales must be f32 or f16");
    if (p->blocks == 0) return VKML_OK;
    VKML_CHECK_ARG(x && values && scales, "quantize: null buffer");
    if (p->src_type == VKML_F32 && p->quant == VKML_Q8_0 && p->scale_type == VKML_F32) {
        ProfileScope prof("quantize");
        const uint64_t threads = static_cast<uint64_t>(p->blocks) * 8;
        hipLaunchKernelGGL(k_quantize_act, dim3(static_cast<uint32_t>((threads + 255) / 256)), dim3(256), 0, S(), p->blocks,
                           static_cast<const float4*>(x), static_cast<uint32_t*>(values), static_cast<float*>(scales));
        return vkml::abi::check_launch("quantize");
    }
    ProfileScope prof("quantize");
    hipLaunchKernelGGL(k_quantize, dim3(blocks_for(p->blocks)), dim3(256), 0, S(), *p, x, static_cast<uint32_t*>(values), scales);
    return vkml::abi::check_launch("quantize");
}

int vkml_swiglu_quantize(uint32_t count, const float* gate, const float* up, void* values, float* scales) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(count % 32 == 0, "swiglu_quantize: count = " + std::to_string(count) + " must be a multiple of 32");
    if (count == 0) return VKML_OK;
    VKML_CHECK_ARG(gate && up && values && scales, "swiglu_quantize: null buffer");
    VKML_CHECK_ARG(reinterpret_cast<uintptr_t>(gate) % 16 == 0 && reinterpret_cast<uintptr_t>(up) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(values) % 4 == 0 && reinterpret_cast<uintptr_t>(scales) % 4 == 0,
                   "swiglu_quantize: gate and up must be 16-byte aligned, values and scales 4-byte aligned");
    ProfileScope prof("swiglu_quantize");
    const uint64_t threads = count / 4;
    hipLaunchKernelGGL(k_swiglu_quantize, dim3(static_cast<uint32_t>((threads + 255) / 256)), dim3(256), 0, S(), count / 32,
                       reinterpret_cast<const float4*>(gate), reinterpret_cast<const float4*>(up), static_cast<uint32_t*>(values), scales);
    return vkml::abi::check_launch("swiglu_quantize");
}

int vkml_dequantize(const vkml_dequantize_params* p, const void* values, const void* scales, float* out) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(p, "dequantize: null params");
    VKML_CHECK_ARG(p->quant >= VKML_Q8_0 && p->quant <= VKML_Q4_K, "dequantize: not a quantized format");
    VKML_CHECK_ARG(p->cols > 0 && p->count % p->cols == 0 && p->cols % (p->quant == VKML_Q4_K ? 256 : 32) == 0,
                   "dequantize: rows must be whole blocks");
    if (p->count == 0) return VKML_OK;
    VKML_CHECK_ARG(values && scales && out, "dequantize: null buffer");
    ProfileScope prof("dequantize");
    hipLaunchKernelGGL(k_dequantize, dim3(blocks_for(p->count)), dim3(256), 0, S(), *p, values, scales, out);
    return vkml::abi::check_launch("dequantize");
}

int vkml_rms_norm(const vkml_rms_norm_params* p, const float* x, const float* w, float* out) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(p, "rms_norm: null params");
    if (p->rows == 0 || p->cols == 0) return VKML_OK;
    VKML_CHECK_ARG(x && w && out, "rms_norm: null buffer");
    ProfileScope prof("rms_norm");
    hipLaunchKernelGGL(k_rms_norm, dim3(std::min<uint32_t>(p->rows, 65535)), dim3(kRowThreads), 0, S(), *p, x, w, out);
    return vkml::abi::check_launch("rms_norm");
}

int vkml_rms_norm_quantize(const vkml_rms_norm_params* p, const float* x, const float* w, float* out, void* values,
                           float* scales) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(p, "rms_norm_quantize: null params");
    VKML_CHECK_ARG(p->cols % 32 == 0, "rms_norm_quantize: columns must be a multiple of 32, got " + std::to_string(p->cols));
    VKML_CHECK_ARG(p->rows <= 65535, "rms_norm_quantize: too many rows");
    if (p->rows == 0 || p->cols == 0) return VKML_OK;
    VKML_CHECK_ARG(x && w && values && scales, "rms_norm_quantize: null buffer");
    ProfileScope prof("rms_norm_quantize");
    hipLaunchKernelGGL(k_rms_norm_quantize, dim3(p->rows), dim3(kRowThreads), 0, S(), *p, x, reinterpret_cast<const float4*>(w),
                       reinterpret_cast<float4*>(out), static_cast<uint32_t*>(values), scales);
    return vkml::abi::check_launch("rms_norm_quantize");
}

int vkml_softmax(const vkml_softmax_params* p, const float* x, float* out) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(p, "softmax: null params");
    VKML_CHECK_ARG(!p->causal || p->q_len > 0, "softmax: causal rows need q_len");
    VKML_CHECK_ARG(!p->ring || (p->causal && p->cols <= p->ring), "softmax: a ring needs the causal mask and at most ring columns");
    // A row's visible positions must fit the ring, or they would wrap onto each other.
    VKML_CHECK_ARG(!p->ring || (p->window >= 1 && p->window <= p->ring),
                   "softmax: a ring needs a window of 1 to " + std::to_string(p->ring) + " positions, got " + std::to_string(p->window));
    if (p->rows == 0 || p->cols == 0) return VKML_OK;
    VKML_CHECK_ARG(x && out, "softmax: null buffer");
    ProfileScope prof("softmax");
    const dim3 grid(std::min<uint32_t>(p->rows, 65535)), block(kRowThreads);
    if (p->ring) hipLaunchKernelGGL(k_softmax, grid, block, 0, S(), *p, x, out);
    else if (p->cols <= kRowThreads * 4) hipLaunchKernelGGL(k_softmax_held<4>, grid, block, 0, S(), *p, x, out);
    else if (p->cols <= kRowThreads * 8) hipLaunchKernelGGL(k_softmax_held<8>, grid, block, 0, S(), *p, x, out);
    else if (p->cols <= kRowThreads * 16) hipLaunchKernelGGL(k_softmax_held<16>, grid, block, 0, S(), *p, x, out);
    else hipLaunchKernelGGL(k_softmax, grid, block, 0, S(), *p, x, out);
    return vkml::abi::check_launch("softmax");
}

int vkml_argmax(uint32_t rows, uint32_t cols, const float* x, int32_t* out) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(cols > 0 || rows == 0, "argmax: the last dimension is empty");
    if (rows == 0) return VKML_OK;
    VKML_CHECK_ARG(x && out, "argmax: null buffer");
    ProfileScope prof("argmax");
    hipLaunchKernelGGL(k_argmax, dim3(std::min<uint32_t>(rows, 65535)), dim3(1024), 0, S(), rows, cols, x, out);
    return vkml::abi::check_launch("argmax");
}

int vkml_rope(const vkml_rope_params* p, const float* x, const float* table, float* out) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(p, "rope: null params");
    VKML_CHECK_ARG(p->half_dim > 0 && 2 * p->half_dim <= p->dim && p->heads > 0 && p->seq > 0, "rope: bad shape");
    const uint64_t total = static_cast<uint64_t>(p->pairs) + p->copies;
    if (total == 0) return VKML_OK;
    VKML_CHECK_ARG(x && table && out, "rope: null buffer");
    ProfileScope prof("rope");
    hipLaunchKernelGGL(k_rope, dim3(blocks_for(total)), dim3(256), 0, S(), *p, x, table, out);
    return vkml::abi::check_launch("rope");
}

int vkml_rope_kv_append(const vkml_rope_kv_params* p, const float* qkv, const float* table, float* q, void* k_cache,
                        void* v_cache, const vkml_decode_state* state) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(p, "rope_kv_append: null params");
    VKML_CHECK_ARG(p->head_dim % 2 == 0 && p->kv_heads > 0 && p->heads % p->kv_heads == 0 && p->capacity > 0,
                   "rope_kv_append: bad head layout");
    VKML_CHECK_ARG(p->kv_type == VKML_F16 || p->kv_type == VKML_F32, "rope_kv_append: caches must be f16 or f32");
    VKML_CHECK_ARG(qkv && q && k_cache && v_cache && (table || !p->rotate), "rope_kv_append: null buffer");
    const uint32_t n = (p->heads + 2 * p->kv_heads) * (p->head_dim / 2);
    ProfileScope prof("rope_kv_append");
    hipLaunchKernelGGL(k_rope_kv_append, dim3((n + 255) / 256), dim3(256), 0, S(), *p, 1u, 0u, qkv, table, q, k_cache, v_cache, state);
    return vkml::abi::check_launch("rope_kv_append");
}

int vkml_rope_kv_prompt(const vkml_rope_kv_params* p, uint32_t tokens, uint32_t row_stride, const float* qkv, const float* table,
                        float* q, void* k_cache, void* v_cache) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(p, "rope_kv_prompt: null params");
    VKML_CHECK_ARG(p->head_dim % 2 == 0 && p->kv_heads > 0 && p->heads % p->kv_heads == 0 && p->capacity > 0,
                   "rope_kv_prompt: bad head layout");
    VKML_CHECK_ARG(p->kv_type == VKML_F16 || p->kv_type == VKML_F32, "rope_kv_prompt: caches must be f16 or f32");
    VKML_CHECK_ARG(row_stride >= (p->heads + 2 * p->kv_heads) * p->head_dim, "rope_kv_prompt: rows overlap");
    VKML_CHECK_ARG(tokens <= p->capacity,
                   "rope_kv_prompt: " + std::to_string(tokens) + " tokens from position " + std::to_string(p->position) +
                       " do not fit a cache of " + std::to_string(p->capacity) + " rows");
    if (tokens == 0) return VKML_OK;
    VKML_CHECK_ARG(qkv && q && k_cache && v_cache && (table || !p->rotate), "rope_kv_prompt: null buffer");
    const uint64_t n = static_cast<uint64_t>(tokens) * (p->heads + 2 * p->kv_heads) * (p->head_dim / 2);
    ProfileScope prof("rope_kv_prompt");
    hipLaunchKernelGGL(k_rope_kv_append, dim3(blocks_for(n)), dim3(256), 0, S(), *p, tokens, row_stride, qkv, table, q, k_cache, v_cache,
                       nullptr);
    return vkml::abi::check_launch("rope_kv_prompt");
}


int vkml_cast(uint32_t count, uint32_t src, uint32_t dst, const void* x, void* out) {
    VKML_REQUIRE_INIT();
    const bool ok = (dst == VKML_F32 && src <= VKML_BF16) || (src == VKML_F32 && (dst == VKML_F16 || dst == VKML_BF16));
    VKML_CHECK_ARG(ok, "cast: from " + std::to_string(src) + " to " + std::to_string(dst) + " is not implemented");
    if (count == 0) return VKML_OK;
    VKML_CHECK_ARG(x && out, "cast: null buffer");
    ProfileScope prof("cast");
    hipLaunchKernelGGL(k_cast, dim3(blocks_for(count)), dim3(256), 0, S(), count, src, dst, x, out);
    return vkml::abi::check_launch("cast");
}

int vkml_copy_rows(const vkml_copy_rows_params* p, const void* src, void* dst) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(p, "copy_rows: null params");
    if (p->count == 0) return VKML_OK;
    VKML_CHECK_ARG(src && dst && p->block > 0, "copy_rows: null buffer");
    ProfileScope prof("write_rows");
    hipLaunchKernelGGL(k_copy_rows, dim3(blocks_for(p->count)), dim3(256), 0, S(), *p, static_cast<const uint32_t*>(src),
                       static_cast<uint32_t*>(dst));
    return vkml::abi::check_launch("copy_rows");
}

int vkml_permute(const vkml_permute_params* p, const void* x, void* out) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(p && p->rank >= 1 && p->rank <= 6, "permute: rank must be 1 to 6");
    uint32_t seen = 0;
    for (uint32_t d = 0; d < p->rank; ++d) {
        VKML_CHECK_ARG(p->dims[d] < p->rank && !(seen & (1u << p->dims[d])), "permute: dims must be a permutation");
        seen |= 1u << p->dims[d];
    }
    if (p->count == 0) return VKML_OK;
    VKML_CHECK_ARG(x && out, "permute: null buffer");
    ProfileScope prof("permute");
    hipLaunchKernelGGL(k_permute, dim3(blocks_for(p->count)), dim3(256), 0, S(), *p, static_cast<const uint32_t*>(x),
                       static_cast<uint32_t*>(out));
    return vkml::abi::check_launch("permute");
}

int vkml_binary(uint32_t op, uint32_t count, uint32_t b_count, const float* a, const float* b, float* out) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(op <= 3, "binary: unknown op");
    if (count == 0) return VKML_OK;
    VKML_CHECK_ARG(b_count > 0 && a && b && out, "binary: null buffer");
    ProfileScope prof("binary");
    hipLaunchKernelGGL(k_binary, dim3(blocks_for(count)), dim3(256), 0, S(), op, count, b_count, a, b, out);
    return vkml::abi::check_launch("binary");
}

int vkml_unary(uint32_t op, uint32_t count, float param, const float* x, float* out) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(op <= 2, "unary: unknown op");
    VKML_CHECK_ARG(op != 2 || param > 0.0f, "softcap: the cap must be positive");
    if (count == 0) return VKML_OK;
    VKML_CHECK_ARG(x && out, "unary: null buffer");
    ProfileScope prof("unary");
    hipLaunchKernelGGL(k_unary, dim3(blocks_for(count)), dim3(256), 0, S(), op, count, param, x, out);
    return vkml::abi::check_launch("unary");
}

static int embedding_checks(const vkml_embedding_params* p) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(p, "embedding: null params");
    VKML_CHECK_ARG(p->table_type <= VKML_Q4_K, "embedding: unknown table type");
    VKML_CHECK_ARG(p->dim > 0 && p->count % p->dim == 0, "embedding: count must be whole rows");
    if (p->table_type >= VKML_Q8_0)
        VKML_CHECK_ARG(p->dim % (p->table_type == VKML_Q4_K ? 256 : 32) == 0, "embedding: rows must be whole blocks");
    return VKML_OK;
}

int vkml_embedding(const vkml_embedding_params* p, const void* values, const void* scales, const int32_t* ids, float* out) {
    if (int r = embedding_checks(p)) return r;
    if (p->count == 0) return VKML_OK;
    VKML_CHECK_ARG(values && ids && out && (p->table_type < VKML_Q8_0 || scales), "embedding: null buffer");
    ProfileScope prof("embedding");
    hipLaunchKernelGGL(k_embedding, dim3(blocks_for(p->count)), dim3(256), 0, S(), *p, values, scales, ids,
                       static_cast<const vkml_decode_state*>(nullptr), out);
    return vkml::abi::check_launch("embedding");
}

int vkml_embedding_state(const vkml_embedding_params* p, const void* values, const void* scales, const vkml_decode_state* state,
                         float* out) {
    if (int r = embedding_checks(p)) return r;
    VKML_CHECK_ARG(p->count == p->dim, "embedding_state: one row");
    VKML_CHECK_ARG(values && state && out && (p->table_type < VKML_Q8_0 || scales), "embedding_state: null buffer");
    ProfileScope prof("embedding");
    hipLaunchKernelGGL(k_embedding, dim3(blocks_for(p->count)), dim3(256), 0, S(), *p, values, scales,
                       static_cast<const int32_t*>(nullptr), state, out);
    return vkml::abi::check_launch("embedding_state");
}

int vkml_state_set(vkml_decode_state* state, int32_t token, int32_t position, int32_t steps) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(state, "state_set: null state");
    ProfileScope prof("state_set");
    hipLaunchKernelGGL(k_state_set, dim3(1), dim3(1), 0, S(), state, token, position, steps);
    return vkml::abi::check_launch("state_set");
}

int vkml_step_finish(uint32_t vocab, const float* logits, vkml_decode_state* state, int32_t* log, uint32_t cap) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(state, "step_finish: null state");
    VKML_CHECK_ARG(!logits || vocab > 0, "step_finish: empty vocabulary");
    ProfileScope prof(logits ? "argmax" : "step_finish");
    hipLaunchKernelGGL(k_step_finish, dim3(1), dim3(1024), 0, S(), vocab, logits, state, log, cap);
    return vkml::abi::check_launch("step_finish");
}

int vkml_matmul(const vkml_matmul_params* p, const float* a, const void* b, float* c, const void* b_scales) {
    VKML_REQUIRE_INIT();
    VKML_CHECK_ARG(p, "matmul: null params");
    VKML_CHECK_ARG(p->b_type <= VKML_Q4_K, "matmul: unknown b type " + std::to_string(p->b_type));
    VKML_CHECK_ARG(p->b_group >= 1 && p->batches >= 1, "matmul: bad batching");
    const bool quant = p->b_type >= VKML_Q8_0;
    VKML_CHECK_ARG(!p->causal || !quant, "matmul: the causal skip is for attention's products, not weights");
    if (quant) {
        VKML_CHECK_ARG(p->b_transposed && p->batches == 1, "matmul: quantized b must be one transposed [n, k] matrix");
        const uint32_t unit = p->b_type == VKML_Q4_K ? 256 : 32;
        VKML_CHECK_ARG(p->k % unit == 0, "matmul: k = " + std::to_string(p->k) + " is not whole blocks of " + std::to_string(unit));
        VKML_CHECK_ARG(p->scale_type == VKML_F16 || (p->scale_type == VKML_F32 && p->b_type != VKML_Q4_K),
                       "matmul: bad scale type");
        VKML_CHECK_ARG(b_scales, "matmul: quantized b needs scales");
    }
    if (p->m == 0 || p->n == 0) return VKML_OK;
    VKML_CHECK_ARG(a && b && c, "matmul: null buffer");
    VKML_CHECK_ARG((p->m + 63) / 64 <= 65535 && p->batches <= 65535, "matmul: too many rows or batches");
    const dim3 grid((p->n + 63) / 64, (p->m + 63) / 64, p->batches);
    ProfileScope prof("matmul");
    const bool t = p->b_transposed != 0;
    // Whole, aligned vec4s along k in a's rows (and b's when transposed),
    // along n in b's rows otherwise.
    const bool vec = p->b_type <= VKML_BF16 && p->k % 4 == 0 && (t || p->n % 4 == 0) && p->b_stride % 4 == 0 &&
                     reinterpret_cast<uintptr_t>(a) % 16 == 0 && reinterpret_cast<uintptr_t>(b) % (p->b_type == VKML_F32 ? 16 : 8) == 0;
    if (vec) {
        const auto launch = [&](auto kernel) { hipLaunchKernelGGL(kernel, grid, dim3(256), 0, S(), *p, a, b, b_scales, c); };
        if (p->b_type == VKML_F32) t ? launch(k_matmul<true, VKML_F32, true>) : launch(k_matmul<false, VKML_F32, true>);
        else if (p->b_type == VKML_F16) t ? launch(k_matmul<true, VKML_F16, true>) : launch(k_matmul<false, VKML_F16, true>);
        else t ? launch(k_matmul<true, VKML_BF16, true>) : launch(k_matmul<false, VKML_BF16, true>);
        return vkml::abi::check_launch("matmul");
    }
    switch (p->b_type) {
        case VKML_F32:
            if (t) hipLaunchKernelGGL((k_matmul<true, VKML_F32>), grid, dim3(256), 0, S(), *p, a, b, b_scales, c);
            else hipLaunchKernelGGL((k_matmul<false, VKML_F32>), grid, dim3(256), 0, S(), *p, a, b, b_scales, c);
            break;
        case VKML_F16:
            if (t) hipLaunchKernelGGL((k_matmul<true, VKML_F16>), grid, dim3(256), 0, S(), *p, a, b, b_scales, c);
            else hipLaunchKernelGGL((k_matmul<false, VKML_F16>), grid, dim3(256), 0, S(), *p, a, b, b_scales, c);
            break;
        case VKML_BF16:
            if (t) hipLaunchKernelGGL((k_matmul<true, VKML_BF16>), grid, dim3(256), 0, S(), *p, a, b, b_scales, c);
            else hipLaunchKernelGGL((k_matmul<false, VKML_BF16>), grid, dim3(256), 0, S(), *p, a, b, b_scales, c);
            break;
        case VKML_Q8_0: hipLaunchKernelGGL((k_matmul<true, VKML_Q8_0>), grid, dim3(256), 0, S(), *p, a, b, b_scales, c); break;
        case VKML_Q4_0: hipLaunchKernelGGL((k_matmul<true, VKML_Q4_0>), grid, dim3(256), 0, S(), *p, a, b, b_scales, c); break;
        case VKML_Q4_1: hipLaunchKernelGGL((k_matmul<true, VKML_Q4_1>), grid, dim3(256), 0, S(), *p, a, b, b_scales, c); break;
        default: hipLaunchKernelGGL((k_matmul<true, VKML_Q4_K>), grid, dim3(256), 0, S(), *p, a, b, b_scales, c); break;
    }
    return vkml::abi::check_launch("matmul");
}


}  // extern "C"
