// device.hpp -- gfx950 device helpers shared by the kernels: 16-bit float
// conversions, wave64 reductions, int8 dot products and the weight decoders.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vkml::dev {

constexpr int kWave = 64;

// ---------------------------------------------------------------- 16-bit floats

// f16 bits to f32, exactly (v_cvt_f32_f16 keeps f16 subnormals: the f16
// denormal mode is IEEE on gfx9).
__device__ __forceinline__ float f16_bits_to_float(uint32_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
}

// f32 to f16 and back, round to nearest even, as the reference rounds
// q4_K's products (src/io/gguf.cpp:609-617); finite inputs only.
__device__ __forceinline__ float round_to_f16(float x) {
    return static_cast<float>(static_cast<_Float16>(x));
}

// f32 bits to f16 bits rounding to nearest even on the bits, so no input is
// flushed (the reference's to_f16, shaders/include/halves.glsl:73-91).
__device__ __forceinline__ uint32_t f32_to_f16_bits(uint32_t bits) {
    const uint32_t sign = (bits >> 16) & 0x8000u;
    const uint32_t a = bits & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return sign | 0x7E00u;
    if (a >= 0x477FF000u) return sign | 0x7C00u;
    if (a < 0x38800000u) {
        const uint32_t e = a >> 23;
        if (e < 102u) return sign;
        const uint32_t m = (a & 0x7FFFFFu) | 0x800000u;
        const uint32_t shift = 126u - e;
        uint32_t q = m >> shift;
        const uint32_t rest = m & ((1u << shift) - 1u), half = 1u << (shift - 1u);
        if (rest > half || (rest == half && (q & 1u) != 0u)) q += 1u;
        return sign | q;
    }
    return sign | ((a + 0xFFFu + ((a >> 13) & 1u) - 0x38000000u) >> 13);
}

// shaders/cast.comp:30-35
__device__ __forceinline__ uint32_t f32_to_bf16_bits(uint32_t bits) {
    if ((bits & 0x7FFFFFFFu) > 0x7F800000u) return (bits >> 16) | 0x40u;
    return (bits + 0x7FFFu + ((bits >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ float bf16_bits_to_float(uint32_t h) { return __uint_as_float(h << 16); }

__device__ __forceinline__ float half_to_float(uint32_t h, uint32_t type) {
    return type == 2 ? bf16_bits_to_float(h) : f16_bits_to_float(h);
}

// ---------------------------------------------------------------- exp

// e^x in f32 with a fixed sequence of IEEE operations, so the CPU oracle
// (oracle/vkml_oracle.c, orc_expf) computes the same bits: the reference's
// GLSL exp has driver-defined accuracy, and softmax weights and SiLU feed
// the int8 quantizer, where one ulp can move a code. Method: Cody-Waite
// range reduction x = n ln2 + r, |r| <= ln2/2, with ln2 split in a 15-bit
// head and a tail; e^r by its degree-7 Taylor polynomial in Horner form
// (truncation below 6e-9 relative); the result scaled by 2^n through the
// exponent bits. Below -86.5 (e^x < 2.7e-38) the result is 0, above
// 88.72 infinity.
__device__ __forceinline__ float vk_expf(float x) {
#pragma clang fp contract(off)
    if (!(x == x)) return x;
    if (x > 88.72283935546875f) return __builtin_inff();
    if (x < -86.5f) return 0.0f;
    const float n = __builtin_rintf(x * 1.44269502162933349609375f);
    const float r = (x - n * 0.693145751953125f) - n * 1.428606765330187045037746429443359375e-6f;
    float p = 1.98412701138295233249664306640625e-4f;
    p = p * r + 1.388888922519981861114501953125e-3f;
    p = p * r + 8.333333767950534820556640625e-3f;
    p = p * r + 4.16666679084300994873046875e-2f;
    p = p * r + 1.6666667163372039794921875e-1f;
    p = p * r + 0.5f;
    p = p * r + 1.0f;
    p = p * r + 1.0f;
    const int e = static_cast<int>(n);
    if (e > 127) return p * 1.70141183460469231731687303715884105728e38f * 2.0f;
    return p * __int_as_float((e + 127) << 23);
}

// ---------------------------------------------------------------- lane moves

// Cross-lane moves that stay in the VALU: DPP (gfx9 controls: quad
// permutations, mirrors within 8 and 16 lanes, shifts within a 16-lane row)
// and gfx950's v_permlane16_swap / v_permlane32_swap, instead of
// ds_bpermute's round trip through the LDS unit.
namespace dpp {
constexpr int kXor1 = 0xB1;        // quad_perm [1, 0, 3, 2]
constexpr int kXor2 = 0x4E;        // quad_perm [2, 3, 0, 1]
constexpr int kXor3 = 0x1B;        // quad_perm [3, 2, 1, 0]
constexpr int kHalfMirror = 0x141;  // lane i of 8 reads lane 7 - i
constexpr int kMirror = 0x140;      // lane i of 16 reads lane 15 - i
constexpr int shl(int n) { return 0x100 + n; }  // lane i reads lane i + n of its row (0 past the row)
}  // namespace dpp

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xF, 0xF, true));
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) { return __uint_as_float(dpp_u<CTRL>(__float_as_uint(v))); }
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) { return static_cast<int>(dpp_u<CTRL>(static_cast<uint32_t>(v))); }

// A swap of v between neighbouring 16-lane rows (W = 16: rows 0/1, 2/3) or
// wave halves (W = 32): .x is v on the lower row or half and the partner's v
// on the upper; .y the partner's v on the lower and v on the upper. So
// {.x, .y} is {own, partner} on every lane, and .y carries lane i + W to
// lane i of the lower one.
template <int W>
__device__ __forceinline__ uint2 swap_rows(uint32_t v) {
    if constexpr (W == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return make_uint2(r[0], r[1]);
    } else {
        const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return make_uint2(r[0], r[1]);
    }
}

// Lane i + O's value (O a power of two <= 32) on lanes 0 .. O - 1 of every
// 2 O-lane group: what a halving tree's step at stride O reads. Other lanes
// get unspecified values, so a tree of descending strides over them is
// valid at each group's first lane.
template <int O>
__device__ __forceinline__ uint32_t lane_down_u(uint32_t v) {
    if constexpr (O >= 16) return swap_rows<O>(v).y;
    else return dpp_u<dpp::shl(O)>(v);
}
template <int O>
__device__ __forceinline__ float lane_down(float v) { return __uint_as_float(lane_down_u<O>(__float_as_uint(v))); }
template <int O>
__device__ __forceinline__ int lane_down_i(int v) { return static_cast<int>(lane_down_u<O>(static_cast<uint32_t>(v))); }

// A halving tree's strides W / 2 .. 1 toward the first lane of each W-lane
// group: lane j < o adds lane j + o, which is also its butterfly partner
// j ^ o, so the first lane's sum is the one a shuffle-xor tree gives it.
template <int W>
__device__ __forceinline__ float tree_to_first(float v) {
#pragma clang fp contract(off)
    if constexpr (W >= 64) v += lane_down<32>(v);
    if constexpr (W >= 32) v += lane_down<16>(v);
    if constexpr (W >= 16) v += lane_down<8>(v);
    if constexpr (W >= 8) v += lane_down<4>(v);
    if constexpr (W >= 4) v += lane_down<2>(v);
    if constexpr (W >= 2) v += lane_down<1>(v);
    return v;
}

// ---------------------------------------------------------------- reductions

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}
// Max over groups of `width` consecutive lanes (a power of two <= 64), on
// every lane of the group (max is exact in any order).
template <int width>
__device__ __forceinline__ float group_max(float v) {
    if constexpr (width >= 2) v = fmaxf(v, dpp_f<dpp::kXor1>(v));
    if constexpr (width >= 4) v = fmaxf(v, dpp_f<dpp::kXor2>(v));
    if constexpr (width >= 8) v = fmaxf(v, dpp_f<dpp::kHalfMirror>(v));
    if constexpr (width >= 16) v = fmaxf(v, dpp_f<dpp::kMirror>(v));
    if constexpr (width >= 32) {
        const uint2 r = swap_rows<16>(__float_as_uint(v));
        v = fmaxf(__uint_as_float(r.x), __uint_as_float(r.y));
    }
    if constexpr (width >= 64) {
        const uint2 r = swap_rows<32>(__float_as_uint(v));
        v = fmaxf(__uint_as_float(r.x), __uint_as_float(r.y));
    }
    return v;
}
__device__ __forceinline__ float wave_max(float v) { return group_max<64>(v); }
// Sum over groups of `width` consecutive lanes (a power of two <= 64).
template <int width>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int o = width / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

// Block-wide sum for blockDim.x a multiple of 64, at most 1024; every
// thread gets the result. scratch: 16 floats of LDS.
__device__ __forceinline__ float block_sum(float v, float* scratch) {
    v = wave_sum(v);
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int waves = blockDim.x / kWave;
    __syncthreads();
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    float s = lane < waves ? scratch[lane] : 0.0f;
    return wave_sum(s);
}
__device__ __forceinline__ float block_max(float v, float* scratch) {
    v = wave_max(v);
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int waves = blockDim.x / kWave;
    __syncthreads();
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    float s = lane < waves ? scratch[lane] : -__builtin_inff();
    return wave_max(s);
}

// ---------------------------------------------------------------- code generation

// threadIdx.x through an empty asm: what a function derives from it is
// computed where that function runs, not hoisted to a kernel's entry and
// kept live (or spilled) across the phases of a kernel that does several
// things in turn (the merge + o launch).
__device__ __forceinline__ uint32_t thread_index() {
    uint32_t t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

// Loads and stores through a pointer cast to the global address space at the
// access. Pointers a kernel reads from memory (not its arguments) are
// generic to the compiler, and accesses through them would be flat_load /
// flat_store, which the LDS counter also tracks: every workgroup barrier
// would then wait for the weight loads a kernel keeps in flight across it.
// HIP's vector types (uint4, float2, ...) are classes whose copies take a
// generic reference, so 8- and 16-byte values move as native vectors.
template <class T>
using global_t = __attribute__((address_space(1))) T;
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
template <class T>
__device__ __forceinline__ T ldg(const T* p) {
    if constexpr (sizeof(T) == 16) return __builtin_bit_cast(T, *(const global_t<u32x4>*)p);
    else if constexpr (sizeof(T) == 8) return __builtin_bit_cast(T, *(const global_t<u32x2>*)p);
    else return *(const global_t<T>*)p;
}
template <class T>
__device__ __forceinline__ void stg(T* p, T v) {
    if constexpr (sizeof(T) == 16) *(global_t<u32x4>*)p = __builtin_bit_cast(u32x4, v);
    else if constexpr (sizeof(T) == 8) *(global_t<u32x2>*)p = __builtin_bit_cast(u32x2, v);
    else *(global_t<T>*)p = v;
}

// A 32-bit value that no workgroup of the launch writes (the decode state's
// position, written by an earlier launch), read through the scalar unit:
// its wait counts scalar loads, so it does not also wait for (or hold up)
// the vector loads in flight around it.
__device__ __forceinline__ int32_t ld_scalar_i32(const int32_t* p) {
    return *reinterpret_cast<const __attribute__((address_space(4))) int32_t*>(reinterpret_cast<uintptr_t>(p));
}

// ---------------------------------------------------------------- coherent access

// Loads and stores of the values one workgroup of a launch produces for
// another (the merge + o launch's attention output). Each XCD has its own
// L2, which may hold a stale line of a buffer another XCD has since written;
// agent-scope relaxed atomics (sc1 accesses) are coherent across XCDs. With
// COH false these are plain accesses.
template <bool COH>
__device__ __forceinline__ uint32_t ld_u32(const uint32_t* p) {
    if constexpr (COH) return __hip_atomic_load((const global_t<uint32_t>*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else return ldg(p);
}
template <bool COH>
__device__ __forceinline__ uint64_t ld_u64(const uint64_t* p) {
    if constexpr (COH) return __hip_atomic_load((const global_t<uint64_t>*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else return ldg(p);
}
template <bool COH>
__device__ __forceinline__ float ld_f32(const float* p) {
    return __uint_as_float(ld_u32<COH>(reinterpret_cast<const uint32_t*>(p)));
}
template <bool COH>
__device__ __forceinline__ uint4 ld_u128(const uint4* p) {
    if constexpr (COH) {
        const uint64_t a = ld_u64<true>(reinterpret_cast<const uint64_t*>(p));
        const uint64_t b = ld_u64<true>(reinterpret_cast<const uint64_t*>(p) + 1);
        return make_uint4(static_cast<uint32_t>(a), static_cast<uint32_t>(a >> 32), static_cast<uint32_t>(b),
                          static_cast<uint32_t>(b >> 32));
    } else {
        return ldg(p);
    }
}
template <bool COH>
__device__ __forceinline__ float4 ld_f32x4(const float4* p) {
    const uint4 u = ld_u128<COH>(reinterpret_cast<const uint4*>(p));
    return make_float4(__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z), __uint_as_float(u.w));
}
template <bool COH>
__device__ __forceinline__ void st_u32(uint32_t* p, uint32_t v) {
    if constexpr (COH) __hip_atomic_store((global_t<uint32_t>*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else stg(p, v);
}
template <bool COH>
__device__ __forceinline__ void st_f32(float* p, float v) {
    st_u32<COH>(reinterpret_cast<uint32_t*>(p), __float_as_uint(v));
}
template <bool COH>
__device__ __forceinline__ void st_u8(uint8_t* p, uint8_t v) {
    if constexpr (COH) __hip_atomic_store((global_t<uint8_t>*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else stg(p, v);
}

// ---------------------------------------------------------------- int8 dot

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4(static_cast<int>(a), static_cast<int>(b), c, false);
}

// Sum of the 16 signed bytes of v.
__device__ __forceinline__ int byte_sum(uint4 v) {
    const uint32_t ones = 0x01010101u;
    return dot4(v.w, ones, dot4(v.z, ones, dot4(v.y, ones, dot4(v.x, ones, 0))));
}

// Activation quantization of one value given its block's inverse scale
// (shaders/quantize.comp:210-221): round half to even, clamp to +-127.
__device__ __forceinline__ int quant_code(float x, float inv) {
    return static_cast<int>(fminf(fmaxf(__builtin_rintf(x * inv), -127.0f), 127.0f));
}

// ---------------------------------------------------------------- q4_K headers

// Scale and offset of sub-blocks 2c and 2c+1 of a q4_K super-block whose
// 16-byte header is hdr (d, dmin, 12 bytes of 6-bit scales and mins),
// as the f32 values of the f16-rounded products f16(d * sc) and
// f16(-(dmin * m)) (src/io/gguf.cpp:123-131,603-617).
__device__ __forceinline__ void q4k_scales(uint4 hdr, uint32_t c, float& s0, float& o0, float& s1,
                                           float& o1) {
    const uint32_t shift = (c & 1u) * 16u;
    const uint32_t Y = (hdr.y >> shift) & 0xFFFFu;
    const uint32_t Z = (hdr.z >> shift) & 0xFFFFu;
    const uint32_t W = (hdr.w >> shift) & 0xFFFFu;
    uint32_t sc, mn;
    if (c < 2) {
        sc = Y & 0x3F3Fu;
        mn = Z & 0x3F3Fu;
    } else {
        sc = (W & 0x0F0Fu) | ((Y & 0xC0C0u) >> 2);
        mn = ((W >> 4) & 0x0F0Fu) | ((Z & 0xC0C0u) >> 2);
    }
    const float d = f16_bits_to_float(hdr.x & 0xFFFFu);
    const float dmin = f16_bits_to_float(hdr.x >> 16);
    s0 = round_to_f16(d * static_cast<float>(sc & 0xFFu));
    s1 = round_to_f16(d * static_cast<float>(sc >> 8));
    o0 = round_to_f16(-(dmin * static_cast<float>(mn & 0xFFu)));
    o1 = round_to_f16(-(dmin * static_cast<float>(mn >> 8)));
}

// Bit offset of value i % 8 within a QuantizedMatrix q4 word
// (shaders/include/halves.glsl:27).
__device__ __forceinline__ uint32_t q4_shift(uint32_t i) { return 8u * (i & 3u) + 4u * ((i >> 2) & 1u); }

// Value col of row `row` of a [rows, cols] weight matrix of `type` (the
// reference's dequantize.comp:37-48 and load_b of gemv.comp:80-92). Products
// and sums are rounded separately, never fused.
__device__ __forceinline__ float weight_value(uint32_t type, uint32_t scale_type, const void* values,
                                              const void* scales, uint64_t cols, uint64_t row,
                                              uint64_t col) {
#pragma clang fp contract(off)
    const uint64_t e = row * cols + col;
    const auto scale_at = [&](uint64_t i) -> float {
        return scale_type == 1 ? f16_bits_to_float(static_cast<const uint16_t*>(scales)[i])
                               : static_cast<const float*>(scales)[i];
    };
    switch (type) {
        case 0: return static_cast<const float*>(values)[e];
        case 1: return f16_bits_to_float(static_cast<const uint16_t*>(values)[e]);
        case 2: return bf16_bits_to_float(static_cast<const uint16_t*>(values)[e]);
        case 3: {
            const int8_t q = static_cast<const int8_t*>(values)[e];
            return static_cast<float>(q) * scale_at(e / 32);
        }
        case 4: {
            const uint32_t w = static_cast<const uint32_t*>(values)[e / 8];
            const float q = static_cast<float>(static_cast<int>((w >> q4_shift(static_cast<uint32_t>(e))) & 15u) - 8);
            return q * scale_at(e / 32);
        }
        case 5: {
            const uint32_t w = static_cast<const uint32_t*>(values)[e / 8];
            const float q = static_cast<float>((w >> q4_shift(static_cast<uint32_t>(e))) & 15u);
            return q * scale_at(2 * (e / 32)) + scale_at(2 * (e / 32) + 1);
        }
        case 6: {
            // q4_K: super-block sb of the row, sub-block j, position l.
            const uint64_t sb = col / 256, j = (col % 256) / 32, l = col % 32;
            const uint8_t* qs = static_cast<const uint8_t*>(values) + row * (cols / 2) + sb * 128 + 32 * (j / 2);
            const uint32_t code = (j % 2 == 0) ? (qs[l] & 15u) : (qs[l] >> 4);
            const uint4 hdr = static_cast<const uint4*>(scales)[row * (cols / 256) + sb];
            float s0, o0, s1, o1;
            q4k_scales(hdr, static_cast<uint32_t>(j / 2), s0, o0, s1, o1);
            const float s = (j % 2 == 0) ? s0 : s1, o = (j % 2 == 0) ? o0 : o1;
            return static_cast<float>(code) * s + o;
        }
        default: return 0.0f;
    }
}

}  // namespace vkml::dev
