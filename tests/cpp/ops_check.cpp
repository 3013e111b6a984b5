// A check program for the C++ ops API on the GPU (links libvkml.so):
// matmul_transposed of one f32 row, whose Q8_0 is computed inside the GEMV
// (one launch), against the same row stacked twice, which takes the
// separate activation quantize and the rows gemv_dot. Both are the
// reference's int8 product (matmul.cpp:225-259), so every output row must
// be the same bits. Prints one line per case: "ok" or "MISMATCH", then the
// microseconds a call of each form takes (output allocation included).
#include <chrono>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

#include "vkml/context.hpp"
#include "vkml/ops.hpp"
#include "vkml/tensor.hpp"

namespace {

double micros_per_call(vkml::Context& ctx, const vkml::Tensor& a, const vkml::QuantizedMatrix& m, int calls) {
    vkml::Tensor keep = vkml::matmul_transposed(a, m);
    ctx.synchronize();
    const auto t0 = std::chrono::steady_clock::now();
    for (int i = 0; i < calls; ++i) keep = vkml::matmul_transposed(a, m);
    ctx.synchronize();
    return std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count() / calls;
}

}  // namespace

int main() {
    vkml::Context ctx;
    std::mt19937 gen(7);
    std::normal_distribution<float> normal;
    int mismatches = 0;
    const char* names[] = {"q8_0", "q4_0", "q4_1"};
    for (const std::int64_t k : {4096, 2048, 96}) {
        for (int q = 0; q < 3; ++q) {
            const std::int64_t n = 4096;
            std::vector<float> w(static_cast<std::size_t>(n * k)), a(static_cast<std::size_t>(2 * k));
            for (float& v : w) v = normal(gen) * 0.05f;
            for (std::int64_t i = 0; i < k; ++i) a[static_cast<std::size_t>(i)] = a[static_cast<std::size_t>(k + i)] = normal(gen);
            const vkml::Tensor tw = vkml::Tensor::from_data<float>(ctx, w, {n, k});
            const vkml::QuantizedMatrix m = q == 0 ? vkml::quantize_q8(tw) : q == 1 ? vkml::quantize_q4(tw) : vkml::quantize_q4_1(tw);
            const vkml::Tensor one = vkml::Tensor::from_data<float>(ctx, std::span<const float>(a).first(static_cast<std::size_t>(k)), {1, k});
            const vkml::Tensor two = vkml::Tensor::from_data<float>(ctx, a, {2, k});
            const std::vector<float> r1 = vkml::matmul_transposed(one, m).to_vector<float>();
            const std::vector<float> r2 = vkml::matmul_transposed(two, m).to_vector<float>();
            const bool same = std::memcmp(r1.data(), r2.data(), static_cast<std::size_t>(n) * 4) == 0 &&
                              std::memcmp(r2.data(), r2.data() + n, static_cast<std::size_t>(n) * 4) == 0;
            mismatches += same ? 0 : 1;
            std::printf("%s %s k=%lld one_row_us=%.2f two_rows_us=%.2f\n", same ? "ok" : "MISMATCH", names[q],
                        static_cast<long long>(k), micros_per_call(ctx, one, m, 200), micros_per_call(ctx, two, m, 200));
        }
    }
    return mismatches ? 1 : 0;
}
