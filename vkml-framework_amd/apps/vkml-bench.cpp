// vkml-bench -- quantized matrix-product microbenchmark (the reference's
// apps/vkml_bench.cpp: result checks against the "quarters" closed form and
// cache-defeating weight copies, :119-151,198-216; its m sweep and prefill
// cases, :51-85), at the shapes of a Mistral-7B-shaped layer in q8_0 and q4_K.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "vkml/ops.hpp"
#include "vkml_hip.h"

namespace {

struct Case {
    const char* name;
    std::int64_t rows, cols;
    std::int64_t m = 1;  // activation rows: 1 decodes, more are a prompt's
};

// Every weight exactly 0.25: q8_0 codes 127 with scale 0.25/127 would not be
// exact, so use code 1 and scale 0.25 (f16 0x3400); q4_K with d = 1/64,
// sc = 16 (d*sc = 0.25), dmin = 0, codes 1.
void quarters(bool q4k, std::int64_t rows, std::int64_t cols, std::vector<std::uint8_t>& values, std::vector<std::uint8_t>& scales) {
    if (!q4k) {
        values.assign(std::size_t(rows * cols), 1);
        scales.resize(std::size_t(rows * cols / 32) * 2);
        for (std::size_t i = 0; i < scales.size(); i += 2) {
            scales[i] = 0x00;
            scales[i + 1] = 0x34;
        }
        return;
    }
    values.assign(std::size_t(rows * cols / 2), 0x11);  // every code 1
    scales.assign(std::size_t(rows * cols / 256) * 16, 0);
    for (std::size_t b = 0; b < scales.size(); b += 16) {
        scales[b + 1] = 0x24;  // d = f16 1/64, dmin = 0
        // 12 scale bytes q[0..11]: sub-blocks 0-3 take sc = q[j] & 63 = 16;
        // 4-7 take (q[j+4] & 15) | (q[j-4] >> 6) << 4 = 16; every min is 0.
        for (int j = 0; j < 4; ++j) scales[b + 4 + j] = 16 | (1 << 6);
    }
}

}  // namespace

int main(int argc, char** argv) {
    int runs = argc > 1 ? std::atoi(argv[1]) : 50;
    if (vkml_init(nullptr) != VKML_OK) {
        std::fprintf(stderr, "error: %s\n", vkml_last_error());
        return 1;
    }
    // Decode shapes (gemv_dot, bound by HBM), then the reference's m sweep and
    // prefill shapes (gemv_dot up to 8 rows, matmul_dot on the matrix cores
    // beyond, bound by arithmetic: reported in TOP/s).
    const Case cases[] = {{"q/o 4096x4096", 4096, 4096},          {"gate|up 14336x4096", 14336, 4096},
                          {"down 4096x14336", 4096, 14336},       {"lm_head 32768x4096", 32768, 4096},
                          {"m=8 gate|up", 14336, 4096, 8},        {"m=64 gate|up", 14336, 4096, 64},
                          {"prefill q/o m=128", 4096, 4096, 128}, {"prefill gate|up m=128", 14336, 4096, 128},
                          {"prefill gate|up m=512", 14336, 4096, 512}};
    std::printf("%-24s %-6s %10s %10s %12s %8s\n", "shape", "format", "best us", "median us", "GB/s | TOP/s", "check");
    for (bool q4k : {false, true}) {
        for (const Case& c : cases) {
            std::vector<std::uint8_t> values, scales;
            quarters(q4k, c.rows, c.cols, values, scales);
            const double bytes = double(values.size() + scales.size());
            // Enough copies to pass 512 MB, so no run reads from cache.
            const int copies = int(std::clamp(512e6 / bytes, 1.0, 64.0));
            std::vector<void*> dv(copies), ds(copies);
            for (int i = 0; i < copies; ++i) {
                vkml_malloc(values.size(), &dv[i]);
                vkml_malloc(scales.size(), &ds[i]);
                vkml_memcpy_h2d(dv[i], values.data(), values.size());
                vkml_memcpy_h2d(ds[i], scales.data(), scales.size());
            }
            std::vector<std::int8_t> aq(std::size_t(c.m * c.cols), 1);
            std::vector<float> as(std::size_t(c.m * c.cols / 32), 1.0f);
            void *da, *das, *dout;
            vkml_malloc(aq.size(), &da);
            vkml_malloc(as.size() * 4, &das);
            vkml_malloc(std::size_t(c.m * c.rows) * 4, &dout);
            vkml_memcpy_h2d(da, aq.data(), aq.size());
            vkml_memcpy_h2d(das, as.data(), as.size() * 4);
            const vkml_gemv_dot_params p{std::uint32_t(c.m), std::uint32_t(c.rows), std::uint32_t(c.cols),
                                         q4k ? std::uint32_t(VKML_Q4_K) : std::uint32_t(VKML_Q8_0), VKML_F16};
            const auto product = c.m <= 8 ? vkml_gemv_dot : vkml_matmul_dot;
            std::vector<double> times;
            for (int r = 0; r < runs + 3; ++r) {
                vkml_synchronize();
                const auto t0 = std::chrono::steady_clock::now();
                if (product(&p, da, dv[r % copies], static_cast<float*>(dout), ds[r % copies], static_cast<const float*>(das)) != VKML_OK) {
                    std::fprintf(stderr, "error: %s\n", vkml_last_error());
                    return 1;
                }
                vkml_synchronize();
                if (r >= 3) times.push_back(std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count());
            }
            std::vector<float> out(std::size_t(c.m * c.rows));
            vkml_memcpy_d2h(out.data(), dout, out.size() * 4);
            const float want = 0.25f * float(c.cols);
            const bool ok = std::all_of(out.begin(), out.end(), [&](float v) { return v == want; });
            std::sort(times.begin(), times.end());
            const double best = times.front(), median = times[times.size() / 2];
            // decode: bytes of weights a microsecond; a prompt: int8 operations
            const double rate = c.m == 1 ? bytes / median / 1e3 : 2.0 * double(c.m * c.rows * c.cols) / median / 1e6;
            std::printf("%-24s %-6s %10.2f %10.2f %12.1f %8s\n", c.name, q4k ? "q4_K" : "q8_0", best, median, rate, ok ? "ok" : "WRONG");
            for (int i = 0; i < copies; ++i) {
                vkml_free(dv[i]);
                vkml_free(ds[i]);
            }
            vkml_free(da);
            vkml_free(das);
            vkml_free(dout);
        }
    }
    vkml_shutdown();
    return 0;
}
