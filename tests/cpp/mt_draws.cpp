// libstdc++'s std::mt19937_64 and uniform_real_distribution<double>, the
// generator and draw of the reference's Sampler, printed for the oracle's
// restatement to be checked against: for each seed argument, 1000 raw
// outputs, then 1000 draws of uniform_real_distribution(0, t) for t cycling
// over 1, 0.37 and 1e6 (a fresh engine of the same seed).
#include <cstdio>
#include <cstdlib>
#include <random>

int main(int argc, char** argv) {
    for (int a = 1; a < argc; ++a) {
        const unsigned long long seed = std::strtoull(argv[a], nullptr, 10);
        std::mt19937_64 raw(seed);
        for (int i = 0; i < 1000; ++i) std::printf("%llu\n", static_cast<unsigned long long>(raw()));
        std::mt19937_64 g(seed);
        const double totals[3] = {1.0, 0.37, 1e6};
        for (int i = 0; i < 1000; ++i) std::printf("%.17g\n", std::uniform_real_distribution<double>(0.0, totals[i % 3])(g));
    }
    return 0;
}
