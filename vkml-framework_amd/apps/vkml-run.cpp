// vkml-run -- prompt then greedy decode, as the reference's apps/vkml_run.cpp
// (flags :78-128, decode loop :282-298), over token ids (this build has no
// tokenizer: --tokens, not --prompt).
#include <algorithm>
#include <chrono>
#include <cstdio>
#include <numeric>
#include <optional>
#include <sstream>
#include <string>
#include <vector>

#include "vkml/llama.hpp"

namespace {

using Clock = std::chrono::steady_clock;
double seconds_since(Clock::time_point t) { return std::chrono::duration<double>(Clock::now() - t).count(); }

struct Args {
    std::string model, device;
    std::vector<std::int32_t> tokens;
    int generate = 16;
    std::int64_t context = 512;
    bool kv_f16 = false, no_dot = false, profile = false, ignore_eos = false, no_graphs = false, device_loop = false;
    std::optional<vkml::QuantType> quantize;
};

std::vector<std::int32_t> parse_tokens(const std::string& text) {
    std::vector<std::int32_t> t;
    std::stringstream in(text);
    std::string item;
    while (std::getline(in, item, ',')) t.push_back(std::stoi(item));
    return t;
}

bool parse(int argc, char** argv, Args& a) {
    for (int i = 1; i < argc; ++i) {
        const std::string f = argv[i];
        if (f == "--kv-f16") a.kv_f16 = true;
        else if (f == "--no-dot") a.no_dot = true;
        else if (f == "--profile") a.profile = true;
        else if (f == "--ignore-eos") a.ignore_eos = true;
        else if (f == "--no-graphs") a.no_graphs = true;
        else if (f == "--device-loop") a.device_loop = true;
        else if (f == "--q8") a.quantize = vkml::QuantType::q8_0;
        else if (f == "--q4") a.quantize = vkml::QuantType::q4_0;
        else if (i + 1 == argc) return false;
        else if (f == "--model") a.model = argv[++i];
        else if (f == "--tokens") a.tokens = parse_tokens(argv[++i]);
        else if (f == "--generate") a.generate = std::stoi(argv[++i]);
        else if (f == "--context") a.context = std::stoll(argv[++i]);
        else if (f == "--device") a.device = argv[++i];
        else return false;
    }
    return !a.model.empty() && !a.tokens.empty();
}

void print_profile(const char* title, const std::vector<vkml::KernelTime>& profile, double steps, double wall) {
    double total = 0;
    for (const auto& k : profile) total += k.milliseconds;
    std::printf("\n%s: GPU busy %.3f ms per step, wall clock %.3f ms per step\n", title, total / steps, wall * 1e3 / steps);
    std::printf("  %-28s %8s %12s %12s %7s\n", "kernel", "calls", "total ms", "ms/step", "share");
    for (const auto& k : profile) {
        std::printf("  %-28s %8llu %12.3f %12.4f %6.1f%%\n", k.name.c_str(), static_cast<unsigned long long>(k.calls), k.milliseconds,
                    k.milliseconds / steps, 100.0 * k.milliseconds / total);
    }
}

}  // namespace

int main(int argc, char** argv) {
    Args args;
    try {
        if (!parse(argc, argv, args)) {
            std::fprintf(stderr,
                         "usage: %s --model <file.gguf> --tokens <id,id,...> [--generate N] [--context N] [--kv-f16] [--no-dot] "
                         "[--q8 | --q4] [--profile] [--no-graphs] [--device-loop] [--ignore-eos] [--device <name>]\n",
                         argv[0]);
            return 2;
        }
    } catch (const std::exception& e) {
        std::fprintf(stderr, "bad argument: %s\n", e.what());
        return 2;
    }
    try {
        vkml::ContextOptions co;
        co.device_name = args.device;
        co.integer_dot_product = !args.no_dot;
        vkml::Context context{co};
        std::printf("device   %s (%s, %u CUs)\n", context.device_info().name.c_str(), context.device_info().arch.c_str(),
                    context.device_info().compute_units);
        auto start = Clock::now();
        vkml::LlamaOptions lo;
        lo.quantize = args.quantize;
        lo.kv_cache = args.kv_f16 ? vkml::DType::F16 : vkml::DType::F32;
        lo.use_graphs = !args.no_graphs;
        vkml::Llama model = vkml::Llama::load(context, args.model, args.context, lo);
        const vkml::LlamaConfig& c = model.config();
        std::printf("model    %lld layers, hidden %lld, %lld/%lld heads, vocab %lld (%.1f s to load)\n", (long long)c.num_layers,
                    (long long)c.hidden_size, (long long)c.num_heads, (long long)c.num_kv_heads, (long long)c.vocab_size, seconds_since(start));
        std::printf("kv cache %.1f MB for %lld positions\n", double(model.kv_cache_bytes()) / 1e6, (long long)model.context_length());

        if (args.profile) context.set_profiling(true);
        start = Clock::now();
        std::vector<float> logits = model.forward(args.tokens).to_vector<float>();
        const double prefill = seconds_since(start);
        if (args.profile) {
            print_profile("prompt", context.profile(), double(args.tokens.size()), prefill);
            context.reset_profile();
        }
        std::printf("prefill  %zu tokens in %.3f s (%.1f tokens/s)\n", args.tokens.size(), prefill, double(args.tokens.size()) / prefill);
        std::int32_t next = static_cast<std::int32_t>(std::max_element(logits.begin(), logits.end()) - logits.begin());
        std::vector<std::int32_t> generated;
        const int n = static_cast<int>(std::min<std::int64_t>(args.generate, model.context_length() - model.position()));
        start = Clock::now();
        if (args.device_loop && !args.profile) {
            // Every step's argmax stays on the device; the ids come back at the end.
            generated.push_back(next);
            const auto rest = model.generate_greedy(next, n - 1);
            generated.insert(generated.end(), rest.begin(), rest.end());
            if (n > 0) model.forward({&generated.back(), 1});
        } else {
            for (int i = 0; i < n; ++i) {
                if (!args.ignore_eos && std::find(c.eos_token_ids.begin(), c.eos_token_ids.end(), next) != c.eos_token_ids.end()) break;
                generated.push_back(next);
                next = vkml::argmax(model.forward({&next, 1})).to_vector<std::int32_t>()[0];
            }
        }
        const double decode = seconds_since(start);
        if (!generated.empty()) {
            if (args.profile) print_profile("generation", context.profile(), double(generated.size()), decode);
            std::printf("decode   %zu tokens in %.3f s (%.1f tokens/s)\n", generated.size(), decode, double(generated.size()) / decode);
            std::printf("generated");
            for (std::size_t i = 0; i < generated.size(); ++i) std::printf("%s%d", i ? "," : " ", generated[i]);
            std::printf("\n");
        }
        return 0;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "error: %s\n", e.what());
        return 1;
    }
}
