// sampling.cpp -- the host-side token sampler (the reference's
// src/io/sampling.cpp:17-164). The logits of a sampled step are read back
// from the device (the greedy case never needs them: the device argmax
// does); the picking is a few hundred microseconds of host work per token.
#include "vkml/sampling.hpp"

#include <algorithm>
#include <cmath>
#include <numeric>
#include <string>
#include <unordered_set>

#include "vkml/error.hpp"

namespace vkml {

namespace {

void require(bool ok, const std::string& what, float value) {
    if (!ok) throw Error("Sampler: " + what + ", got " + std::to_string(value));
}

// Descending logit, then ascending id: a total order, so the candidates
// (and hence the draws) do not depend on the sort's handling of ties.
struct ByLogit {
    std::span<const float> logits;
    bool operator()(std::int32_t a, std::int32_t b) const {
        const float la = logits[std::size_t(a)], lb = logits[std::size_t(b)];
        return la > lb || (la == lb && a < b);
    }
};

}  // namespace

Sampler::Sampler(SamplingOptions options) : options_(options), rng_(options.seed) {
    require(options.temperature >= 0.0f, "temperature must be 0 or more", options.temperature);
    require(options.top_p > 0.0f && options.top_p <= 1.0f, "top_p must be in (0, 1]", options.top_p);
    require(options.top_k >= 0, "top_k must be 0 (off) or more", float(options.top_k));
    require(options.repetition_penalty > 0.0f, "repetition_penalty must be more than 0", options.repetition_penalty);
    require(options.min_p >= 0.0f && options.min_p <= 1.0f, "min_p must be in [0, 1]", options.min_p);
    require(std::abs(options.frequency_penalty) <= 2.0f, "frequency_penalty must be in [-2, 2]", options.frequency_penalty);
    require(std::abs(options.presence_penalty) <= 2.0f, "presence_penalty must be in [-2, 2]", options.presence_penalty);
}

bool Sampler::greedy() const noexcept {
    const SamplingOptions& o = options_;
    return (o.temperature == 0.0f || o.top_k == 1) && o.repetition_penalty == 1.0f && o.frequency_penalty == 0.0f &&
           o.presence_penalty == 0.0f;
}

std::int32_t Sampler::sample(std::span<const float> logits, std::span<const std::int32_t> previous) {
    if (logits.empty()) throw Error("Sampler: the logits are empty");
    std::vector<float> adjusted;
    const auto own = [&] {
        if (adjusted.empty()) adjusted.assign(logits.begin(), logits.end());
    };
    // The repetition penalty: each distinct token seen, once.
    if (options_.repetition_penalty != 1.0f && !previous.empty()) {
        own();
        std::unordered_set<std::int32_t> seen;
        for (const std::int32_t id : previous) {
            if (id < 0 || std::size_t(id) >= adjusted.size() || !seen.insert(id).second) continue;
            float& l = adjusted[std::size_t(id)];
            l = l < 0.0f ? l * options_.repetition_penalty : l / options_.repetition_penalty;
        }
    }
    // The frequency and presence penalties of the tokens this sampler picked.
    if (!picked_.empty()) {
        own();
        for (const auto& [id, count] : picked_) {
            if (std::size_t(id) < adjusted.size())
                adjusted[std::size_t(id)] -= float(count) * options_.frequency_penalty + options_.presence_penalty;
        }
    }
    const std::int32_t id = pick(adjusted.empty() ? logits : std::span<const float>(adjusted));
    if (options_.frequency_penalty != 0.0f || options_.presence_penalty != 0.0f) ++picked_[id];
    return id;
}

std::int32_t Sampler::pick(std::span<const float> logits) {
    const std::size_t n = logits.size();
    if (options_.temperature == 0.0f || options_.top_k == 1)
        return static_cast<std::int32_t>(std::max_element(logits.begin(), logits.end()) - logits.begin());

    const double top = *std::max_element(logits.begin(), logits.end());
    const double temperature = options_.temperature;
    const auto weight = [&](std::int32_t id) { return std::exp((double(logits[std::size_t(id)]) - top) / temperature); };
    // Without top_k, the weights of every token (the softmax's denominator).
    double everything = 0.0;
    if (options_.top_k == 0)
        for (std::size_t i = 0; i < n; ++i) everything += weight(static_cast<std::int32_t>(i));

    // The candidates, most likely first: top_k of them, or without top_k
    // for top_p only as many as reach top_p of the total (256, then four
    // times as many until they do), or all.
    std::vector<std::int32_t> order(n);
    std::iota(order.begin(), order.end(), 0);
    const bool grow = options_.top_k == 0 && options_.top_p < 1.0f;
    std::size_t keep = options_.top_k > 0 ? std::size_t(options_.top_k) : grow ? 256 : n;
    for (;;) {
        keep = std::min(keep, n);
        std::partial_sort(order.begin(), order.begin() + std::ptrdiff_t(keep), order.end(), ByLogit{logits});
        if (!grow || keep == n) break;
        double mass = 0.0;
        for (std::size_t i = 0; i < keep; ++i) mass += weight(order[i]);
        if (mass >= options_.top_p * everything) break;
        keep *= 4;
    }
    order.resize(keep);

    std::vector<double> p(keep);
    for (std::size_t i = 0; i < keep; ++i) p[i] = weight(order[i]);
    double total = options_.top_k > 0 ? std::accumulate(p.begin(), p.end(), 0.0) : everything;
    if (options_.top_p < 1.0f) {  // the fewest candidates whose mass reaches top_p (at least one)
        double cumulative = 0.0;
        std::size_t m = 0;
        while (m < p.size() && cumulative < options_.top_p * total) cumulative += p[m++];
        p.resize(std::max<std::size_t>(m, 1));
        total = std::accumulate(p.begin(), p.end(), 0.0);
    }
    if (options_.min_p > 0.0f) {  // at least min_p times as likely as the first
        std::size_t m = 1;
        while (m < p.size() && p[m] >= options_.min_p * p[0]) ++m;
        p.resize(m);
        total = std::accumulate(p.begin(), p.end(), 0.0);
    }
    double draw = std::uniform_real_distribution<double>(0.0, total)(rng_);
    for (std::size_t i = 0; i < p.size(); ++i) {
        draw -= p[i];
        if (draw < 0.0) return order[i];
    }
    return order[p.size() - 1];  // rounding left the draw at the very end
}

TokenLogprobs token_logprobs(std::span<const float> logits, std::int32_t token, int top) {
    if (token < 0 || std::size_t(token) >= logits.size())
        throw Error("token_logprobs: token " + std::to_string(token) + " is outside the logits");
    const double peak = *std::max_element(logits.begin(), logits.end());
    double sum = 0.0;
    for (const float l : logits) sum += std::exp(double(l) - peak);
    const double log_total = peak + std::log(sum);
    const auto logprob = [&](std::int32_t id) { return float(double(logits[std::size_t(id)]) - log_total); };
    TokenLogprobs out;
    out.logprob = logprob(token);
    std::vector<std::int32_t> order(logits.size());
    std::iota(order.begin(), order.end(), 0);
    const std::size_t k = std::min<std::size_t>(std::size_t(std::max(top, 0)), order.size());
    std::partial_sort(order.begin(), order.begin() + std::ptrdiff_t(k), order.end(), ByLogit{logits});
    for (std::size_t i = 0; i < k; ++i) out.top.emplace_back(order[i], logprob(order[i]));
    return out;
}

}  // namespace vkml
