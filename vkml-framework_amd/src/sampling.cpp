// sampling.cpp -- picking the next token from a step's logits on the host,
// with the semantics of the reference's Sampler (src/io/sampling.cpp:17-139)
// and its log probabilities (:141-164).
//
// Design. Candidates leave a binary max-heap over token ids one at a time,
// in the order (larger logit first, then smaller id) -- a total order, so no
// result depends on how ties are sorted. Building the heap is linear, and a
// request then orders only as many tokens as its cuts look at: top_k, the
// fewest whose mass reaches top_p, those within min_p of the first, or, with
// no cut, as many as the draw walks past. Which token comes out is fixed by
// the arithmetic, which is the reference's: a candidate's weight
// exp((l - max) / T) in double; the softmax's denominator summed in token
// order when no top_k applies, else (and after any cut) over the kept
// candidates in their order; one std::uniform_real_distribution<double>
// (0, total) draw from std::mt19937_64; then the kept weights subtracted in
// order until the draw drops below zero (the last kept one if rounding
// leaves it at or above zero).
#include "vkml/sampling.hpp"

#include <algorithm>
#include <cmath>
#include <string>
#include <unordered_set>

#include "vkml/error.hpp"

namespace vkml {

namespace {

void require(bool ok, const std::string& what, float value) {
    if (!ok) throw Error("Sampler: " + what + ", got " + std::to_string(value));
}

// The heap's "less": token a is ranked after token b.
struct RankedAfter {
    std::span<const float> logits;
    bool operator()(std::int32_t a, std::int32_t b) const {
        const float la = logits[std::size_t(a)], lb = logits[std::size_t(b)];
        return la < lb || (la == lb && a > b);
    }
};

// Token ids by descending logit, then ascending id, popped one at a time.
class Ranking {
public:
    explicit Ranking(std::span<const float> logits) : after_{logits}, heap_(logits.size()) {
        for (std::size_t i = 0; i < heap_.size(); ++i) heap_[i] = static_cast<std::int32_t>(i);
        std::make_heap(heap_.begin(), heap_.end(), after_);
    }
    bool empty() const noexcept { return heap_.empty(); }
    std::int32_t next() {
        std::pop_heap(heap_.begin(), heap_.end(), after_);
        const std::int32_t id = heap_.back();
        heap_.pop_back();
        return id;
    }

private:
    RankedAfter after_;
    std::vector<std::int32_t> heap_;
};

// max + log(sum exp(l - max)) in double, summed in token order: the log of
// the softmax's denominator.
double log_partition(std::span<const float> logits) {
    const double peak = *std::max_element(logits.begin(), logits.end());
    double sum = 0.0;
    for (const float l : logits) sum += std::exp(double(l) - peak);
    return peak + std::log(sum);
}

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
    const bool no_penalty = o.repetition_penalty == 1.0f && o.frequency_penalty == 0.0f && o.presence_penalty == 0.0f;
    return no_penalty && (o.temperature == 0.0f || o.top_k == 1);
}

std::int32_t Sampler::sample(std::span<const float> logits, std::span<const std::int32_t> previous) {
    if (logits.empty()) throw Error("Sampler: the logits are empty");
    const bool repeat = options_.repetition_penalty != 1.0f && !previous.empty();
    if (!repeat && picked_.empty()) return remember(pick(logits));
    // The penalties change a copy: the repetition penalty once for each
    // distinct token seen (a positive logit divided by it, a negative one
    // multiplied), then the frequency and presence penalties of the tokens
    // this sampler has picked.
    std::vector<float> adjusted(logits.begin(), logits.end());
    if (repeat) {
        std::unordered_set<std::int32_t> done;
        for (const std::int32_t id : previous) {
            if (id < 0 || std::size_t(id) >= adjusted.size() || !done.insert(id).second) continue;
            float& l = adjusted[std::size_t(id)];
            l = l < 0.0f ? l * options_.repetition_penalty : l / options_.repetition_penalty;
        }
    }
    for (const auto& [id, times] : picked_) {
        if (std::size_t(id) < adjusted.size()) adjusted[std::size_t(id)] -= float(times) * options_.frequency_penalty + options_.presence_penalty;
    }
    return remember(pick(adjusted));
}

std::int32_t Sampler::remember(std::int32_t id) {
    if (options_.frequency_penalty != 0.0f || options_.presence_penalty != 0.0f) ++picked_[id];
    return id;
}

std::int32_t Sampler::pick(std::span<const float> logits) {
    if (options_.temperature == 0.0f || options_.top_k == 1)
        return static_cast<std::int32_t>(std::max_element(logits.begin(), logits.end()) - logits.begin());

    const double peak = *std::max_element(logits.begin(), logits.end());
    const double t = options_.temperature;
    const auto weight = [&](std::int32_t id) { return std::exp((double(logits[std::size_t(id)]) - peak) / t); };
    const auto sum_of = [](const std::vector<double>& w) {
        double s = 0.0;
        for (const double x : w) s += x;
        return s;
    };
    Ranking ranking(logits);
    std::vector<std::int32_t> ids;  // the kept candidates, in rank order
    std::vector<double> w;          // and their weights
    const auto take = [&] {
        const std::int32_t id = ranking.next();
        ids.push_back(id);
        w.push_back(weight(id));
    };

    double total = 0.0;
    if (options_.top_k > 0) {
        while (ids.size() < std::size_t(options_.top_k) && !ranking.empty()) take();
        total = sum_of(w);
    } else {
        for (std::size_t i = 0; i < logits.size(); ++i) total += weight(static_cast<std::int32_t>(i));
    }
    const bool from_heap = options_.top_k == 0;  // candidates still come off the ranking on demand
    bool cut = options_.top_k > 0;
    if (options_.top_p < 1.0f) {
        // the fewest candidates whose mass reaches top_p of the total (at least one)
        const double target = double(options_.top_p) * total;
        double mass = 0.0;
        std::size_t m = 0;
        while (mass < target) {
            if (m == ids.size()) {
                if (!from_heap || ranking.empty()) break;
                take();
            }
            mass += w[m++];
        }
        m = std::max<std::size_t>(m, 1);
        if (from_heap && ids.empty()) take();
        ids.resize(m);
        w.resize(m);
        total = sum_of(w);
        cut = true;
    }
    if (options_.min_p > 0.0f) {
        // the candidates at least min_p times as likely as the first
        if (ids.empty()) take();
        const double floor = double(options_.min_p) * w[0];
        std::size_t m = 1;
        for (;; ++m) {
            if (m == ids.size()) {
                if (cut || ranking.empty()) break;
                take();
            }
            if (!(w[m] >= floor)) break;
        }
        ids.resize(m);
        w.resize(m);
        total = sum_of(w);
        cut = true;
    }
    double draw = std::uniform_real_distribution<double>(0.0, total)(rng_);
    for (std::size_t i = 0;; ++i) {
        if (i == ids.size()) {
            if (cut || ranking.empty()) return ids.back();
            take();
        }
        draw -= w[i];
        if (draw < 0.0) return ids[i];
    }
}

TokenLogprobs token_logprobs(std::span<const float> logits, std::int32_t token, int top) {
    if (token < 0 || std::size_t(token) >= logits.size())
        throw Error("token_logprobs: token " + std::to_string(token) + " is outside the logits");
    const double lz = log_partition(logits);
    const auto logprob = [&](std::int32_t id) { return static_cast<float>(double(logits[std::size_t(id)]) - lz); };
    TokenLogprobs out;
    out.logprob = logprob(token);
    Ranking ranking(logits);
    for (int i = 0; i < top && !ranking.empty(); ++i) {
        const std::int32_t id = ranking.next();
        out.top.emplace_back(id, logprob(id));
    }
    return out;
}

}  // namespace vkml
