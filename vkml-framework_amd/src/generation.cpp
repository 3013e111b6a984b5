// generation.cpp -- a request loop over vkml::Llama with KV-cache reuse
// (the reference's apps/generation.hpp:139-202).
#include "vkml/generation.hpp"

#include <algorithm>
#include <limits>
#include <string>

#include "vkml/error.hpp"
#include "vkml/ops.hpp"

namespace vkml {

namespace {

// Greedy steps run on the device per host round trip.
constexpr std::int64_t kGreedyBatch = 16;

}  // namespace

Session::Session(Llama& model, std::vector<std::int32_t> stop) : model_(&model), stop_(std::move(stop)) {}

bool Session::is_stop(std::int32_t id) const { return std::find(stop_.begin(), stop_.end(), id) != stop_.end(); }

Session::Finish Session::generate(std::span<const std::int32_t> prompt, Sampler& sampler, std::int64_t max_tokens,
                                  std::vector<std::int32_t>& reply, std::vector<TokenLogprobs>* logprobs, int top) {
    if (prompt.empty()) throw Error("Session::generate: the prompt is empty");
    // Only the tokens after the part the cache already holds run; at least
    // one, for the logits. The model may start over instead (a sliding
    // window's rings no longer holding that prefix).
    const auto differ = std::mismatch(cached_.begin(), cached_.end(), prompt.begin(), prompt.end());
    std::size_t common = std::size_t(differ.second - prompt.begin());
    common = std::min(common, prompt.size() - 1);
    common = std::size_t(model_->rewind(std::int64_t(common)));
    cached_.assign(prompt.begin(), prompt.end());
    try {
        return decode(model_->forward(prompt.subspan(common)), sampler, max_tokens, reply, logprobs, top);
    } catch (...) {
        cached_.clear();  // what the cache holds is unknown: start over next time
        throw;
    }
}

Session::Finish Session::decode(Tensor logits, Sampler& sampler, std::int64_t max_tokens, std::vector<std::int32_t>& reply,
                                std::vector<TokenLogprobs>* logprobs, int top) {
    reply.clear();
    if (logprobs) logprobs->clear();
    Llama& m = *model_;
    // Greedy steps stay on the device unless the logits are wanted anyway.
    const bool greedy = sampler.greedy() && !logprobs;
    std::vector<float> host;
    const auto pick = [&](const Tensor& l) {
        if (greedy) return argmax(l).to_vector<std::int32_t>()[0];
        host = l.to_vector<float>();
        return sampler.sample(host, cached_);
    };
    std::int32_t next = pick(logits);
    for (;;) {
        // Every picked token is run (its keys and values join the cache)
        // before the next is picked, as the reference's loop does.
        if (max_tokens >= 0 && std::int64_t(reply.size()) >= max_tokens) return Finish::length;
        if (m.position() >= m.context_length()) return Finish::length;
        if (is_stop(next)) return Finish::stop;
        reply.push_back(next);
        if (logprobs) logprobs->push_back(token_logprobs(host, next, top));
        if (!greedy) {
            logits = m.forward({&next, 1});
            cached_.push_back(next);
            next = pick(logits);
            continue;
        }
        // Greedy: run `next` and up to n - 1 of the tokens after it on the
        // device; the batch's picks go through the same checks, and the
        // model is rewound to the last token the loop would have run.
        std::int64_t n = std::min(kGreedyBatch, m.context_length() - m.position());
        if (max_tokens >= 0) n = std::min<std::int64_t>(n, max_tokens - std::int64_t(reply.size()) + 1);
        const std::vector<std::int32_t> picks = m.generate_greedy(next, n);
        cached_.push_back(next);
        for (std::int64_t i = 0; i + 1 < n; ++i) {
            const std::int32_t t = picks[std::size_t(i)];
            const bool full = max_tokens >= 0 && std::int64_t(reply.size()) >= max_tokens;
            if (full || is_stop(t)) {
                cached_.resize(std::size_t(m.rewind(std::int64_t(cached_.size()))));
                return full ? Finish::length : Finish::stop;
            }
            reply.push_back(t);
            cached_.push_back(t);
        }
        next = picks.back();
    }
}

std::vector<TokenLogprobs> Session::score(std::span<const std::int32_t> prompt, int top) {
    if (prompt.empty()) throw Error("Session::score: the prompt is empty");
    Llama& m = *model_;
    if (std::int64_t(prompt.size()) > m.context_length()) {
        throw Error("Session::score: a prompt of " + std::to_string(prompt.size()) + " tokens exceeds the context length of " +
                    std::to_string(m.context_length()));
    }
    m.reset();
    cached_.clear();
    std::vector<TokenLogprobs> out;
    out.reserve(prompt.size());
    out.push_back(TokenLogprobs{std::numeric_limits<float>::quiet_NaN(), {}});
    // Row r of a piece's logits scores the token after it.
    const std::size_t vocab = std::size_t(m.config().vocab_size);
    const std::size_t rows = std::max<std::size_t>(1, (std::size_t{128} << 20) / (4 * vocab));
    for (std::size_t begin = 0; begin < prompt.size(); begin += rows) {
        const std::size_t n = std::min(rows, prompt.size() - begin);
        const std::vector<float> logits = m.forward_all(prompt.subspan(begin, n)).to_vector<float>();
        for (std::size_t r = 0; r < n && begin + r + 1 < prompt.size(); ++r)
            out.push_back(token_logprobs({logits.data() + r * vocab, vocab}, prompt[begin + r + 1], top));
    }
    cached_.assign(prompt.begin(), prompt.end());
    return out;
}

}  // namespace vkml
