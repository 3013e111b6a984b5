#pragma once

#include <cstdint>
#include <random>
#include <span>
#include <unordered_map>
#include <utility>
#include <vector>

namespace vkml {

// How the next token is picked from a model's logits (reference:
// include/vkml/sampling.hpp:14-31).
struct SamplingOptions {
    float temperature = 0.0f;  // 0: always the most likely token (greedy)
    int top_k = 0;             // keep only the k most likely tokens; 0 keeps all
    float top_p = 1.0f;        // keep the fewest tokens whose probability sums to top_p
    std::uint64_t seed = 0;    // the same seed and logits give the same tokens
    // Tokens already seen get their logit divided by this (multiplied when
    // negative), once each, as transformers' repetition_penalty; 1 is off.
    float repetition_penalty = 1.0f;
    // Keep only tokens at least min_p times as likely as the most likely; 0 is off.
    float min_p = 0.0f;
    // As OpenAI's API, in [-2, 2]: a token's logit drops by frequency_penalty
    // for every time this sampler has picked it, and by presence_penalty once
    // if it has at all; 0 is off. The prompt does not count.
    float frequency_penalty = 0.0f;
    float presence_penalty = 0.0f;
};

// Picks tokens as transformers' generate does (reference: src/io/sampling.cpp:
// 17-139): the repetition penalty over the tokens seen so far and the
// frequency and presence penalties over those this sampler picked, then
// (sampling) logits over the temperature, cut to top_k, top_p and min_p,
// and a draw from the softmax of what remains, with std::mt19937_64 seeded
// by SamplingOptions::seed. Candidates of equal logit are ordered by token
// id (the reference leaves that order to std::partial_sort).
class Sampler {
public:
    explicit Sampler(SamplingOptions options);

    // previous: the tokens so far (prompt and reply), for the repetition penalty.
    std::int32_t sample(std::span<const float> logits, std::span<const std::int32_t> previous = {});

    // Whether sample() is the argmax of the logits as given (greedy without
    // penalties), which the device finds without reading the logits back.
    bool greedy() const noexcept;

    const SamplingOptions& options() const noexcept { return options_; }

private:
    std::int32_t pick(std::span<const float> logits);
    // Counts a picked token for the frequency and presence penalties.
    std::int32_t remember(std::int32_t id);

    SamplingOptions options_;
    std::mt19937_64 rng_;
    std::unordered_map<std::int32_t, int> picked_;  // times each token was picked, for the penalties
};

// A token's log probability under logits (their log-softmax, computed in
// double and rounded to float), and the `top` most likely tokens with
// theirs, most likely first, equal logits by ascending id (reference:
// src/io/sampling.cpp:141-164).
struct TokenLogprobs {
    float logprob = 0.0f;
    std::vector<std::pair<std::int32_t, float>> top;
};
TokenLogprobs token_logprobs(std::span<const float> logits, std::int32_t token, int top);

}  // namespace vkml
