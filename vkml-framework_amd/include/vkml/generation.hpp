#pragma once

#include <cstdint>
#include <span>
#include <vector>

#include "vkml/llama.hpp"
#include "vkml/sampling.hpp"

namespace vkml {

// A model and the tokens its KV cache holds, serving one request after
// another as the reference's ChatModel does (apps/generation.hpp:35-202,
// without its tokenizer and chat template, which are out of this build's
// scope): each request's prompt reuses the cache of its longest common
// prefix with what the cache holds (through Llama::rewind), and the reply
// is picked token by token until a stop token, max_tokens or the end of the
// context. One thread at a time (the reference's server holds a mutex
// around it, apps/server.hpp:257).
class Session {
public:
    enum class Finish { stop, length };

    // stop: the tokens that end a reply (the model's end-of-sequence ids).
    explicit Session(Llama& model, std::vector<std::int32_t> stop = {});

    // The reply to prompt (at least one token, fitting the context) of at
    // most max_tokens tokens (negative: no limit), without the stop token.
    // Greedy samplers take each argmax on the device, several steps per
    // host round trip (Llama::generate_greedy); others read each step's
    // logits back for Sampler::sample, whose repetition penalty counts the
    // prompt and the reply so far.
    //
    // With logprobs, each reply token's log probability under the model's
    // logits (before any sampling setting) and the `top` likeliest tokens
    // with theirs go there, one entry per reply token (ChatModel::generate
    // with logprobs, apps/generation.hpp:139-142,176-190): every step's
    // logits are then read back, greedy or not.
    Finish generate(std::span<const std::int32_t> prompt, Sampler& sampler, std::int64_t max_tokens,
                    std::vector<std::int32_t>& reply, std::vector<TokenLogprobs>* logprobs = nullptr, int top = 0);

    // Each of prompt's tokens with its log probability given the tokens
    // before it and the `top` likeliest alternatives there, from the logits
    // of every position (Llama::forward_all, in pieces of about 128 MB of
    // logits); the first token has none (NaN, no alternatives). Starts the
    // model over and leaves it holding the prompt, for generate to continue
    // (ChatModel::score, apps/generation.hpp:104-131).
    std::vector<TokenLogprobs> score(std::span<const std::int32_t> prompt, int top);

    // The tokens whose keys and values the model's cache holds, in order.
    const std::vector<std::int32_t>& cached() const noexcept { return cached_; }
    // Forgets them: the next request runs its whole prompt.
    void clear() noexcept { cached_.clear(); }

private:
    bool is_stop(std::int32_t id) const;
    Finish decode(Tensor logits, Sampler& sampler, std::int64_t max_tokens, std::vector<std::int32_t>& reply,
                  std::vector<TokenLogprobs>* logprobs, int top);

    Llama* model_;
    std::vector<std::int32_t> stop_;
    std::vector<std::int32_t> cached_;
};

}  // namespace vkml
