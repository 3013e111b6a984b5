"""The request loop over vkml::Llama (vkml::Session, the reference's
ChatModel::generate, apps/generation.hpp:139-202) on the MI355X against the
CPU oracle: the oracle's model gives the logits and the oracle's sampler
picks from them, step by step as the reference's decode loop does; the
session must produce the same reply, stop at the same place, and leave the
same tokens in its cache, whether it samples on the host or takes greedy
steps on the device several at a time, and whether or not it reuses a
cached prefix."""
import os

import numpy as np
import pytest

import oracle as O
from vkml_amd import gguf, synth
from vkml_amd import llama as L

pytestmark = pytest.mark.gpu

STOP, LENGTH = L.Session.STOP, L.Session.LENGTH


@pytest.fixture(scope="module", autouse=True)
def threads():
    O.set_threads(min(16, os.cpu_count() or 1))


@pytest.fixture(scope="module")
def path(tmp_path_factory):
    spec = synth.ModelSpec("serve-q4k", 2, 256, 4, 2, 64, 512, 1000, 10000.0, max_positions=512,
                           matrix_type=gguf.Q4_K, embed_type=gguf.Q4_K, output_type=gguf.Q6_K)
    return synth.write_model(spec, str(tmp_path_factory.mktemp("m") / "serve.gguf"), seed=3)


def oracle_reply(model, cached, prompt, sampler, max_tokens, stop):
    """The reference's generate + decode loop on the oracle: returns (reply,
    finish, cached after)."""
    common = 0
    while common < min(len(cached), len(prompt)) and cached[common] == prompt[common]:
        common += 1
    common = min(common, len(prompt) - 1)
    model.rewind(common)
    cached = list(prompt)
    logits = model.forward(np.array(prompt[common:], np.int32))
    reply = []
    while max_tokens < 0 or len(reply) < max_tokens:
        if model.position >= model.context:
            return reply, LENGTH, cached
        nxt = sampler.sample(logits, cached)
        if nxt in stop:
            return reply, STOP, cached
        reply.append(nxt)
        logits = model.forward(np.array([nxt], np.int32))
        cached.append(nxt)
    return reply, LENGTH, cached


@pytest.mark.parametrize("opts", [dict(temperature=0.8, top_k=40, seed=5),
                                  dict(temperature=1.2, top_p=0.9, min_p=0.02, repetition_penalty=1.2, seed=17),
                                  dict(temperature=0.9, frequency_penalty=0.5, presence_penalty=0.3, seed=2)])
def test_sampled_replies_match_the_oracle(path, opts):
    ctx = 64
    gpu, ref = L.Llama(path, ctx, kv_f16=True), O.Model(path, ctx, kv_f16=True)
    session = L.Session(gpu)
    prompt = list(np.random.default_rng(1).integers(0, 1000, 10))
    reply, finish = session.generate(prompt, L.Sampler(**opts), 14)
    want, wfinish, wcached = oracle_reply(ref, [], prompt, O.Sampler(**opts), 14, [])
    assert list(reply) == want and finish == wfinish
    assert list(session.cached) == wcached and gpu.position == len(wcached)


@pytest.mark.parametrize("max_tokens,stop_at", [(5, None), (16, None), (17, None), (40, None), (-1, 19), (40, 1), (40, 16)])
def test_greedy_replies_stop_where_the_oracle_stops(path, max_tokens, stop_at):
    """Greedy steps run 16 to a host round trip: limits and stop tokens in
    and across those batches must cut the reply where the one-step loop
    does, and leave the model at the same position."""
    ctx = 80
    prompt = list(np.random.default_rng(2).integers(0, 1000, 12))
    ref = O.Model(path, ctx, kv_f16=True)
    stop = []
    if stop_at is not None:
        toks, _, _ = oracle_reply(ref, [], prompt, O.Sampler(), stop_at + 1, [])
        stop = [toks[stop_at]]
        assert stop[0] not in toks[:stop_at]
        ref.reset()
    want, wfinish, wcached = oracle_reply(ref, [], prompt, O.Sampler(), max_tokens, stop)
    gpu = L.Llama(path, ctx, kv_f16=True)
    session = L.Session(gpu, stop)
    reply, finish = session.generate(prompt, L.Sampler(), max_tokens)
    assert list(reply) == want and finish == wfinish
    assert list(session.cached) == wcached and gpu.position == len(wcached)
    if max_tokens < 0 and stop_at is None:
        assert gpu.position == ctx


def test_context_end_finishes_the_reply(path):
    ctx = 40
    prompt = list(np.random.default_rng(3).integers(0, 1000, 9))
    gpu = L.Llama(path, ctx, kv_f16=True)
    reply, finish = L.Session(gpu).generate(prompt, L.Sampler(), -1)
    ref = O.Model(path, ctx, kv_f16=True)
    want, wfinish, _ = oracle_reply(ref, [], prompt, O.Sampler(), -1, [])
    assert finish == LENGTH == wfinish and list(reply) == want and len(reply) == ctx - len(prompt)


@pytest.mark.parametrize("greedy", [True, False])
def test_a_second_request_reuses_the_common_prefix(path, greedy):
    """Request two shares a prefix with request one's prompt and reply: the
    session runs only what follows it (4 tokens, through gemv_dot's order;
    a fresh model would run all 20 through matmul_dot's, so its logits may
    differ in the last bits), and replies as the oracle does from the same
    cache."""
    ctx = 96
    opts = {} if greedy else dict(temperature=0.9, top_k=20, seed=4)
    rng = np.random.default_rng(4)
    p1 = list(rng.integers(0, 1000, 11))
    gpu = L.Llama(path, ctx, kv_f16=True)
    session = L.Session(gpu)
    r1, _ = session.generate(p1, L.Sampler(**opts), 9)
    p2 = p1 + list(r1[:5]) + list(rng.integers(0, 1000, 4))
    r2, f2 = session.generate(p2, L.Sampler(**opts), 9)
    assert gpu.position == len(p2) + len(r2)
    ref = O.Model(path, ctx, kv_f16=True)
    _, _, cached = oracle_reply(ref, [], p1, O.Sampler(**opts), 9, [])
    want, _, wcached = oracle_reply(ref, cached, p2, O.Sampler(**opts), 9, [])
    assert list(r2) == want and list(session.cached) == wcached


def oracle_reply_logprobs(model, prompt, sampler, max_tokens, top):
    """oracle_reply from an empty cache, with each reply token's
    token_logprobs under the step's logits (generate with logprobs,
    apps/generation.hpp:176-190)."""
    model.rewind(0)
    logits = model.forward(np.array(prompt, np.int32))
    cached, reply, rows = list(prompt), [], []
    while len(reply) < max_tokens and model.position < model.context:
        nxt = sampler.sample(logits, cached)
        reply.append(nxt)
        rows.append(O.token_logprobs(logits, nxt, top))
        logits = model.forward(np.array([nxt], np.int32))
        cached.append(nxt)
    return reply, rows


@pytest.mark.parametrize("opts", [dict(), dict(temperature=0.8, top_k=40, seed=5)])
def test_reply_logprobs_match_the_oracle(path, opts):
    """Each reply token's log probability and top alternatives, from the
    model's own logits (before sampling settings), bit for bit as the
    oracle's model and token_logprobs give them; a greedy sampler reads the
    logits back and still replies as on the device."""
    ctx, top, n = 64, 5, 12
    prompt = list(np.random.default_rng(6).integers(0, 1000, 10))
    gpu = L.Llama(path, ctx, kv_f16=True)
    session = L.Session(gpu)
    reply, finish, lp, ids, lps = session.generate_logprobs(prompt, L.Sampler(**opts), n, top)
    ref = O.Model(path, ctx, kv_f16=True)
    want, rows = oracle_reply_logprobs(ref, prompt, O.Sampler(**opts), n, top)
    assert list(reply) == want and finish == LENGTH
    for i, (wl, wi, wls) in enumerate(rows):
        assert np.float32(lp[i]).view(np.uint32) == np.float32(wl).view(np.uint32), i
        assert list(ids[i]) == list(wi) and np.array_equal(lps[i].view(np.uint32), wls.view(np.uint32)), i
    if not opts:
        plain, _ = L.Session(L.Llama(path, ctx, kv_f16=True)).generate(prompt, L.Sampler(), n)
        assert list(plain) == list(reply)


@pytest.mark.parametrize("length", [1, 9, 37])
def test_score_matches_the_oracle(path, length):
    """Session.score (ChatModel::score, apps/generation.hpp:104-131): each
    prompt token's log probability given the ones before from forward_all's
    rows, NaN for the first; the session then holds the prompt and a
    request extending it runs only the new tokens."""
    ctx, top = 64, 3
    prompt = list(np.random.default_rng(length).integers(0, 1000, length))
    gpu = L.Llama(path, ctx, kv_f16=True)
    session = L.Session(gpu)
    session.generate(list(np.random.default_rng(99).integers(0, 1000, 5)), L.Sampler(), 3)  # something cached first
    lp, ids, lps = session.score(prompt, top)
    assert np.isnan(lp[0]) and np.all(ids[0] == -1) and np.all(np.isnan(lps[0]))
    assert list(session.cached) == prompt and gpu.position == length
    ref = O.Model(path, ctx, kv_f16=True)
    rows = ref.forward_all(np.array(prompt, np.int32))
    for i in range(1, length):
        wl, wi, wls = O.token_logprobs(rows[i - 1], prompt[i], top)
        assert np.float32(lp[i]).view(np.uint32) == np.float32(wl).view(np.uint32), i
        assert list(ids[i]) == list(wi) and np.array_equal(lps[i].view(np.uint32), wls.view(np.uint32)), i
    reply, _ = session.generate(prompt + [5], L.Sampler(), 4)
    assert list(session.cached) == prompt + [5] + list(reply) and gpu.position == length + 1 + len(reply)
