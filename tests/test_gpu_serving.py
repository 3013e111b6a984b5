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
