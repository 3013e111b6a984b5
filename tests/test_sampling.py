"""The token sampler on the CPU (host code of libvkml.so: no device needed).

The oracle's C restatement (oracle/oracle_sampling.c) is pinned first: its
64-bit Mersenne Twister against the C++ standard's known output and both its
generator and its uniform draws against libstdc++ itself (the reference's
Sampler uses std::mt19937_64 and std::uniform_real_distribution<double>,
src/io/sampling.cpp:17,133); its draws against the softmax they sample from.
Then the product's vkml::Sampler must pick the same tokens as the oracle on
the same logits, options and seed, call after call."""
import os
import subprocess

import numpy as np
import pytest

import oracle as O
from vkml_amd import llama as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_generator_10000th_output_is_the_standards():
    # [rand.predef]: the 10000th consecutive invocation of a default-
    # constructed mt19937_64 (seed 5489) produces 9981545732273789042.
    s = O.Sampler(seed=5489)
    for _ in range(9999):
        s.draw_u64()
    assert s.draw_u64() == 9981545732273789042


@pytest.fixture(scope="module")
def libstdcxx_draws(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("bin") / "mt_draws")
    subprocess.run(["g++", "-std=c++20", "-O1", os.path.join(ROOT, "tests", "cpp", "mt_draws.cpp"), "-o", exe], check=True)
    seeds = [0, 1, 12345, 2 ** 63 + 7]
    out = subprocess.run([exe] + [str(s) for s in seeds], capture_output=True, text=True, check=True).stdout.split()
    return seeds, out


def test_generator_and_draws_match_libstdcxx(libstdcxx_draws):
    seeds, out = libstdcxx_draws
    at = 0
    for seed in seeds:
        raw = O.Sampler(seed=seed)
        assert [raw.draw_u64() for _ in range(1000)] == [int(x) for x in out[at:at + 1000]]
        at += 1000
        g = O.Sampler(seed=seed)
        totals = (1.0, 0.37, 1e6)
        got = [g.draw_uniform(totals[i % 3]) for i in range(1000)]
        want = [float(x) for x in out[at:at + 1000]]
        assert got == want
        at += 1000


def test_draws_follow_the_softmax():
    # temperature 1, nothing cut: token i is drawn with probability
    # exp(l_i) / sum exp(l_j); 40000 draws, every count within 4.5 sigma.
    logits = np.array([2.0, 1.0, 0.5, 0.0, -1.0, -3.0, 1.5, 0.25], np.float32)
    p = np.exp(logits.astype(np.float64) - logits.max())
    p /= p.sum()
    s = O.Sampler(temperature=1.0, seed=3)
    n = 40000
    counts = np.bincount([s.sample(logits) for _ in range(n)], minlength=logits.size)
    sigma = np.sqrt(n * p * (1 - p))
    assert np.all(np.abs(counts - n * p) <= 4.5 * sigma), (counts, n * p)


def test_cuts_keep_the_right_candidates():
    logits = np.log(np.array([0.4, 0.25, 0.15, 0.1, 0.06, 0.04], np.float64)).astype(np.float32)
    for kw, allowed in (({"top_k": 3}, {0, 1, 2}), ({"top_p": 0.5}, {0, 1}), ({"top_p": 0.65}, {0, 1}),
                        ({"top_p": 0.66}, {0, 1, 2}), ({"min_p": 0.3}, {0, 1, 2}), ({"top_k": 1}, {0})):
        s = O.Sampler(temperature=1.0, seed=11, **kw)
        seen = {s.sample(logits) for _ in range(3000)}
        assert seen == allowed, (kw, seen)


def test_greedy_is_the_first_argmax():
    logits = np.array([0.5, 3.0, -1.0, 3.0], np.float32)
    assert O.Sampler().sample(logits) == 1
    assert L.Sampler().sample(logits) == 1
    assert L.Sampler(temperature=0.7, top_k=1, seed=9).sample(logits) == 1


OPTIONS = [
    dict(temperature=0.8),
    dict(temperature=0.8, top_k=40),
    dict(temperature=1.3, top_p=0.9),
    dict(temperature=0.5, top_p=0.5, min_p=0.05),
    dict(temperature=1.0, top_k=5, repetition_penalty=1.3),
    dict(temperature=0.9, top_p=0.95, frequency_penalty=0.7, presence_penalty=-0.4),
    dict(temperature=2.0, min_p=0.2, repetition_penalty=0.8, presence_penalty=1.5),
    dict(temperature=0.7, top_k=1000, top_p=0.8),
    dict(temperature=1.0, min_p=0.01),
    dict(temperature=0.6, top_k=200000),
    dict(temperature=1.1, top_p=1e-6),
    dict(temperature=0.9, top_k=30, min_p=0.1),
    dict(temperature=3.0),
]


@pytest.mark.parametrize("vocab", [50, 4096, 128256])
@pytest.mark.parametrize("opt", range(len(OPTIONS)))
def test_product_sampler_picks_the_oracles_tokens(vocab, opt):
    kw = OPTIONS[opt]
    rng = np.random.default_rng(vocab + opt)
    seed = int(rng.integers(0, 2 ** 63))
    a, b = L.Sampler(seed=seed, **kw), O.Sampler(seed=seed, **kw)
    previous = list(rng.integers(0, vocab, 20))
    got, want = [], []
    for step in range(12):
        logits = (rng.standard_normal(vocab) * 3).astype(np.float32)
        if step % 4 == 1:
            logits[:7] = logits[7]  # ties among candidates
        x, y = a.sample(logits, previous), b.sample(logits, previous)
        got.append(x)
        want.append(y)
        previous.append(y)
    assert got == want


def test_options_are_checked():
    for kw, msg in ((dict(temperature=-1.0), "temperature must be 0 or more"), (dict(top_p=0.0), "top_p must be in"),
                    (dict(top_k=-2), "top_k must be 0"), (dict(repetition_penalty=0.0), "repetition_penalty"),
                    (dict(min_p=1.5), "min_p must be in"), (dict(frequency_penalty=3.0), "frequency_penalty")):
        with pytest.raises(L.VkmlError, match=msg):
            L.Sampler(**kw)
    with pytest.raises(L.VkmlError, match="empty"):
        L.Sampler(temperature=1.0).sample(np.zeros(0, np.float32))


def test_oracle_logprobs_are_the_log_softmax():
    """The oracle's token_logprobs (the reference's, sampling.cpp:141-164)
    against float64 log-softmax (scipy), and exact on equal logits."""
    from scipy.special import log_softmax
    rng = np.random.default_rng(4)
    for vocab in (7, 1000, 32768):
        logits = (rng.standard_normal(vocab) * 4).astype(np.float32)
        want = log_softmax(logits.astype(np.float64))
        tok = int(rng.integers(0, vocab))
        lp, ids, lps = O.token_logprobs(logits, tok, 5)
        assert abs(lp - want[tok]) <= 1e-6 * (1 + abs(want[tok]))
        order = np.lexsort((np.arange(vocab), -logits))[:5]
        assert list(ids) == list(order)
        assert np.allclose(lps, want[order], rtol=1e-6, atol=1e-6)
    flat = np.zeros(10, np.float32)
    lp, ids, lps = O.token_logprobs(flat, 3, 4)
    assert lp == np.float32(-np.log(10.0)) and list(ids) == [0, 1, 2, 3]


@pytest.mark.parametrize("vocab", [3, 4096, 128256])
def test_product_logprobs_equal_the_oracles(vocab):
    rng = np.random.default_rng(vocab)
    for rep in range(5):
        logits = (rng.standard_normal(vocab) * 5).astype(np.float32)
        if rep == 2:
            logits[: min(vocab, 9)] = logits.max()  # ties at the top: by ascending id
        tok = int(rng.integers(0, vocab))
        top = min(8, vocab + 2)
        got = L.token_logprobs(logits, tok, top)
        want = O.token_logprobs(logits, tok, top)
        assert np.float32(got[0]).view(np.uint32) == np.float32(want[0]).view(np.uint32)
        k = min(top, vocab)
        assert list(got[1][:k]) == list(want[1])
        assert np.array_equal(got[2][:k].view(np.uint32), want[2].view(np.uint32))
        assert all(i == -1 for i in got[1][k:]) and np.all(np.isnan(got[2][k:]))
    with pytest.raises(L.VkmlError, match="outside the logits"):
        L.token_logprobs(np.zeros(4, np.float32), 4, 1)
