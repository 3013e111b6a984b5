"""Sliding-window attention over ring caches on the MI355X, against the CPU
oracle's restatement of the reference's detail::sliding_attention
(attention.cpp:229-294) and of its Llama ring bookkeeping (llama.cpp:
236-241,273-285,356-364).

Kernel level: the reference's own ring test (tests/test_kv_cache.cpp:
215-266) with this build's kernels composed as ring_attention composes
them -- keys appended to a NaN-poisoned ring, one query through the fused
decode kernel, more through scores, the ring-masked softmax and probs . v
-- bit for bit with the oracle. Model level: a llama file with a sliding
window whose rings wrap many times in the prompt and in decoding, and
rewinds inside and past what the rings still hold."""
import math
import os

import numpy as np
import pytest

import oracle as O
from vkml_amd import gguf, synth
from vkml_amd import hip as H
from vkml_amd.llama import Llama

pytestmark = pytest.mark.gpu

MAX_SCORE_BYTES = 64 << 20


@pytest.fixture(scope="module", autouse=True)
def setup():
    H.init()
    O.set_threads(min(16, os.cpu_count() or 1))


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def sliding_rows(heads, t, q0, start, ring, window):
    first = start + q0
    rows = max(ring - window + 1, ring - first)
    keys = min(first + rows, ring)
    rows = min(rows, max(1, MAX_SCORE_BYTES // (heads * keys * 4)))
    if rows >= 64:
        rows -= rows % 64
    return min(rows, t - q0)


def gpu_sliding(q, k, v, k_ring, v_ring, start, window, softcap, kv_type):
    """detail::sliding_attention through the C ABI: q [heads, t, hd] f32; k,
    v [kv_heads, t, hd] in the cache type; k_ring / v_ring device buffers."""
    heads, t, hd = q.shape
    kvh = k.shape[0]
    ring = k_ring.nbytes // (kvh * hd * (2 if kv_type == H.F16 else 4))
    group = heads // kvh
    words = hd * (2 if kv_type == H.F16 else 4) // 4
    dk, dv = H.to_device(k), H.to_device(v)
    out = np.empty((heads, t, hd), np.float32)
    q0 = 0
    while q0 < t:
        rows = sliding_rows(heads, t, q0, start, ring, window)
        first, end = start + q0, start + q0 + rows
        at = first % ring
        head = min(rows, ring - at)
        for src, dst in ((dk, k_ring), (dv, v_ring)):
            for r_src, r_dst, n in ((q0, at, head), (q0 + head, 0, rows - head)):
                if n:
                    H.call("vkml_copy_rows", H.CopyRowsParams(kvh * n * words, n * words, t * words, r_src * words, ring * words,
                                                              r_dst * words), src.p, dst.p)
        qc = H.to_device(np.ascontiguousarray(q[:, q0:q0 + rows]))
        block = H.empty(heads * rows * hd * 4)
        if rows == 1:
            kv_start = max(0, end - window)
            chunks = (end - kv_start + 127) // 128
            prm = H.AttendParams(kv_start, end, ring, heads, kvh, hd, kv_type, chunks, 1.0 / math.sqrt(hd), softcap)
            part, stats = H.empty(heads * chunks * hd * 4), H.empty(heads * chunks * 8)
            H.call("vkml_attend", prm, qc.p, k_ring.p, v_ring.p, part.p, stats.p, None)
            H.call("vkml_attend_merge", prm, part.p, stats.p, block.p, None, None)
        else:
            keys = min(end, ring)
            scores, probs = H.empty(heads * rows * keys * 4), H.empty(heads * rows * keys * 4)
            if rows <= 8:
                H.call("vkml_gemv", H.GemvParams(rows, keys, hd, kv_type, H.F16, ring * hd, group, heads), qc.p, k_ring.p, scores.p, None)
            else:
                H.call("vkml_matmul", H.MatmulParams(rows, keys, hd, ring * hd, group, heads, 1, kv_type, H.F32), qc.p, k_ring.p,
                       scores.p, None)
            H.call("vkml_softmax", H.SoftmaxParams(heads * rows, keys, 1.0 / math.sqrt(hd), 1, rows, first, window, softcap, ring),
                   scores.p, probs.p)
            H.call("vkml_matmul", H.MatmulParams(rows, hd, keys, ring * hd, group, heads, 0, kv_type, H.F32), probs.p, v_ring.p,
                   block.p, None)
        out[:, q0:q0 + rows] = block.download(np.float32, (heads, rows, hd))
        q0 += rows
    return out


@pytest.mark.parametrize("hd", [64, 128, 256])
@pytest.mark.parametrize("kv_type", [H.F32, H.F16])
@pytest.mark.parametrize("softcap", [0.0, 0.5])
def test_ring_attention_matches_the_oracle_with_nan_rows(hd, kv_type, softcap):
    heads, kvh, total, window, ring = 4, 2, 31, 5, 8
    steps = [7, 1, 1, 1, 3, 10, 1, 2, 4, 1]
    rng = np.random.default_rng(71 + hd)
    q = rng.standard_normal((heads, total, hd)).astype(np.float32)
    k = rng.standard_normal((kvh, total, hd)).astype(np.float32)
    v = rng.standard_normal((kvh, total, hd)).astype(np.float32)
    if kv_type == H.F16:
        k, v = k.astype(np.float16).view(np.uint16), v.astype(np.float16).view(np.uint16)
        poison = np.full((kvh, ring, hd), 0x7E00, np.uint16)
    else:
        poison = np.full((kvh, ring, hd), np.nan, np.float32)
    g_k, g_v = H.to_device(poison), H.to_device(poison)
    o_k, o_v = poison.copy(), poison.copy()
    start = 0
    for n in steps:
        print(f"ring case hd={hd} kv_type={kv_type} softcap={softcap} start={start} n={n}", flush=True)
        got = gpu_sliding(q[:, start:start + n], np.ascontiguousarray(k[:, start:start + n]), np.ascontiguousarray(v[:, start:start + n]),
                          g_k, g_v, start, window, softcap, kv_type)
        want = O.attention_sliding(q[:, start:start + n], k[:, start:start + n], v[:, start:start + n], o_k, o_v, start, window, softcap)
        if softcap:
            # tanh is the device's and the host's libm's: the last bits may differ
            assert np.all(np.isfinite(got)) and np.allclose(got, want, rtol=2e-5, atol=2e-6), (start, n)
        else:
            assert np.array_equal(bits(got), bits(want)), (start, n)
        start += n
    H.synchronize()


def sliding_spec(window=24, softcaps=(0.0, 0.0)):
    return synth.ModelSpec("slide-q4k", 2, 256, 4, 2, 64, 512, 1000, 10000.0, max_positions=512,
                           matrix_type=gguf.Q4_K, embed_type=gguf.Q4_K, output_type=gguf.Q6_K,
                           sliding_window=window, attn_softcap=softcaps[0], final_softcap=softcaps[1])


def same(got, want, what=""):
    assert np.array_equal(bits(got), bits(want)), (what, float(np.max(np.abs(np.asarray(got) - np.asarray(want)))))


def greedy(m, first, n):
    out, nxt, logits = [], first, None
    for _ in range(n):
        logits = m.forward(np.array([nxt], np.int32))
        nxt = int(O.argmax(logits))
        out.append(nxt)
    return out, logits


@pytest.mark.parametrize("kv_f16", [True, False])
@pytest.mark.parametrize("prompt_len", [9, 50, 130])
def test_sliding_model_matches_the_oracle_through_ring_wraps(tmp_path, kv_f16, prompt_len):
    """Window 24 in rings of 32 rows (8 extra): the prompt appends in the
    reference's pieces (32 rows, then 9 at a time), decoding wraps the
    rings every 32 steps; logits, greedy tokens and ring rows equal the
    oracle's."""
    path = synth.write_model(sliding_spec(), str(tmp_path / "slide.gguf"), seed=8)
    ctx = 256
    gpu = Llama(path, ctx, kv_f16=kv_f16, sliding_extra_rows=8, sliding_window=24)
    ref = O.Model(path, ctx, kv_f16=kv_f16, sliding_extra_rows=8, sliding_window=24)
    assert ref.ring == 32
    prompt = np.random.default_rng(prompt_len).integers(0, 1000, prompt_len).astype(np.int32)
    same(gpu.forward(prompt), ref.forward(prompt), "prompt")
    step = ref.forward(np.array([3], np.int32))
    same(gpu.forward(np.array([3], np.int32)), step, "decode step")
    first = int(O.argmax(step))
    want, _ = greedy(ref, first, 40)
    assert list(gpu.generate_greedy(first, 40)) == want
    for layer in range(2):
        k, v = gpu.read_kv_cache(layer)
        kr, vr = ref.kv_cache(layer)
        assert k.shape == kr.shape == (2, 32, 64)
        assert np.array_equal(k, kr) and np.array_equal(v, vr)


def test_rewind_keeps_the_window_or_starts_over(tmp_path):
    """Rewinding within what the rings hold keeps the cache; past it the
    model starts over at position 0 (llama.cpp:273-285), as the oracle."""
    path = synth.write_model(sliding_spec(), str(tmp_path / "slide.gguf"), seed=9)
    ctx = 200
    gpu = Llama(path, ctx, kv_f16=True, sliding_extra_rows=8, sliding_window=24)
    ref = O.Model(path, ctx, kv_f16=True, sliding_extra_rows=8, sliding_window=24)
    prompt = np.random.default_rng(3).integers(0, 1000, 60).astype(np.int32)
    same(gpu.forward(prompt), ref.forward(prompt))
    # rings of 32 hold positions 28..59; position 55's window is 32..55
    for target in (57, 55, 52):
        assert gpu.rewind(target) == ref.rewind(target) == target
        same(gpu.forward(prompt[target:target + 1]), ref.forward(prompt[target:target + 1]), f"after rewind to {target}")
    # position 40's window starts at 17, no longer held: both start over
    assert gpu.rewind(40) == ref.rewind(40) == 0
    same(gpu.forward(prompt[:12]), ref.forward(prompt[:12]), "after starting over")


def test_soft_caps_track_the_oracle(tmp_path):
    """Attention and final logit soft caps (tanh from the device's and the
    host's libraries: within 1e-4 of the largest logit, same argmax)."""
    path = synth.write_model(sliding_spec(window=0, softcaps=(50.0, 30.0)), str(tmp_path / "caps.gguf"), seed=10)
    gpu = Llama(path, 64, kv_f16=True, attn_softcap=50.0, final_softcap=30.0)
    ref = O.Model(path, 64, kv_f16=True, attn_softcap=50.0, final_softcap=30.0)
    prompt = np.random.default_rng(5).integers(0, 1000, 20).astype(np.int32)
    for tokens in (prompt, np.array([7], np.int32), np.array([9], np.int32)):
        got, want = gpu.forward(tokens), ref.forward(tokens)
        assert np.max(np.abs(got - want)) <= 1e-4 * np.abs(want).max()
        assert int(np.argmax(got)) == int(np.argmax(want))
        assert np.abs(want).max() <= 30.0


def test_llama_file_window_and_cap_keys_are_ignored(tmp_path):
    """A llama GGUF carrying llama.attention.sliding_window and the
    soft-capping keys runs full attention without caps, as the reference
    (it reads those keys for Gemma only, config.cpp:114-133): the same
    logits as the file without them, on the GPU and in the oracle."""
    with_keys = synth.write_model(sliding_spec(window=8, softcaps=(5.0, 3.0)), str(tmp_path / "keys.gguf"), seed=11)
    plain = synth.write_model(sliding_spec(window=0), str(tmp_path / "plain.gguf"), seed=11)
    prompt = np.random.default_rng(6).integers(0, 1000, 40).astype(np.int32)
    a, b = Llama(with_keys, 64, kv_f16=True), Llama(plain, 64, kv_f16=True)
    ref = O.Model(with_keys, 64, kv_f16=True)
    assert ref.ring == 64
    want = ref.forward(prompt)
    same(a.forward(prompt), want, "prompt")
    same(b.forward(prompt), want, "prompt, plain file")
    step = ref.forward(np.array([5], np.int32))
    same(a.forward(np.array([5], np.int32)), step, "step")
    same(b.forward(np.array([5], np.int32)), step, "step, plain file")
    a.close()
    b.close()
    ref.close()


def test_softmax_over_a_ring_needs_a_window_inside_it():
    """A ring's rows see at most `ring` positions: a window of 0 or past the
    ring would wrap positions onto each other, so the call is refused
    before anything is launched."""
    H.init()
    x = H.empty(4 * 8 * 4)
    for window in (0, 9):
        with pytest.raises(H.VkmlError, match="a ring needs a window of 1 to 8"):
            H.call("vkml_softmax", H.SoftmaxParams(4, 8, 1.0, 1, 4, 0, window, 0.0, 8), x.p, x.p)
    H.call("vkml_softmax", H.SoftmaxParams(4, 8, 1.0, 1, 4, 0, 8, 0.0, 8), x.p, x.p)
    H.synchronize()
