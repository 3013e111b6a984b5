"""Whole-model parity on the MI355X: vkml::Llama (through include/vkml_llama.h)
against the CPU oracle's restatement of the reference's Llama::run on the
same seeded GGUF files. A prompt runs at once, as the reference runs it
(projections of all its rows through gemv_dot for up to 8 rows, matmul_dot
beyond; attention as scores, causal softmax and probs v in the reference's
query chunks); a single token runs the decode step. Every kernel keeps the
reference's order of f32 operations, so logits, greedy token ids and
KV-cache rows must be identical to the oracle's, bit for bit. (The north-star
bound, logits within 1e-4 of the largest, is what a reordered sum would be
allowed; the reference's own f32 test uses 1e-4 * (1 + |want|),
tests/test_llama.cpp:758-764 there.)"""
import os

import numpy as np
import pytest

import oracle as O
from vkml_amd import gguf, synth
from vkml_amd.llama import Llama, VkmlError

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def threads():
    O.set_threads(min(16, os.cpu_count() or 1))


def spec_small_q4k():
    return synth.ModelSpec("small-q4k", 2, 256, 4, 2, 64, 512, 1000, 10000.0, max_positions=512,
                           matrix_type=gguf.Q4_K, embed_type=gguf.Q4_K, output_type=gguf.Q6_K)


def cfg_reduced(name, layers=2):
    s = synth.CONFIGS[name]
    return synth.ModelSpec(s.name + "-%dl" % layers, layers, s.hidden, s.heads, s.kv_heads, s.head_dim, s.ffn, s.vocab,
                           s.theta, max_positions=s.max_positions, tied=s.tied, matrix_type=s.matrix_type,
                           embed_type=s.embed_type, output_type=s.output_type)


@pytest.fixture(scope="module")
def files(tmp_path_factory):
    d = tmp_path_factory.mktemp("models")
    return {
        "cfg1": synth.write_model(synth.CONFIGS["cfg1"], str(d / "cfg1.gguf"), seed=1),
        "q4k": synth.write_model(spec_small_q4k(), str(d / "q4k.gguf"), seed=3),
        "cfg3": synth.write_model(cfg_reduced("cfg3"), str(d / "cfg3r.gguf"), seed=4),
        "cfg5": synth.write_model(cfg_reduced("cfg5"), str(d / "cfg5r.gguf"), seed=6),
    }


def close(got, want, tol=1e-4):
    err = np.max(np.abs(got - want))
    assert err <= tol * np.abs(want).max(), (err, np.abs(want).max())


def same(got, want):
    got, want = np.asarray(got, np.float32), np.asarray(want, np.float32)
    if not np.array_equal(got.view(np.uint32), want.view(np.uint32)):
        bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
        err = np.max(np.abs(got - want))
        raise AssertionError(f"{bad.size} of {got.size} logits differ (first at {bad[0]}), max |diff| {err:.3g}, "
                             f"max |want| {np.abs(want).max():.3g}")


def greedy_oracle(m, first, count):
    out, logits, nxt = [], None, first
    for _ in range(count):
        logits = m.forward(np.array([nxt]))
        nxt = int(O.argmax(logits))
        out.append(nxt)
    return np.array(out), logits


@pytest.mark.parametrize("name,ctx,kv_f16,prompt,steps", [
    ("cfg1", 64, False, 32, 32), ("cfg1", 64, True, 32, 32), ("q4k", 64, True, 20, 24), ("q4k", 64, False, 20, 8),
    ("cfg3", 40, True, 8, 8), ("cfg5", 40, True, 8, 8), ("cfg5", 48, True, 24, 4), ("q4k", 16, True, 1, 4)])
def test_prompt_then_greedy_matches_oracle(files, name, ctx, kv_f16, prompt, steps):
    path = files[name]
    vocab = gguf.read(path)[1]["token_embd.weight"][0][0]
    tokens = np.random.default_rng(2).integers(0, vocab, prompt).astype(np.int32)
    gpu = Llama(path, ctx, kv_f16=kv_f16)
    ref = O.Model(path, ctx, kv_f16=kv_f16)
    got = gpu.forward(tokens)
    want = ref.forward(tokens)
    same(got, want)
    first = int(O.argmax(want))
    toks, last = greedy_oracle(ref, first, steps)
    g = gpu.generate_greedy(first, steps)
    assert list(g) == list(toks)
    assert gpu.position == prompt + steps
    # logits of the last step, recomputed through forward
    gpu.rewind(prompt + steps - 1)
    same(gpu.forward(np.array([toks[-2] if steps > 1 else first])), last)


def spec_many_heads():
    # 32 query heads: a 709-token prompt's scores [32, 709, 709] f32 exceed
    # the reference's 64 MiB budget, so its queries run in chunks of 704
    # rows and then 5 (attention.cpp:209-212), the last through gemv.comp.
    return synth.ModelSpec("heads32", 1, 256, 32, 8, 64, 512, 1000, 10000.0, max_positions=1024,
                           matrix_type=gguf.Q4_K, embed_type=gguf.Q4_K, output_type=gguf.Q6_K)


@pytest.mark.parametrize("prompt,pieces", [(709, 1), (300, 1), (709, 11), (300, 4)])
def test_long_prompt_takes_the_reference_query_chunks(tmp_path, prompt, pieces):
    # pieces: this build's own split of the queries past the gemv tail (a
    # score budget of that many 64-query pieces), which must change nothing
    path = synth.write_model(spec_many_heads(), str(tmp_path / "heads32.gguf"), seed=5)
    tokens = np.random.default_rng(7).integers(0, 1000, prompt).astype(np.int32)
    budget = 0 if pieces == 1 else 32 * prompt * 4 * 64
    gpu = Llama(path, 720, kv_f16=True, prompt_score_bytes=budget)
    ref = O.Model(path, 720, kv_f16=True)
    got = gpu.forward(tokens)
    want = ref.forward(tokens)
    same(got, want)
    k, v = gpu.read_kv_cache(0)
    kv_shape = k.shape
    import ctypes
    n = int(np.prod(kv_shape))
    kr = np.ctypeslib.as_array(ctypes.cast(O.lib().orc_model_k_cache(ref._h, 0), ctypes.POINTER(ctypes.c_uint16)), (n,)).reshape(kv_shape)
    assert np.array_equal(k[:, :prompt], kr[:, :prompt])
    first = int(np.argmax(got))
    toks, _ = greedy_oracle(ref, first, 3)
    assert list(gpu.generate_greedy(first, 3)) == list(toks)


def test_f32_model_matches_double_reference(files):
    path = files["cfg1"]
    tokens = np.random.default_rng(5).integers(0, 4096, 12).astype(np.int32)
    got = Llama(path, 16, kv_f16=False).forward(tokens)
    want = O.reference_f64(path, tokens)
    assert np.all(np.abs(got - want) <= 1e-4 * (1 + np.abs(want)))


def test_int8_model_tracks_double_reference(files):
    path = files["q4k"]
    tokens = np.random.default_rng(6).integers(0, 1000, 16).astype(np.int32)
    got = Llama(path, 16, kv_f16=True).forward(tokens)
    want = O.reference_f64(path, tokens)
    assert np.max(np.abs(got - want)) <= 0.04 * np.abs(want).max()
    assert int(np.argmax(got)) == int(np.argmax(want))


def test_kv_cache_rows_match_oracle(files):
    path = files["cfg5"]
    tokens = np.random.default_rng(8).integers(0, 32768, 6).astype(np.int32)
    gpu = Llama(path, 16, kv_f16=True)
    gpu.forward(tokens)
    ref = O.Model(path, 16, kv_f16=True)
    ref.forward(tokens)
    k, v = gpu.read_kv_cache(1)
    kv_shape = k.shape
    import ctypes
    n = int(np.prod(kv_shape))
    kr = np.ctypeslib.as_array(ctypes.cast(O.lib().orc_model_k_cache(ref._h, 1), ctypes.POINTER(ctypes.c_uint16)), (n,)).reshape(kv_shape)
    vr = np.ctypeslib.as_array(ctypes.cast(O.lib().orc_model_v_cache(ref._h, 1), ctypes.POINTER(ctypes.c_uint16)), (n,)).reshape(kv_shape)
    assert np.array_equal(k[:, :6], kr[:, :6]) and np.array_equal(v[:, :6], vr[:, :6])


def test_forward_all_reset_rewind_and_errors(files):
    path = files["q4k"]
    tokens = np.random.default_rng(9).integers(0, 1000, 10).astype(np.int32)
    m = Llama(path, 16, kv_f16=True)
    ref = O.Model(path, 16, kv_f16=True)
    rows = m.forward_all(tokens)
    assert rows.shape == (10, 1000) and m.position == 10
    same(rows, ref.forward_all(tokens))  # every row through matmul_dot
    m.reset()
    ref.reset()
    assert m.position == 0
    last = m.forward(tokens)
    same(last, ref.forward(tokens))  # the last row alone through gemv_dot
    close(last, rows[-1], 1e-5)
    assert m.rewind(4) == 4 and ref.rewind(4) == 4
    again = m.forward(tokens[4:])
    same(again, ref.forward(tokens[4:]))  # 6 rows after a rewound prefix
    with pytest.raises(VkmlError, match="exceed the context length of 16"):
        m.forward(np.zeros(7, np.int32))
    with pytest.raises(VkmlError, match="rewind"):
        m.rewind(11)
    with pytest.raises(VkmlError, match="no tokens"):
        m.forward(np.zeros(0, np.int32))
    one = m.forward_all(tokens[:1])  # one row: the decode step
    assert one.shape == (1, 1000) and m.position == 11
    same(one[0], ref.forward(tokens[:1]))


def test_advance_keeps_the_rows_it_skips(files):
    """Llama::advance moves the position without running tokens: rows a
    rewind left behind still hold the prompt's keys and values, so the next
    step equals the oracle's straight run."""
    path = files["q4k"]
    tokens = np.random.default_rng(12).integers(0, 1000, 8).astype(np.int32)
    m = Llama(path, 16, kv_f16=True)
    ref = O.Model(path, 16, kv_f16=True)
    m.forward(tokens[:6])
    ref.forward(tokens[:6])
    assert m.rewind(2) == 2
    m.advance(6)
    assert m.position == 6
    same(m.forward(tokens[6:7]), ref.forward(tokens[6:7]))
    with pytest.raises(VkmlError, match="cannot advance to position 3 from 7"):
        m.advance(3)
    with pytest.raises(VkmlError, match="in a context of 16"):
        m.advance(17)


def test_graphs_and_eager_steps_agree_exactly(files):
    path = files["q4k"]
    tokens = np.random.default_rng(10).integers(0, 1000, 10).astype(np.int32)
    a = Llama(path, 16, kv_f16=True, use_graphs=True)
    b = Llama(path, 16, kv_f16=True, use_graphs=False)
    same(a.forward(tokens[:6]), b.forward(tokens[:6]))
    for t in tokens[6:]:  # decode steps: graph replays against eager launches
        same(a.forward(np.array([t])), b.forward(np.array([t])))


def test_greedy_on_device_equals_forward_then_argmax(files):
    path = files["q4k"]
    m1 = Llama(path, 40, kv_f16=True)
    m2 = Llama(path, 40, kv_f16=True)
    prompt = np.arange(5, dtype=np.int32)
    first = int(np.argmax(m1.forward(prompt)))
    m2.forward(prompt)
    fast = m1.generate_greedy(first, 12)
    slow, nxt = [], first
    for _ in range(12):
        nxt = int(np.argmax(m2.forward(np.array([nxt]))))
        slow.append(nxt)
    assert list(fast) == slow


@pytest.mark.parametrize("prompt", [8, 12])
def test_no_dot_path_uses_f32_activations(files, prompt):
    # f32 rows against the widened weights: gemv.comp for 8 rows, matmul.comp
    # for 12 (matmul.cpp:96), then decode steps
    path = files["q4k"]
    tokens = np.random.default_rng(11).integers(0, 1000, prompt + 2).astype(np.int32)
    gpu = Llama(path, 16, kv_f16=True, integer_dot=False)
    ref = O.Model(path, 16, kv_f16=True, int_dot=False)
    same(gpu.forward(tokens[:prompt]), ref.forward(tokens[:prompt]))
    for t in tokens[prompt:]:
        same(gpu.forward(np.array([t])), ref.forward(np.array([t])))


@pytest.mark.parametrize("ctx,prompt,steps", [(40, 8, 8), (300, 130, 6), (260, 254, 5)])
def test_decode_steps_across_chunk_boundaries_match_oracle(files, ctx, prompt, steps):
    """The cfg5-shaped model's decode steps against the oracle, bit for bit,
    with prompts and generations that cross 128-key chunk boundaries (the
    last case ends at the cache's final row): logits, greedy tokens and the
    KV-cache rows."""
    path = files["cfg5"]
    tokens = np.random.default_rng(12).integers(0, 32768, prompt).astype(np.int32)
    gpu = Llama(path, ctx, kv_f16=True)
    ref = O.Model(path, ctx, kv_f16=True)
    got = gpu.forward(tokens)
    same(got, ref.forward(tokens))
    first = int(np.argmax(got))
    toks, _ = greedy_oracle(ref, first, steps - 1)
    assert list(gpu.generate_greedy(first, steps - 1)) == list(toks)
    n = prompt + steps - 1
    for layer in range(2):
        k, v = gpu.read_kv_cache(layer)
        kr, vr = ref.kv_cache(layer)
        assert np.array_equal(k[:, :n], kr[:, :n]) and np.array_equal(v[:, :n], vr[:, :n])


@pytest.mark.parametrize("kv_f16", [True, False])
def test_chunk_launch_follows_the_position(files, kv_f16):
    """A 4096-row cache decoding near position 1000: each step launches the
    128-key chunks its position needs, in powers of two (8 chunks up to
    position 1023, then 16), not the cache's 32. Greedy steps and single
    steps across the 1024 boundary, graph replays and eager launches, equal
    the oracle's bit for bit. With an f32 cache (head_dim 128, q4_K o) the
    one attention launch's f32 V tile leaves it short of LDS, and the model
    must then size its launches for the separate chunk pass, merge and o
    GEMV instead of by position tier."""
    path = files["cfg5"]
    tokens = np.random.default_rng(13).integers(0, 32768, 1000).astype(np.int32)
    gpu = Llama(path, 4096, kv_f16=kv_f16)
    eager = Llama(path, 4096, kv_f16=kv_f16, use_graphs=False)
    ref = O.Model(path, 4096, kv_f16=kv_f16)
    got = gpu.forward(tokens)
    same(got, ref.forward(tokens))
    same(eager.forward(tokens), got)
    first = int(np.argmax(got))
    toks, _ = greedy_oracle(ref, first, 30)
    assert list(gpu.generate_greedy(first, 30)) == list(toks)
    assert list(eager.generate_greedy(first, 30)) == list(toks)
    assert gpu.position == 1030
    for t in toks[-1:] + [5, 77]:
        want = ref.forward(np.array([t], np.int32))
        same(gpu.forward(np.array([t], np.int32)), want)
        same(eager.forward(np.array([t], np.int32)), want)
    for layer in range(2):
        k, v = gpu.read_kv_cache(layer)
        kr, vr = ref.kv_cache(layer)
        assert np.array_equal(k[:, :1033], kr[:, :1033]) and np.array_equal(v[:, :1033], vr[:, :1033])


@pytest.mark.parametrize("hidden,ffn", [(288, 544), (256, 33280)])
def test_widths_off_the_64_grid_and_past_the_staged_bound_take_the_int8_path(tmp_path, hidden, ffn):
    """q8_0 matrices whose K is 32 mod 64 (hidden 288, ffn 544) or above the
    LDS-staged bound (ffn 33280): the reference takes its int8 path for every
    K a multiple of 32 (matmul.cpp:226-259), so prompts of 6 rows (gemv_dot)
    and 12 rows (matmul_dot) and decode steps equal the oracle's int8 path
    bit for bit."""
    spec = synth.ModelSpec(f"odd-{hidden}-{ffn}", 2, hidden, 4, 2, 64, ffn, 1000, 10000.0, max_positions=256,
                           matrix_type=gguf.Q8_0, embed_type=gguf.Q8_0, output_type=gguf.Q8_0)
    path = synth.write_model(spec, str(tmp_path / "odd.gguf"), seed=14)
    tokens = np.random.default_rng(14).integers(0, 1000, 22).astype(np.int32)
    for prompt in (6, 12):
        gpu = Llama(path, 64, kv_f16=True)
        ref = O.Model(path, 64, kv_f16=True)
        same(gpu.forward(tokens[:prompt]), ref.forward(tokens[:prompt]))
        for t in tokens[prompt:prompt + 4]:
            same(gpu.forward(np.array([t])), ref.forward(np.array([t])))


def test_vkml_bench_app_results_are_exact():
    """bin/vkml-bench's decode, m-sweep and prefill cases (gemv_dot and the
    matrix-core matmul_dot) against the "quarters" closed form: every output
    is 0.25 x K exactly."""
    import subprocess
    exe = os.path.join(os.path.dirname(__file__), "..", "vkml-framework_amd", "bin", "vkml-bench")
    if not os.path.exists(exe):
        pytest.skip("bin/vkml-bench is not built (__graft_entry__.build() builds it)")
    r = subprocess.run([exe, "3"], capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stderr
    lines = [ln for ln in r.stdout.splitlines()[1:] if ln.strip()]
    assert len(lines) == 18 and all(ln.split()[-1] == "ok" for ln in lines), r.stdout


def test_context_past_the_merge_limit_is_rejected_at_load(tmp_path):
    """Decode attention merges at most 1024 chunks of 128 keys a head, so a
    model loads with a context of 131072 positions and is refused at
    131073 with a message naming the limit (not later, at a step)."""
    spec = synth.ModelSpec("long-ctx", 1, 256, 4, 2, 64, 512, 1000, 10000.0, max_positions=140000,
                           matrix_type=gguf.Q8_0, embed_type=gguf.Q8_0, output_type=gguf.Q8_0)
    path = synth.write_model(spec, str(tmp_path / "long.gguf"), seed=9)
    with pytest.raises(VkmlError, match="at most 131072 keys"):
        Llama(path, 131073, kv_f16=True)
    m = Llama(path, 131072, kv_f16=True)
    ref = O.Model(path, 64, kv_f16=True)
    tokens = np.array([3, 17, 5], np.int32)
    for t in tokens:
        got = m.forward(np.array([t], np.int32))
        want = ref.forward(np.array([t], np.int32))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    m.close()
    ref.close()


@pytest.mark.parametrize("name,ctx", [("cfg5", 2048), ("q4k", 64)])
def test_a_wait_that_gives_up_reruns_through_launches_that_never_wait(files, name, ctx):
    """Forced from the host: with a poll limit of 1 (vkml_set_wait_limit)
    the o GEMV's workgroups give up waiting for the merges almost at once,
    set the launch's error flag and exit (every kernel still ends). The
    model notices at the end of the steps, runs them again through the
    separate chunk, merge and o launches (which never wait), and keeps
    those: logits and greedy ids equal the oracle's bit for bit, and the
    profile shows the separate launches. Then the limit is restored and a
    fresh model takes the one launch again."""
    from vkml_amd import hip as H
    from vkml_amd import llama as LL
    path = files[name]
    vocab = gguf.read(path)[1]["token_embd.weight"][0][0]
    prompt = np.random.default_rng(12).integers(0, vocab, 9).astype(np.int32)
    ref = O.Model(path, ctx, kv_f16=True)
    want = ref.forward(prompt)
    H.lib().vkml_set_wait_limit(1)
    try:
        gpu = Llama(path, ctx, kv_f16=True)
        same(gpu.forward(prompt), want)
        tok = int(O.argmax(want))
        for i in range(4):
            if i == 3:  # by now the model has fallen back
                LL.set_profiling(True)
                LL.reset_profile()
            got, exp = gpu.forward(np.array([tok], np.int32)), ref.forward(np.array([tok], np.int32))
            same(got, exp)
            tok = int(O.argmax(exp))
        labels = {n.split(":")[0] for n, _, _ in LL.profile()}
        LL.set_profiling(False)
        assert "attend_merge" in labels and "attend_fused" not in labels, labels
        g = gpu.generate_greedy(tok, 6)
        w, _ = greedy_oracle(ref, tok, 6)
        assert list(g) == list(w)
        gpu.close()
    finally:
        H.lib().vkml_set_wait_limit(0)
        LL.set_profiling(False)
    fresh = Llama(path, ctx, kv_f16=True)
    LL.set_profiling(True)
    LL.reset_profile()
    fresh.forward(prompt[:1])
    labels = {n.split(":")[0] for n, _, _ in LL.profile()}
    LL.set_profiling(False)
    assert "attend_fused" in labels, labels
    fresh.close()
    ref.close()
