"""The loader's GGUF reader and host f16 conversions (vkml-framework_amd/
src/gguf.cpp), on the CPU: a small check program built from that file alone
(tests/cpp/gguf_host_check.cpp) widens every f16 bit pattern and narrows
f32 patterns, compared with numpy's float16; and it parses GGUF headers,
well-formed ones written by the synthetic-model writer and damaged ones,
which must fail with a message that says what is wrong."""
import os
import struct
import subprocess

import numpy as np
import pytest

from vkml_amd import gguf, synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("bin") / "gguf_host_check")
    subprocess.run(["g++", "-std=c++20", "-O1", "-I" + os.path.join(ROOT, "vkml-framework_amd", "include"),
                    "-I" + os.path.join(ROOT, "include"), os.path.join(ROOT, "tests", "cpp", "gguf_host_check.cpp"),
                    os.path.join(ROOT, "vkml-framework_amd", "src", "gguf.cpp"), "-o", exe], check=True)
    return exe


def run(checker, *args):
    r = subprocess.run([checker, *args], capture_output=True, text=True, timeout=60)
    return r.returncode, r.stdout


def test_every_half_widens_as_numpy(checker):
    rc, out = run(checker, "halves")
    assert rc == 0
    got = np.array([int(x, 16) for x in out.split()], np.uint32)
    want = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32).view(np.uint32)
    assert np.array_equal(got, want)


def test_narrowing_rounds_to_nearest_even_as_numpy(checker, tmp_path):
    rng = np.random.default_rng(1)
    special = np.array([0.0, -0.0, 1.0, 65504.0, 65519.996, 65520.0, 65536.0, 1e9, np.inf, -np.inf,
                        2.0 ** -14, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 2.0 ** -26, 2.0 ** -14 - 2.0 ** -25,
                        1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 1e-30, -5.960464477539063e-08], np.float32)
    # every f32 exponent, random fractions, both signs; and values halfway
    # between neighbouring halves (ties)
    rand = rng.integers(0, 1 << 32, 200000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    rand = rand[~np.isnan(rand)]
    halves = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float64)
    ties = ((halves[:-1] + halves[1:]) / 2).astype(np.float32)
    x = np.concatenate([special, rand, ties, -ties])
    path = tmp_path / "f32.txt"
    path.write_text("\n".join("%08x" % v for v in x.view(np.uint32)))
    rc, out = run(checker, "narrow", str(path))
    assert rc == 0
    got = np.array([int(v, 16) for v in out.split()], np.uint16)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, [(hex(x.view(np.uint32)[i]), hex(got[i]), hex(want[i])) for i in bad[:5]]
    # NaN narrows to a quiet NaN of the same sign
    path.write_text("7fc00000\nffa00001\n7f800001")
    rc, out = run(checker, "narrow", str(path))
    assert out.split() == ["7e00", "fe00", "7e00"]


def test_well_formed_header(checker, tmp_path):
    spec = synth.ModelSpec("hdr", 1, 256, 4, 2, 64, 512, 300, 10000.0, max_positions=64,
                           matrix_type=gguf.Q4_K, embed_type=gguf.Q4_K, output_type=gguf.Q6_K)
    path = synth.write_model(spec, str(tmp_path / "m.gguf"), seed=1)
    rc, out = run(checker, "config", path)
    assert rc == 0, out
    lines = out.splitlines()
    assert lines[0] == "version 3"
    meta = dict(ln.split(" ", 2)[1:] for ln in lines[1:])
    assert meta["general.architecture"] == '"llama"'
    assert float(meta["llama.block_count"]) == 1 and float(meta["llama.embedding_length"]) == 256
    assert float(meta["llama.rope.freq_base"]) == 10000.0


def header(version=3, tensors=(), meta=(), magic=b"GGUF"):
    """GGUF bytes: meta as (key, type, payload bytes); tensors as (name,
    dims, type, offset)."""
    b = magic + struct.pack("<IQQ", version, len(tensors), len(meta))
    for key, t, payload in meta:
        k = key.encode()
        b += struct.pack("<Q", len(k)) + k + struct.pack("<I", t) + payload
    for name, dims, t, off in tensors:
        n = name.encode()
        b += struct.pack("<Q", len(n)) + n + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        b += struct.pack("<IQ", t, off)
    return b


def gguf_string(s):
    return struct.pack("<Q", len(s)) + s


def nested_array(depth):
    # an array of one array of ... of one u32
    inner = struct.pack("<IQ", 4, 1) + struct.pack("<I", 7)
    for _ in range(depth - 1):
        inner = struct.pack("<IQ", 9, 1) + inner
    return inner


@pytest.mark.parametrize("name,data,message", [
    ("magic", header(magic=b"GGML"), "not a GGUF file"),
    ("empty", b"", "not a GGUF file"),
    ("version", header(version=4), "GGUF version 4 is not supported"),
    ("short", header()[:10], "truncated"),
    ("counts", b"GGUF" + struct.pack("<IQQ", 3, 1 << 40, 0), "truncated"),
    ("string", header(meta=[("k", 8, struct.pack("<Q", 1 << 40) + b"abc")]), "truncated"),
    ("array", header(meta=[("k", 9, struct.pack("<IQ", 4, 1 << 40))]), "truncated"),
    ("type", header(meta=[("k", 13, b"")]), "unknown type 13"),
    ("nested", header(meta=[("k", 9, nested_array(9))]), "nested more than 8 deep"),
    ("dims", header(tensors=[("t", (1, 1, 1, 1, 1), 0, 0)]), "5 dimensions"),
    ("past_end", header(tensors=[("t", (64, 64), 0, 0)]), "runs past the end of the file"),
    ("alignment", header(meta=[("general.alignment", 4, struct.pack("<I", 0))]), "general.alignment is 0"),
    ("alignment_large", header(meta=[("general.alignment", 4, struct.pack("<I", (1 << 30) + 1))]), "general.alignment is 1073741825"),
    ("array_count", header(meta=[("k", 9, struct.pack("<IQ", 8, 1 << 29))]), "truncated"),
    ("array_strings", header(meta=[("k", 9, struct.pack("<IQ", 8, 3) + b"\0" * 20)]), "truncated"),
    ("too_large", header(tensors=[("t", (1 << 62, 1 << 3), 0, 0)]), "too large"),
])
def test_damaged_header_fails_with_a_message(checker, tmp_path, name, data, message):
    path = tmp_path / (name + ".gguf")
    path.write_bytes(data)
    rc, out = run(checker, "config", str(path))
    assert rc == 1 and out.startswith("error gguf: ") and message in out, out


def test_what_the_reference_accepts_parses(checker, tmp_path):
    """A rank-0 tensor and an alignment that is not a power of two are
    accepted, as the reference's reader accepts them (gguf.cpp:341-362)."""
    path = tmp_path / "ok.gguf"
    path.write_bytes(header(meta=[("general.alignment", 4, struct.pack("<I", 24))], tensors=[("scalar", (), 0, 0)]) + b"\0" * 64)
    rc, out = run(checker, "config", str(path))
    assert rc == 0, out


def test_nesting_up_to_the_limit_parses(checker, tmp_path):
    path = tmp_path / "ok.gguf"
    path.write_bytes(header(meta=[("k", 9, nested_array(8)), ("s", 8, gguf_string(b"hi"))]))
    rc, out = run(checker, "config", str(path))
    assert rc == 0, out
    assert 'meta s "hi"' in out


@pytest.mark.parametrize("name", ["cfg1", "cfg3", "cfg5"])
def test_llama_config_from_gguf(tmp_path, name):
    """LlamaConfig::from_gguf through the C ABI (vkml_llama_read_config),
    which needs no device: the synthetic files' shapes, tying and rope."""
    from vkml_amd import llama as L
    s = synth.CONFIGS[name]
    # one layer is enough for the header (the config reads block_count)
    spec = synth.ModelSpec(s.name, 1, s.hidden, s.heads, s.kv_heads, s.head_dim, s.ffn, s.vocab, s.theta,
                           max_positions=s.max_positions, tied=s.tied, matrix_type=s.matrix_type,
                           embed_type=s.embed_type, output_type=s.output_type)
    path = synth.write_model(spec, str(tmp_path / "m.gguf"), seed=1)
    c = L.read_config(path)
    assert (c["vocab_size"], c["hidden_size"], c["intermediate_size"], c["num_layers"]) == (s.vocab, s.hidden, s.ffn, 1)
    assert (c["num_heads"], c["num_kv_heads"], c["head_dim"], c["max_positions"]) == (s.heads, s.kv_heads, s.head_dim, s.max_positions)
    assert c["tie_word_embeddings"] == int(s.tied) and c["rope_interleaved"] == 1
    assert c["rope_theta"] == np.float32(s.theta) and abs(c["rms_norm_eps"] - 1e-5) < 1e-12


def test_llama_config_errors(tmp_path):
    from vkml_amd import llama as L
    path = tmp_path / "bad.gguf"
    path.write_bytes(header(meta=[("general.architecture", 8, gguf_string(b"gpt2"))]))
    with pytest.raises(L.VkmlError, match="gpt2 model"):
        L.read_config(str(path))
    with pytest.raises(L.VkmlError, match="cannot open"):
        L.read_config(str(tmp_path / "missing.gguf"))
