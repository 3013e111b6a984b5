"""The C++ ops API (include/vkml/ops.hpp) on the MI355X, through check
programs linked against libvkml.so (what vkml-run, vkml-bench and
vkml-server call):

- tests/cpp/ops_dump.cpp runs every op on seeded inputs written here and
  writes the results back; each is compared with the CPU oracle's
  restatement of the reference's kernel (bit for bit), or, for ops the
  oracle does not restate, with numpy (exactly where the op is exact:
  casts, permutes, gathers; within f32 rounding of float64 for softmax,
  gelu, soft caps and windowed attention, where the device's exp/tanh
  decide the last bits). It also makes the calls the reference's tests
  expect to throw (tests/test_attention.cpp:212-229) and their messages
  are matched.
- tests/cpp/ops_check.cpp: matmul_transposed of one f32 row takes one
  launch (the Q8_0 of the row inside the GEMV) and must give the same bits
  as the two-launch form the same row takes when stacked twice, for q8_0,
  q4_0 and q4_1 matrices at k = 4096, 2048 and 96.
"""
import math
import os
import subprocess

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "vkml-framework_amd")


def build(tmp_path_factory, source):
    exe = str(tmp_path_factory.mktemp("bin") / os.path.splitext(source)[0])
    lib = os.path.join(PKG, "lib")
    subprocess.run(["g++", "-std=c++20", "-O1", "-I" + os.path.join(PKG, "include"), "-I" + os.path.join(ROOT, "include"),
                    os.path.join(ROOT, "tests", "cpp", source), "-L" + lib, "-lvkml", "-Wl,-rpath," + lib, "-o", exe],
                   check=True)
    return exe


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    return build(tmp_path_factory, "ops_check.cpp")


def test_one_row_matmul_transposed_is_one_launch_with_the_same_bits(checker):
    print("ops_check: matmul_transposed one row vs two rows", flush=True)
    r = subprocess.run([checker], capture_output=True, text=True, timeout=120)
    print(r.stdout, flush=True)
    lines = r.stdout.split("\n")
    assert r.returncode == 0, r.stdout + r.stderr
    assert sum(1 for ln in lines if ln.startswith("ok ")) == 9


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32 if np.asarray(a).dtype.itemsize == 4 else np.uint16)


def same(got, want, what):
    got, want = np.asarray(got), np.asarray(want)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    ok = np.array_equal(bits(got), bits(want))
    if not ok:
        d = np.flatnonzero(bits(got).ravel() != bits(want).ravel())
        raise AssertionError(f"{what}: {d.size} of {got.size} differ (first at {d[0]})")


def near(got, want, tol, what):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    err = np.max(np.abs(got - want))
    assert err <= tol, f"{what}: max |err| {err:.3g} above {tol:.3g}"


@pytest.fixture(scope="module")
def ops(tmp_path_factory):
    d = tmp_path_factory.mktemp("ops")
    rng = np.random.default_rng(2024)
    f32 = lambda *s: rng.standard_normal(s).astype(np.float32)  # noqa: E731
    inputs = {
        "a": f32(3, 5, 64), "b": f32(5, 64) + 3.0,
        "x": (f32(4, 300) * 4),
        "xr": f32(4, 4096), "w": f32(4096),
        "p": f32(2, 3, 4, 5),
        "table": f32(100, 64), "ids": np.array([0, 99, 5, -1, 100, 42, 7], np.int32),
        "rx": f32(5, 4, 128),
        "ma": f32(2, 9, 96), "mb": f32(96, 40), "mbt": f32(40, 96), "ma3": f32(3, 96),
        "qw": f32(64, 256), "qids": np.array([3, 63, 0, 64, 17], np.int32), "qa1": f32(1, 256), "qa12": f32(12, 256),
        "dq": f32(8, 1, 64), "dk": f32(2, 50, 64), "dv": f32(2, 50, 64),
        "pq": f32(8, 20, 64), "pk": f32(2, 20, 64), "pv": f32(2, 20, 64),
    }
    x = inputs["x"]
    x[0, :7] = [np.inf, -np.inf, 0.0, -0.0, 70000.0, 3e-8, -6e-5]  # casts: overflow, zeros, f16 subnormals
    x[1, :] = -np.inf
    x[1, 17] = 2.0  # softmax: -inf entries give 0
    x[2, 40:44] = x[2].max() + 1.0  # argmax: the first of equal maxima
    x[3, 5] = np.nan  # argmax skips NaN
    inputs["h"] = rng.standard_normal((4, 300)).astype(np.float16)
    inputs["mbt16"] = inputs["mbt"].astype(np.float16)
    inputs["dk16"], inputs["dv16"] = inputs["dk"].astype(np.float16), inputs["dv"].astype(np.float16)
    for name, arr in inputs.items():
        np.ascontiguousarray(arr).tofile(str(d / (name + ".bin")))
    exe = build(tmp_path_factory, "ops_dump.cpp")
    print("ops_dump: every op of the C++ API", flush=True)
    r = subprocess.run([exe, str(d)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    types = {"f32": np.float32, "f16": np.float16, "bf16": np.uint16, "i32": np.int32}
    out, errors = {}, {}
    for line in r.stdout.splitlines():
        f = line.split()
        if f[0] == "out":
            out[f[1]] = np.fromfile(str(d / (f[1] + ".bin")), types[f[2]]).reshape([int(v) for v in f[3:]])
        elif f[0] == "error":
            errors[f[1]] = " ".join(f[2:])
    return inputs, out, errors


def test_elementwise(ops):
    i, o, _ = ops
    a, b = i["a"], np.broadcast_to(i["b"], i["a"].shape)
    for op, name in enumerate(("add", "sub", "mul", "div")):
        want = np.empty(a.size, np.float32)
        O.lib().orc_binary(op, O._p(np.ascontiguousarray(a)), O._p(np.ascontiguousarray(i["b"])), a.size, i["b"].size, O._p(want))
        same(o[name], want.reshape(a.shape), name)
    # the oracle's binary is IEEE f32 arithmetic (one rounding), as numpy's
    same(o["add"], a + b, "add vs numpy")
    same(o["div"], a / b, "div vs numpy")


def test_unary_and_softmax(ops):
    i, o, _ = ops
    x = i["x"]
    fin = np.isfinite(x)
    same(o["silu"][fin], O.silu(x[fin]), "silu")
    xd = x.astype(np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        gelu = 0.5 * xd * (1.0 + np.tanh(np.clip(0.7978845608 * (xd + 0.044715 * xd ** 3), -10, 10)))
        cap = 3.0 * np.tanh(np.clip(xd / 3.0, -10, 10))
    near(o["gelu"][fin], gelu[fin], 2e-6 * np.abs(gelu[fin]).max(), "gelu")
    near(o["softcap"][fin], cap[fin], 4e-7 * 3.0, "softcap")
    sm = np.exp(xd - np.nanmax(np.where(np.isnan(xd), -np.inf, xd), axis=1, keepdims=True))
    sm /= sm.sum(axis=1, keepdims=True)
    rows = [r for r in range(4) if not (np.isnan(x[r]).any() or np.isposinf(x[r]).any()) and np.isfinite(x[r]).any()]
    assert rows == [1, 2]
    for r in rows:
        near(o["softmax"][r], sm[r], 2e-7 * 300, f"softmax row {r}")
    assert o["softmax"][1][17] == 1.0 and np.count_nonzero(o["softmax"][1]) == 1
    want = [O.argmax(x[r]) for r in range(4)]
    assert list(o["argmax"].reshape(-1)) == want
    assert want[2] == 40


def test_casts_permutes_and_gathers(ops):
    i, o, _ = ops
    x = i["x"]
    same(o["cast_f16"].view(np.uint16), O.f32_to_f16(x), "cast to f16 (the reference's to_f16)")
    fin = np.isfinite(x) & (np.abs(x) < 65504)
    same(o["cast_f16"][fin], x[fin].astype(np.float16), "cast to f16 vs numpy")
    u = x.view(np.uint32).astype(np.uint64)
    nan = np.isnan(x)
    bf = np.where(nan, (u >> 16) | 0x40, (u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    same(o["cast_bf16"], bf, "cast to bf16")
    same(o["cast_f32"], i["h"].astype(np.float32), "cast from f16")
    p = i["p"]
    same(o["permute"], np.ascontiguousarray(p.transpose(2, 0, 3, 1)), "permute")
    same(o["transpose"], np.ascontiguousarray(p.swapaxes(1, 3)), "transpose")
    t, ids = i["table"], i["ids"]
    want = np.stack([t[k] if 0 <= k < 100 else np.zeros(64, np.float32) for k in ids])
    same(o["embedding"], want, "embedding")


def test_rms_norm_and_rope(ops):
    i, o, _ = ops
    same(o["rms_norm"], O.rms_norm(i["xr"], i["w"], 1e-5), "rms_norm")
    table = O.rope_table(64, 128, 10000.0)
    same(o["rope_table"], table, "rope_table")
    assert o["rope_table"][1, 0, 0] == np.float32(math.cos(1.0)) and o["rope_table"][1, 0, 1] == np.float32(math.sin(1.0))
    same(o["rope_interleaved"], O.rope(i["rx"], table, 3, 0), "rope interleaved")
    same(o["rope_rotate_half"], O.rope(i["rx"], table, 3, 1), "rope rotate-half")


def test_matmuls(ops):
    i, o, _ = ops
    ma = i["ma"].reshape(18, 96)
    # matmul.comp's k order beyond 8 rows; gemv.comp's lanes for a few rows
    same(o["matmul"].reshape(18, 40), O.matmul_float(O.T_F32, ma, np.ascontiguousarray(i["mb"].T), None, 40, 96), "matmul")
    same(o["matmul_transposed"].reshape(18, 40), O.matmul_float(O.T_F32, ma, i["mbt"], None, 40, 96), "matmul_transposed")
    same(o["matmul_transposed_few"], O.gemv_float(O.T_F32, i["ma3"], i["mbt"], None, 40, 96), "matmul_transposed, 3 rows")
    same(o["matmul_transposed_f16"].reshape(18, 40),
         O.matmul_float(O.T_F16, ma, i["mbt16"].view(np.uint16), None, 40, 96), "matmul_transposed, f16 b")


@pytest.mark.parametrize("name,quant", [("q8_0", O.Q8_0), ("q4_0", O.Q4_0), ("q4_1", O.Q4_1)])
def test_quantized_matrices(ops, name, quant):
    i, o, _ = ops
    words, halves = O.quantize(quant, i["qw"], True)
    same(o[name + "_values"].reshape(-1).view(np.uint32), words, name + " codes")
    same(o[name + "_scales"].reshape(-1).view(np.uint16), halves, name + " scales")
    same(o[name + "_dequantized"], O.dequantize(quant, words, halves, 64, 256), name + " dequantize")
    qids = i["qids"]
    same(o[name + "_embedding"], O.embedding_quantized(quant, words, halves, 64, 256, qids), name + " embedding")
    assert not o[name + "_embedding"][3].any()  # id 64 is outside the table
    for rows, key in ((i["qa1"], "_times_one"), (i["qa12"], "_times_many")):
        aw, asc = O.quantize(O.Q8_0, rows, False)
        m = rows.shape[0]
        fn = O.gemv_dot if m <= 8 else O.matmul_dot
        same(o[name + key], fn(quant, aw, asc, m, words, halves, 64, 256), name + key)


def attention_f64(q, k, v, causal, window=0, softcap=0.0):
    heads, t, hd = q.shape
    kvh, n = k.shape[0], k.shape[1]
    out = np.empty(q.shape)
    for h in range(heads):
        kk, vv = k[h // (heads // kvh)].astype(np.float64), v[h // (heads // kvh)].astype(np.float64)
        for r in range(t):
            pos = n - t + r
            lo = max(0, pos - window + 1) if window else 0
            hi = pos + 1 if causal else n
            s = kk[lo:hi] @ q[h, r].astype(np.float64) / math.sqrt(hd)
            if softcap:
                s = softcap * np.tanh(np.clip(s / softcap, -10, 10))
            e = np.exp(s - s.max())
            out[h, r] = e @ vv[lo:hi] / e.sum()
    return out


def test_attention(ops):
    i, o, _ = ops
    same(o["attention_decode"].reshape(8, 64), O.attend_decode(i["dq"].reshape(8, 64), i["dk"], i["dv"], 0, 50), "decode f32 cache")
    same(o["attention_decode_f16"].reshape(8, 64),
         O.attend_decode(i["dq"].reshape(8, 64), i["dk16"].view(np.uint16), i["dv16"].view(np.uint16), 0, 50), "decode f16 cache")
    same(o["attention_prompt"], O.attention_prefill(i["pq"], i["pk"], i["pv"], 20), "causal prompt")
    near(o["attention_window"], attention_f64(i["pq"], i["pk"], i["pv"], True, 8, 30.0), 2e-5, "window 8 with a soft cap")
    near(o["attention_full"], attention_f64(i["pq"], i["pk"], i["pv"], False), 2e-5, "non-causal")
    assert np.array_equal(o["attention_prompt"][:, 0], np.repeat(i["pv"][:, 0], 4, axis=0)), "the first query sees v0 alone"


def test_errors_carry_the_references_messages(ops):
    _, _, e = ops
    assert "multiple" in e["heads"], e["heads"]
    assert "[4, 6, 8]" in e["v_shape"], e["v_shape"]
    assert "[4, 5, 4]" in e["head_dim"], e["head_dim"]
    assert "[heads, seq, head_dim]" in e["rank"], e["rank"]
    assert "more queries" in e["causal"], e["causal"]
    assert "broadcast" in e["broadcast"], e["broadcast"]
    assert "multiple of 32" in e["quantize_width"], e["quantize_width"]
