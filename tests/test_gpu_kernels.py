"""Kernel parity on the MI355X: each HIP kernel through the C ABI against the
CPU oracle on the same seeded inputs. The kernels of the decode path keep the
reference's order of f32 operations, so their results must be identical to
the oracle's, bit for bit: codes, scales, casts, copies, argmax, embeddings,
GEMV (int8 and float), RMSNorm, RoPE, SiLU, attention and its merge. GEMV
results are also held to the f32 dot-product error bound against exact sums
(tests/test_quantize.cpp:197-224 in the reference: 2 k 2^-24 sum|a b|), which
pins the oracle itself. Only the matmul and softmax of the prefill-shaped ops,
whose order this build does not follow, are checked within a tolerance."""
import ctypes as C
import math

import numpy as np
import pytest

import oracle as O
from vkml_amd import hip as H
from vkml_amd import synth

pytestmark = pytest.mark.gpu


_live = []  # device buffers of the running test: freed only after it synchronizes


@pytest.fixture(scope="module", autouse=True)
def device():
    H.init()
    yield
    H.synchronize()


@pytest.fixture(autouse=True)
def keep_buffers():
    yield
    H.synchronize()
    _live.clear()


def dev(a):
    buf = H.to_device(np.ascontiguousarray(a))
    _live.append(buf)
    return buf


def p(buf):
    return buf.p if buf is not None else None


# ---------------------------------------------------------------- helpers

def q4k_layout(blocks: np.ndarray, rows: int, cols: int):
    """GGUF q4_K blocks [rows, cols/256, 144] -> (codes [rows, cols/2] u8, headers [rows, cols/256, 16] u8)."""
    b = blocks.reshape(rows, cols // 256, 144)
    return np.ascontiguousarray(b[:, :, 16:]).reshape(rows, cols // 2), np.ascontiguousarray(b[:, :, :16])


def weights(fmt, rows, cols, seed, f16_scales=True):
    """(device values, device scales, oracle quant, oracle words, oracle halves/scales, host arrays)."""
    rng = np.random.default_rng(seed)
    if fmt == H.Q4_K:
        blocks = synth.q4_k_blocks(rng, rows * cols // 256)
        codes, hdr = q4k_layout(blocks, rows, cols)
        quant, words, halves = O.load_quantized(O.GGML_Q4_K, blocks.tobytes(), rows, cols)
        return dev(codes), dev(hdr), quant, words, halves
    quant = {H.Q8_0: O.Q8_0, H.Q4_0: O.Q4_0, H.Q4_1: O.Q4_1}[fmt]
    w = (rng.standard_normal((rows, cols)) * 0.05).astype(np.float32)
    words, scales = O.quantize(quant, w, f16_scales)
    return dev(words), dev(scales), quant, words, scales


def activation(k, seed, m=1):
    a = np.random.default_rng(seed).standard_normal((m, k)).astype(np.float32)
    words, scales = O.quantize(O.Q8_0, a, False)
    return a, words, scales


def dot_bound(aw, asc, m, k, quant, words, scales, n):
    ad = O.dequantize(O.Q8_0, aw, asc, m, k).astype(np.float64)
    wd = O.dequantize(quant, words, scales, n, k).astype(np.float64)
    return ad @ wd.T, 3 * k * 2.0 ** -24 * (np.abs(ad) @ np.abs(wd).T) + 1e-30


# ---------------------------------------------------------------- quantize

@pytest.mark.parametrize("quant,hq", [(O.Q8_0, H.Q8_0), (O.Q4_0, H.Q4_0), (O.Q4_1, H.Q4_1)])
@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("src", [H.F32, H.F16, H.BF16])
def test_quantize_bit_exact(quant, hq, f16, src):
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((7, 96)) * 0.3).astype(np.float32)
    x[0, :32] = 0.0  # an all-zero block
    x[1, 5] = 40.0   # an outlier
    x[2, 32:64] = 2.0 ** -20 * rng.standard_normal(32)  # tiny: subnormal f16 scales
    if src == H.F16:
        host = x.astype(np.float16)
        x = host.astype(np.float32)
        xin = host.view(np.uint16)
    elif src == H.BF16:
        bits = (x.view(np.uint32) >> 16).astype(np.uint16)
        x = (bits.astype(np.uint32) << 16).view(np.float32)
        xin = bits
    else:
        xin = x
    want_w, want_s = O.quantize(quant, x, f16)
    blocks = x.size // 32
    dw, ds = H.empty(want_w.nbytes), H.empty(want_s.nbytes)
    H.call("vkml_quantize", H.QuantizeParams(blocks, src, hq, H.F16 if f16 else H.F32), p(dev(xin)), p(dw), p(ds))
    assert np.array_equal(dw.download(np.uint32, want_w.shape), want_w)
    assert np.array_equal(ds.download(want_s.dtype, want_s.shape).view(np.uint8), want_s.view(np.uint8))


@pytest.mark.parametrize("fmt", [H.Q8_0, H.Q4_0, H.Q4_1, H.Q4_K])
def test_dequantize_bit_exact(fmt):
    rows, cols = 6, 512
    v, s, quant, words, scales = weights(fmt, rows, cols, 5)
    want = O.dequantize(quant, words, scales, rows, cols)
    out = H.empty(want.nbytes)
    H.call("vkml_dequantize", H.DequantizeParams(rows * cols, fmt, H.F16, cols), p(v), p(s), p(out))
    assert np.array_equal(out.download(np.float32, want.shape).view(np.uint32), want.view(np.uint32))


def test_q4_k_subnormal_and_extreme_scales_bit_exact():
    rng = np.random.default_rng(9)
    blocks = synth.q4_k_blocks(rng, 64)
    d = np.array([2.0 ** -24, 3 * 2.0 ** -24, 6.0e-5, 1.0, 65504.0 / 64, 0.0, 2.0 ** -14, 7.0e-6] * 8, np.float16)
    blocks[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
    blocks[:, 2:4] = d[::-1].copy().view(np.uint8).reshape(-1, 2)
    rows, cols = 8, 2048
    codes, hdr = q4k_layout(blocks, rows, cols)
    quant, words, halves = O.load_quantized(O.GGML_Q4_K, blocks.tobytes(), rows, cols)
    want = O.dequantize(quant, words, halves, rows, cols)
    out = H.empty(want.nbytes)
    H.call("vkml_dequantize", H.DequantizeParams(rows * cols, H.Q4_K, H.F16, cols), p(dev(codes)), p(dev(hdr)), p(out))
    got = out.download(np.float32, want.shape)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# ---------------------------------------------------------------- GEMV

GEMV_SHAPES = [(256, 256), (37 * 16, 1024), (4096, 4096), (14336, 4096), (4096, 14336)]


@pytest.mark.parametrize("fmt", [H.Q8_0, H.Q4_0, H.Q4_1, H.Q4_K])
@pytest.mark.parametrize("n,k", GEMV_SHAPES)
def test_gemv_dot_matches_oracle_within_the_dot_bound(fmt, n, k):
    v, s, quant, words, scales = weights(fmt, n, k, n + k)
    a, aw, asc = activation(k, 3)
    out = H.empty(n * 4)
    H.call("vkml_gemv_dot", H.GemvDotParams(1, n, k, fmt, H.F16), p(dev(aw)), p(v), p(out), p(s), p(dev(asc)))
    got = out.download(np.float32, (1, n))
    want = O.gemv_dot(quant, aw, asc, 1, words, scales, n, k)
    exact, bound = dot_bound(aw, asc, 1, k, quant, words, scales, n)
    assert np.all(np.abs(got - exact) <= bound)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def bits(x):
    return np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)


@pytest.mark.parametrize("fmt", [H.Q8_0, H.Q4_0, H.Q4_1, H.Q4_K])
@pytest.mark.parametrize("m,n,k", [(2, 300, 512), (8, 1000, 4096), (5, 77, 768)])
def test_gemv_dot_several_rows_in_one_launch(fmt, m, n, k):
    # gemv_dot.comp's M rows (2 .. 8) in one launch, each row in the
    # single-row order: against the oracle bit for bit, f16 scales, ragged
    # n and a K that is not whole rounds of 512
    v, s, quant, words, scales = weights(fmt, n, k, m + n)
    a, aw, asc = activation(k, 9, m)
    out = H.empty(m * n * 4)
    H.call("vkml_gemv_dot", H.GemvDotParams(m, n, k, fmt, H.F16), p(dev(aw)), p(v), p(out), p(s), p(dev(asc)))
    got = out.download(np.float32, (m, n))
    assert np.array_equal(bits(got), bits(O.gemv_dot(quant, aw, asc, m, words, scales, n, k)))
    # and each row as the single-row launch gives it
    one = H.empty(n * 4)
    for i in (0, m - 1):
        aw1 = np.ascontiguousarray(aw.reshape(-1)[i * k // 4:(i + 1) * k // 4])
        as1 = np.ascontiguousarray(asc.reshape(-1)[i * k // 32:(i + 1) * k // 32])
        H.call("vkml_gemv_dot", H.GemvDotParams(1, n, k, fmt, H.F16), p(dev(aw1)), p(v), p(one), p(s), p(dev(as1)))
        assert np.array_equal(bits(one.download(np.float32, n)), bits(got[i]))


def edge_activation(m, k, seed):
    """Q8_0 rows whose blocks take the folded scaling's corner cases: all
    +127 and all -127 codes (the largest block sums), all-zero blocks (a
    zero scale and zero sums), blocks of alternating +-127 (a zero code sum
    whose dot products can also be zero), and random blocks."""
    rng = np.random.default_rng(seed)
    a = rng.standard_normal((m, k)).astype(np.float32)
    kind = rng.integers(0, 5, size=(m, k // 32))
    for r in range(m):
        for b in range(k // 32):
            blk = a[r, 32 * b:32 * b + 32]
            if kind[r, b] == 0:
                blk[:] = 0.75
            elif kind[r, b] == 1:
                blk[:] = -1.5
            elif kind[r, b] == 2:
                blk[:] = 0.0
            elif kind[r, b] == 3:
                blk[:] = np.where(np.arange(32) % 2 == 0, 0.5, -0.5)
    words, scales = O.quantize(O.Q8_0, a, False)
    return words, scales


@pytest.mark.parametrize("fmt", [H.Q4_K, H.Q4_1])
@pytest.mark.parametrize("m,n,k", [(20, 64, 512), (256, 2048, 256), (512, 4096, 256), (2048, 4096, 256)])
def test_matmul_dot_folded_scaling_corner_cases(fmt, m, n, k):
    # q4_K and q4_1 with f16 scales take the folded scaling (the block sum
    # biased by 1.5 * 2^23 in the matrix instruction's accumulator, two
    # fmas): bit for bit the reference's six operations, including negative
    # and zero (+0 and -0) scales and offsets, whole blocks of code 15 and
    # of code 0, the largest block sums and exact zero sums (where -0 * sb
    # and +0 differ in the intermediate). The shapes take the direct-load
    # kernel and the 16-, 32- and 64-row staged tiles.
    rng = np.random.default_rng(m + n + k)
    if fmt == H.Q4_K:
        blocks = synth.q4_k_blocks(rng, n * k // 256)
        sel = rng.integers(0, 8, size=len(blocks))
        blocks[sel == 0, 1] |= 0x80                # d < 0: every sub-block scale negative
        blocks[sel == 1, 3] |= 0x80                # dmin < 0: offsets positive
        blocks[sel == 2, 0:2] = 0                   # d = +0
        blocks[sel == 3, 0:2] = [0x00, 0x80]        # d = -0
        blocks[sel == 4, 16:] = 0xFF                # every code 15
        blocks[sel == 5, 16:] = 0x00                # every code 0
        blocks[sel == 6, 4:16] = 0                  # sub-block scales and mins 0
        codes, hdr = q4k_layout(blocks, n, k)
        quant, words, scales = O.load_quantized(O.GGML_Q4_K, blocks.tobytes(), n, k)
        v, s = dev(codes), dev(hdr)
    else:
        w = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
        quant = O.Q4_1
        words, scales = O.quantize(quant, w, True)
        sel = rng.integers(0, 6, size=scales.size)
        scales[sel == 0] |= 0x8000                  # negative scales and offsets
        scales[sel == 1] = 0x0000
        scales[sel == 2] = 0x8000
        v, s = dev(words), dev(scales)
    aw, asc = edge_activation(m, k, m * 7 + k)
    out = H.empty(m * n * 4)
    H.call("vkml_matmul_dot", H.GemvDotParams(m, n, k, fmt, H.F16), p(dev(aw)), p(v), p(out), p(s), p(dev(asc)))
    got = out.download(np.float32, (m, n))
    want = O.matmul_dot(quant, aw, asc, m, words, scales, n, k)
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("fmt", [H.Q8_0, H.Q4_0, H.Q4_1])
def test_gemv_dot_f32_scales_and_several_rows(fmt):
    n, k, m = 300, 512, 3
    v, s, quant, words, scales = weights(fmt, n, k, 21, f16_scales=False)
    a, aw, asc = activation(k, 4, m)
    out = H.empty(m * n * 4)
    H.call("vkml_gemv_dot", H.GemvDotParams(m, n, k, fmt, H.F32), p(dev(aw)), p(v), p(out), p(s), p(dev(asc)))
    got = out.download(np.float32, (m, n))
    exact, bound = dot_bound(aw, asc, m, k, quant, words, scales, n)
    assert np.all(np.abs(got - exact) <= bound)
    assert np.array_equal(bits(got), bits(O.gemv_dot(quant, aw, asc, m, words, scales, n, k)))


@pytest.mark.parametrize("fmt,f16", [(H.Q8_0, True), (H.Q8_0, False), (H.Q4_0, True), (H.Q4_1, True), (H.Q4_1, False), (H.Q4_K, True)])
@pytest.mark.parametrize("m,n,k", [(9, 64, 256), (37, 100, 512), (130, 1000, 2048), (512, 4096, 4096), (64, 16384, 256),
                                   (250, 16400, 256), (100, 4100, 256)])
def test_matmul_dot_bit_exact(fmt, f16, m, n, k):
    # matmul_dot.comp's order (the reference's int8 product for m > 8) on the
    # matrix cores, against the oracle bit for bit, and within the f32 dot
    # bound of the exact product; ragged tiles at m = 9, 37, 130, 250 and
    # n = 100, 1000, 16400, 4100. Operands from memory (the first three),
    # staged in LDS in 32-row tiles (512 and 250 rows) and 16-row tiles (64
    # and 100 rows); the 64-row staged tile takes the 2048 rows of
    # test_matmul_dot_folded_scaling_corner_cases.
    v, s, quant, words, scales = weights(fmt, n, k, m + n, f16_scales=f16)
    a, aw, asc = activation(k, m, m)
    out = H.empty(m * n * 4)
    H.call("vkml_matmul_dot", H.GemvDotParams(m, n, k, fmt, H.F16 if f16 else H.F32), p(dev(aw)), p(v), p(out), p(s), p(dev(asc)))
    got = out.download(np.float32, (m, n))
    assert np.array_equal(bits(got), bits(O.matmul_dot(quant, aw, asc, m, words, scales, n, k)))
    if m <= 130:
        exact, bound = dot_bound(aw, asc, m, k, quant, words, scales, n)
        assert np.all(np.abs(got - exact) <= bound)


@pytest.mark.parametrize("fmt", [H.Q8_0, H.Q4_K])
def test_gemv_dot_add_and_swiglu(fmt):
    n, k = 1024, 4096
    v, s, quant, words, scales = weights(fmt, n, k, 31)
    v2, s2, _, words2, scales2 = weights(fmt, n, k, 32)
    a, aw, asc = activation(k, 5)
    res = np.random.default_rng(6).standard_normal(n).astype(np.float32)
    out = dev(res)
    H.call("vkml_gemv_dot_add", H.GemvDotParams(1, n, k, fmt, H.F16), p(dev(aw)), p(v), p(out), p(s), p(dev(asc)), p(out))
    got = out.download(np.float32, n)
    g = O.gemv_dot(quant, aw, asc, 1, words, scales, n, k)[0]
    assert np.array_equal(bits(got), bits(res + g))
    h = H.empty(n * 4)
    H.call("vkml_gemv_dot_swiglu", H.GemvDotParams(1, n, k, fmt, H.F16), p(dev(aw)), p(dev(asc)), p(v), p(s), p(v2), p(s2), p(h))
    got = h.download(np.float32, n)
    u = O.gemv_dot(quant, aw, asc, 1, words2, scales2, n, k)[0]
    assert np.array_equal(bits(got), bits(O.silu(g) * u))


@pytest.mark.parametrize("fmt,m,n,k,f16", [(H.Q8_0, 37, 100, 512, True), (H.Q4_1, 64, 16384, 256, True),
                                           (H.Q4_K, 512, 4096, 4096, True), (H.Q4_K, 2048, 4096, 256, True),
                                           (H.Q8_0, 130, 1000, 2048, False), (H.Q4_0, 250, 2048, 1024, True),
                                           (H.Q4_1, 300, 640, 512, False)])
def test_matmul_dot_add_bit_exact(fmt, m, n, k, f16):
    # A prompt's o / down projection with the residual add in the store:
    # residual + matmul_dot's output, the binary add's f32 sum, into a
    # separate buffer and in place. The shapes take each launch form: tiles
    # read from memory (37, 130 and 300 rows), staged 16-, 32- and 64-row
    # tiles; f16 and f32 weight scales.
    v, s, quant, words, scales = weights(fmt, n, k, m + 7, f16_scales=f16)
    a, aw, asc = activation(k, m, m)
    res = np.random.default_rng(m).standard_normal((m, n)).astype(np.float32)
    want = res + O.matmul_dot(quant, aw, asc, m, words, scales, n, k)
    prm = H.GemvDotParams(m, n, k, fmt, H.F16 if f16 else H.F32)
    dres, out = dev(res), H.empty(m * n * 4)
    H.call("vkml_matmul_dot_add", prm, p(dev(aw)), p(v), p(out), p(s), p(dev(asc)), p(dres))
    assert np.array_equal(bits(out.download(np.float32, (m, n))), bits(want))
    H.call("vkml_matmul_dot_add", prm, p(dev(aw)), p(v), p(dres), p(s), p(dev(asc)), p(dres))
    assert np.array_equal(bits(dres.download(np.float32, (m, n))), bits(want))
    with pytest.raises(H.VkmlError, match="null residual"):
        H.call("vkml_matmul_dot_add", prm, p(dev(aw)), p(v), p(out), p(s), p(dev(asc)), None)


@pytest.mark.parametrize("count", [32, 4096 + 32 * 5, 512 * 14336])
def test_swiglu_quantize_bit_exact(count):
    # The prompt MLP's silu(gate) * up and its Q8_0 form in one pass: the
    # codes and scales vkml_quantize gives on the oracle's silu and product,
    # bit for bit. Blocks of zeros (scale 0), gates past exp's range both
    # ways (silu -0 and the gate itself), a ragged tail of 32-value blocks
    # against the 256-thread workgroups.
    rng = np.random.default_rng(count)
    g = (rng.standard_normal(count) * 8).astype(np.float32)
    u = rng.standard_normal(count).astype(np.float32)
    if count >= 128:
        g[:32] = 0.0
        g[32:64] = -200.0
        g[64:96] = 200.0
        u[96:128] = 0.0
    want_w, want_s = O.quantize(O.Q8_0, O.silu(g) * u, False)
    dw, ds = H.empty(count), H.empty(count // 8)
    H.call("vkml_swiglu_quantize", count, p(dev(g)), p(dev(u)), p(dw), p(ds))
    assert np.array_equal(dw.download(np.uint32, count // 4), want_w)
    assert np.array_equal(bits(ds.download(np.float32, count // 32)), bits(want_s))
    with pytest.raises(H.VkmlError, match="multiple of 32"):
        H.call("vkml_swiglu_quantize", 48, p(dev(g)), p(dev(u)), p(dw), p(ds))


@pytest.mark.parametrize("fmt,n,k", [(H.Q4_K, 4096, 4096), (H.Q4_K, 384, 256), (H.Q8_0, 4096, 4096), (H.Q4_0, 1024, 2048),
                                     (H.Q4_1, 72, 96), (H.Q8_0, 72, 96), (H.Q4_K, 6144, 4096), (H.Q4_K, 5000, 4096)])
def test_gemv_fused_quantize_prologue_bit_exact(fmt, n, k):
    # norm = 2: the Q8_0 of the f32 row inside the GEMV (the ops API's one
    # launch for a row), against quantize.comp + gemv_dot in the oracle;
    # q4_K at 6144 and 5000 rows of 4096 take the 16-lane, 24-row form (5000:
    # a last workgroup of 8 rows)
    v, s, quant, words, scales = weights(fmt, n, k, n + 11)
    a = (np.random.default_rng(k + 1).standard_normal(k) * 3).astype(np.float32)
    aw, asc = O.quantize(O.Q8_0, a.reshape(1, k), False)
    want = O.gemv_dot(quant, aw, asc, 1, words, scales, n, k)[0]
    out = H.empty(n * 4)
    prm = H.GemvFusedParams(n, k, fmt, H.F16, 0, 2, 0.0, 0)
    H.call("vkml_gemv_fused", prm, p(dev(a)), None, None, p(v), p(s), None, None, None, p(out), None, None)
    assert np.array_equal(bits(out.download(np.float32, n)), bits(want))


@pytest.mark.parametrize("fmt,n,k", [(H.Q4_K, 6144, 4096), (H.Q4_K, 384, 256), (H.Q8_0, 8192, 4096), (H.Q4_0, 1024, 2048),
                                     (H.Q4_K, 5000, 4096), (H.Q8_0, 6144, 4096)])
def test_gemv_fused_norm_prologue_bit_exact(fmt, n, k):
    # rms_norm + Q8_0 inside the GEMV == the separate kernels' results
    v, s, quant, words, scales = weights(fmt, n, k, n + 7)
    rng = np.random.default_rng(k)
    x = (rng.standard_normal(k) * 2).astype(np.float32)
    nw = rng.standard_normal(k).astype(np.float32)
    xn = O.rms_norm(x.reshape(1, k), nw, 1e-5)
    aw, asc = O.quantize(O.Q8_0, xn, False)
    want = O.gemv_dot(quant, aw, asc, 1, words, scales, n, k)[0]
    out = H.empty(n * 4)
    prm = H.GemvFusedParams(n, k, fmt, H.F16, 0, 1, 1e-5, 0)
    H.call("vkml_gemv_fused", prm, p(dev(x)), None, p(dev(nw)), p(v), p(s), None, None, None, p(out), None, None)
    assert np.array_equal(bits(out.download(np.float32, n)), bits(want))


@pytest.mark.parametrize("norm", [0, 1])
@pytest.mark.parametrize("fmt,n,k", [(H.Q4_K, 14336, 4096), (H.Q4_K, 512, 256), (H.Q8_0, 2048, 1024), (H.Q4_K, 1056, 512)])
def test_gemv_fused_swiglu_quantized_output_bit_exact(norm, fmt, n, k):
    # (n = 1056: 33 of the epilogue's 32-row Q8_0 blocks)
    v, s, quant, words, scales = weights(fmt, n, k, 41)
    v2, s2, _, words2, scales2 = weights(fmt, n, k, 42)
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(k) * 2).astype(np.float32)
    nw = rng.standard_normal(k).astype(np.float32)
    if norm:
        aw, asc = O.quantize(O.Q8_0, O.rms_norm(x.reshape(1, k), nw, 1e-5), False)
        a_in, a_sc = dev(x), None
    else:
        aw, asc = O.quantize(O.Q8_0, x.reshape(1, k), False)
        a_in, a_sc = dev(aw), dev(asc)
    g = O.gemv_dot(quant, aw, asc, 1, words, scales, n, k)[0]
    u = O.gemv_dot(quant, aw, asc, 1, words2, scales2, n, k)[0]
    want = O.silu(g) * u
    hw, hs = O.quantize(O.Q8_0, want.reshape(1, n), False)
    h, hv, hsc = H.empty(n * 4), H.empty(n), H.empty(n // 32 * 4)
    prm = H.GemvFusedParams(n, k, fmt, H.F16, 2, norm, 1e-5, 1)
    H.call("vkml_gemv_fused", prm, p(a_in), p(a_sc), p(dev(nw)), p(v), p(s), p(v2), p(s2), None, p(h), p(hv), p(hsc))
    assert np.array_equal(bits(h.download(np.float32, n)), bits(want))
    assert np.array_equal(hv.download(np.uint32, hw.shape), hw)
    assert np.array_equal(hsc.download(np.float32, hs.shape).view(np.uint32), hs.view(np.uint32))


@pytest.mark.parametrize("bt", [H.F32, H.F16, H.BF16, H.Q8_0, H.Q4_0, H.Q4_1, H.Q4_K])
def test_float_gemv_path(bt):
    n, k, m = 100, 512, 2
    rng = np.random.default_rng(7)
    a = rng.standard_normal((m, k)).astype(np.float32)
    sc = None
    if bt == H.F32:
        b = (rng.standard_normal((n, k)) * 0.05).astype(np.float32); wd = b; ot = O.T_F32; ob, osc = b, None
    elif bt in (H.F16, H.BF16):
        w = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
        if bt == H.F16:
            b = w.astype(np.float16).view(np.uint16); wd = b.view(np.float16).astype(np.float32); ot = O.T_F16
        else:
            b = (w.view(np.uint32) >> 16).astype(np.uint16); wd = (b.astype(np.uint32) << 16).view(np.float32); ot = O.T_BF16
        ob, osc = b, None
    else:
        dv, ds, quant, words, scales = weights(bt, n, k, 8)
        wd = O.dequantize(quant, words, scales, n, k)
        b, sc = None, None
        # q4_K runs as the reference's q4_1 repack, which the oracle holds
        ot, ob, osc = {O.Q8_0: O.T_Q8, O.Q4_0: O.T_Q4, O.Q4_1: O.T_Q4_1}[quant], words, scales
    out = H.empty(m * n * 4)
    if b is not None:
        H.call("vkml_gemv", H.GemvParams(m, n, k, bt, H.F16), p(dev(a)), p(dev(b)), p(out), None)
    else:
        H.call("vkml_gemv", H.GemvParams(m, n, k, bt, H.F16), p(dev(a)), p(dv), p(out), p(ds))
    got = out.download(np.float32, (m, n))
    want = a.astype(np.float64) @ wd.astype(np.float64).T
    bound = 3 * k * 2.0 ** -24 * (np.abs(a.astype(np.float64)) @ np.abs(wd.astype(np.float64)).T) + 1e-30
    assert np.all(np.abs(got - want) <= bound)
    assert np.array_equal(bits(got), bits(O.gemv_float(ot, a, ob, osc, n, k)))


# ---------------------------------------------------------------- norms and rope

@pytest.mark.parametrize("cols", [256, 4096, 14336, 2048])
def test_rms_norm_quantize(cols):
    rng = np.random.default_rng(cols)
    x = (rng.standard_normal((2, cols)) * 3).astype(np.float32)
    w = rng.standard_normal(cols).astype(np.float32)
    y, vals, scs = H.empty(x.nbytes), H.empty(x.size), H.empty(x.size // 32 * 4)
    H.call("vkml_rms_norm_quantize", H.RmsNormParams(2, cols, 1e-5), p(dev(x)), p(dev(w)), p(y), p(vals), p(scs))
    got = y.download(np.float32, x.shape)
    want = O.rms_norm(x, w, 1e-5)
    assert np.array_equal(bits(got), bits(want))
    # the quantized form is exactly the reference quantizer's of these f32 values
    ww, ws = O.quantize(O.Q8_0, got, False)
    assert np.array_equal(vals.download(np.uint32, ww.shape), ww)
    assert np.array_equal(scs.download(np.float32, ws.shape).view(np.uint32), ws.view(np.uint32))
    plain = H.empty(x.nbytes)
    H.call("vkml_rms_norm", H.RmsNormParams(2, cols, 1e-5), p(dev(x)), p(dev(w)), p(plain))
    assert np.array_equal(bits(plain.download(np.float32, x.shape)), bits(want))


@pytest.mark.parametrize("style", [0, 1])
def test_rope_bit_exact(style):
    seq, heads, dim = 3, 4, 128
    x = np.random.default_rng(1).standard_normal((seq, heads, dim)).astype(np.float32)
    table = O.rope_table(9000, dim, 1e6)
    want = O.rope(x, table, 8000, style)
    out = H.empty(x.nbytes)
    rows = seq * heads
    H.call("vkml_rope", H.RopeParams(rows * dim // 2, dim // 2, dim, heads, seq, 8000, 0, style), p(dev(x)), p(dev(table)), p(out))
    assert np.array_equal(out.download(np.float32, x.shape).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("kv_type", [H.F16, H.F32])
def test_rope_kv_append_bit_exact(kv_type):
    heads, kvh, hd, cap, pos = 32, 8, 128, 64, 37
    rng = np.random.default_rng(2)
    qkv = rng.standard_normal((heads + 2 * kvh) * hd).astype(np.float32)
    table = O.rope_table(cap, hd, 1e6)
    dt = np.uint16 if kv_type == H.F16 else np.float32
    kc, vc = H.empty(kvh * cap * hd * 4), H.empty(kvh * cap * hd * 4)
    q = H.empty(heads * hd * 4)
    H.call("vkml_rope_kv_append", H.RopeKvParams(heads, kvh, hd, cap, pos, 0, kv_type, 1), p(dev(qkv)), p(dev(table)),
           p(q), p(kc), p(vc), None)
    qr = O.rope(qkv[:heads * hd].reshape(1, heads, hd), table, pos, 0).ravel()
    kr = O.rope(qkv[heads * hd:(heads + kvh) * hd].reshape(1, kvh, hd), table, pos, 0).reshape(kvh, hd)
    vr = qkv[(heads + kvh) * hd:].reshape(kvh, hd)
    assert np.array_equal(q.download(np.float32, heads * hd).view(np.uint32), qr.view(np.uint32))
    kg = kc.download(dt, (kvh, cap, hd))[:, pos]
    vg = vc.download(dt, (kvh, cap, hd))[:, pos]
    if kv_type == H.F16:
        assert np.array_equal(kg, O.f32_to_f16(kr)) and np.array_equal(vg, O.f32_to_f16(vr))
    else:
        assert np.array_equal(kg.view(np.uint32), kr.view(np.uint32)) and np.array_equal(vg.view(np.uint32), vr.view(np.uint32))


@pytest.mark.parametrize("fmt,heads,kvh,hd,kv_type,split", [
    (H.Q4_K, 32, 8, 128, H.F16, False), (H.Q8_0, 16, 4, 64, H.F32, False), (H.Q4_K, 8, 8, 64, H.F16, True)])
def test_gemv_rope_bit_exact(fmt, heads, kvh, hd, kv_type, split):
    # the q|k|v GEMV with the RMSNorm + Q8_0 prologue and the RoPE + KV append
    # epilogue: q and k rotated as rope.comp does at the state's position, v
    # as is, the new key and value in the caches' row position % capacity;
    # split: q, k and v as three matrices at their row offsets
    k, cap, pos = 2048 if hd == 128 else 512, 96, 133
    rows = (heads + 2 * kvh) * hd
    rng = np.random.default_rng(heads + hd + kvh)
    x = (rng.standard_normal(k) * 3).astype(np.float32)
    nw = rng.standard_normal(k).astype(np.float32)
    table = O.rope_table(pos + 1, hd, 1e6)
    aw, asc = O.quantize(O.Q8_0, O.rms_norm(x.reshape(1, k), nw, 1e-5), False)
    dt = np.uint16 if kv_type == H.F16 else np.float32
    kc, vc = dev(np.zeros((kvh, cap, hd), dt)), dev(np.zeros((kvh, cap, hd), dt))
    st, qkv = H.empty(16), H.empty(rows * 4)
    H.call("vkml_state_set", p(st), 0, pos, 0)
    parts = [(0, heads * hd), (heads * hd, kvh * hd), ((heads + kvh) * hd, kvh * hd)] if split else [(0, rows)]
    y = np.empty(rows, np.float32)
    for i, (row0, n) in enumerate(parts):
        v, s_, quant, words, scales = weights(fmt, n, k, 60 + i)
        y[row0:row0 + n] = O.gemv_dot(quant, aw, asc, 1, words, scales, n, k)[0]
        prm = H.GemvRopeParams(n, k, fmt, H.F16, 1e-5, row0, heads, kvh, hd, cap, kv_type, 1)
        H.call("vkml_gemv_rope", prm, p(dev(x)), p(dev(nw)), p(v), p(s_), p(qkv), p(dev(table)), p(st), p(kc), p(vc))
    q = O.rope(y[:heads * hd].reshape(1, heads, hd), table, pos, 0).ravel()
    kr = O.rope(y[heads * hd:(heads + kvh) * hd].reshape(1, kvh, hd), table, pos, 0).reshape(kvh, hd)
    vr = y[(heads + kvh) * hd:].reshape(kvh, hd)
    want = np.concatenate([q, kr.ravel(), vr.ravel()])
    assert np.array_equal(bits(qkv.download(np.float32, rows)), bits(want))
    row = pos % cap
    kg, vg = kc.download(dt, (kvh, cap, hd)), vc.download(dt, (kvh, cap, hd))
    if kv_type == H.F16:
        assert np.array_equal(kg[:, row], O.f32_to_f16(kr)) and np.array_equal(vg[:, row], O.f32_to_f16(vr))
    else:
        assert np.array_equal(bits(kg[:, row]), bits(kr)) and np.array_equal(bits(vg[:, row]), bits(vr))
    others = np.delete(np.arange(cap), row)
    assert not kg[:, others].any() and not vg[:, others].any()


def test_gemv_rope_rejects_odd_rows():
    prm = H.GemvRopeParams(63, 256, H.Q4_K, H.F16, 1e-5, 1, 4, 2, 32, 16, H.F16, 1)
    with pytest.raises(H.VkmlError, match="even-aligned"):
        H.call("vkml_gemv_rope", prm, None, None, None, None, None, None, None, None, None)


# ---------------------------------------------------------------- attention

@pytest.mark.parametrize("hd,heads,kvh,kv_len,kv_type,extra", [
    (128, 32, 8, 4096, H.F16, 0), (128, 32, 8, 1, H.F16, 3), (64, 32, 8, 640, H.F16, 0),
    (64, 4, 2, 45, H.F32, 1), (128, 32, 8, 300, H.F32, 0), (256, 8, 8, 200, H.F16, 0), (128, 8, 1, 1000, H.F16, 2),
    (256, 16, 2, 129, H.F32, 0), (64, 16, 4, 128, H.F16, 0), (64, 8, 2, 9000, H.F16, 0),
    # past 16 chunks the merge spreads over (head, 32-element slice) workgroups,
    # past 256 in passes of 256 chunks; empty chunks among them
    (128, 8, 2, 3000, H.F32, 20), (64, 8, 2, 40000, H.F16, 2), (256, 4, 4, 33000, H.F16, 0),
    # four heads a chunk workgroup (GQA groups of 4 and 8, enough chunks)
    (128, 16, 2, 40000, H.F16, 0), (128, 32, 8, 20000, H.F32, 1)])
def test_attend_bit_exact(hd, heads, kvh, kv_len, kv_type, extra):
    cap = kv_len + 7
    rng = np.random.default_rng(kv_len)
    q = rng.standard_normal((heads, hd)).astype(np.float32)
    k = rng.standard_normal((kvh, cap, hd)).astype(np.float32)
    v = rng.standard_normal((kvh, cap, hd)).astype(np.float32)
    if kv_type == H.F16:
        kc, vc = k.astype(np.float16).view(np.uint16), v.astype(np.float16).view(np.uint16)
    else:
        kc, vc = k, v
    chunks = (kv_len + 127) // 128 + extra  # spare chunks come out empty
    prm = H.AttendParams(0, kv_len, cap, heads, kvh, hd, kv_type, chunks, 1.0 / math.sqrt(hd), 0.0)
    part, stats = H.empty(heads * chunks * hd * 4), H.empty(heads * chunks * 8)
    out, vals, scs = H.empty(heads * hd * 4), H.empty(heads * hd), H.empty(heads * hd // 32 * 4)
    H.call("vkml_attend", prm, p(dev(q)), p(dev(kc)), p(dev(vc)), p(part), p(stats), None)
    H.call("vkml_attend_merge", prm, p(part), p(stats), p(out), p(vals), p(scs))
    got = out.download(np.float32, (heads, hd))
    want = O.attend_decode(q, kc, vc, 0, kv_len)
    assert np.array_equal(bits(got), bits(want))
    ww, ws = O.quantize(O.Q8_0, got, False)
    assert np.array_equal(vals.download(np.uint32, ww.shape), ww)
    assert np.array_equal(scs.download(np.float32, ws.shape).view(np.uint32), ws.view(np.uint32))


def test_attend_reads_kv_len_from_the_decode_state():
    hd, heads, kvh, cap = 128, 32, 8, 512
    rng = np.random.default_rng(3)
    q = rng.standard_normal((heads, hd)).astype(np.float32)
    kc = rng.standard_normal((kvh, cap, hd)).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal((kvh, cap, hd)).astype(np.float16).view(np.uint16)
    st = H.empty(16)
    H.call("vkml_state_set", p(st), 5, 299, 0)
    chunks = cap // 128
    prm = H.AttendParams(0, 0, cap, heads, kvh, hd, H.F16, chunks, 1.0 / math.sqrt(hd), 0.0)
    part, stats, out = H.empty(heads * chunks * hd * 4), H.empty(heads * chunks * 8), H.empty(heads * hd * 4)
    H.call("vkml_attend", prm, p(dev(q)), p(dev(kc)), p(dev(vc)), p(part), p(stats), p(st))
    H.call("vkml_attend_merge", prm, p(part), p(stats), p(out), None, None)
    want = O.attend_decode(q, kc, vc, 0, 300)
    assert np.array_equal(bits(out.download(np.float32, (heads, hd))), bits(want))


def test_attend_from_a_window_start():
    # keys 100..499 (a sliding window's start), chunks of 128 from key 100
    hd, heads, kvh, cap = 64, 8, 2, 512
    rng = np.random.default_rng(8)
    q = rng.standard_normal((heads, hd)).astype(np.float32)
    kc = rng.standard_normal((kvh, cap, hd)).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal((kvh, cap, hd)).astype(np.float16).view(np.uint16)
    chunks = (500 - 100 + 127) // 128
    prm = H.AttendParams(100, 500, cap, heads, kvh, hd, H.F16, chunks, 1.0 / math.sqrt(hd), 0.0)
    part, stats, out = H.empty(heads * chunks * hd * 4), H.empty(heads * chunks * 8), H.empty(heads * hd * 4)
    H.call("vkml_attend", prm, p(dev(q)), p(dev(kc)), p(dev(vc)), p(part), p(stats), None)
    H.call("vkml_attend_merge", prm, p(part), p(stats), p(out), None, None)
    want = O.attend_decode(q, kc, vc, 100, 500)
    assert np.array_equal(bits(out.download(np.float32, (heads, hd))), bits(want))


@pytest.mark.parametrize("hd,heads,kvh,pos,kv_type,style", [
    (128, 32, 8, 4096, H.F16, 0), (64, 32, 8, 200, H.F16, 1), (64, 4, 2, 45, H.F32, 0), (128, 8, 8, 127, H.F16, 0),
    (256, 8, 4, 300, H.F16, 1), (128, 16, 2, 700, H.F32, 0), (128, 32, 8, 0, H.F16, 0)])
def test_attend_step_bit_exact(hd, heads, kvh, pos, kv_type, style):
    # rope + append + attention + merge + quantize, two steps in a row,
    # against the oracle's pieces
    cap = pos + 67
    chunks = (cap + 127) // 128
    rng = np.random.default_rng(pos + hd)
    dt = np.uint16 if kv_type == H.F16 else np.float32
    prior = rng.standard_normal((2, kvh, cap, hd)).astype(np.float32)
    caches = [prior[i].astype(np.float16).view(np.uint16) if kv_type == H.F16 else prior[i] for i in range(2)]
    kc, vc = dev(caches[0]), dev(caches[1])
    table = O.rope_table(cap, hd, 1e6)
    dtab = dev(table)
    part, stats = H.empty(heads * chunks * hd * 4), H.empty(heads * chunks * 8)
    for step in range(2):
        p_now = pos + step
        qkv = rng.standard_normal((heads + 2 * kvh) * hd).astype(np.float32)
        out, vals, scs = H.empty(heads * hd * 4), H.empty(heads * hd), H.empty(heads * hd // 32 * 4)
        prm = H.AttendStepParams(heads, kvh, hd, cap, 0, p_now, kv_type, chunks, style, 1, 1.0 / math.sqrt(hd), 0.0)
        H.call("vkml_attend_step", prm, p(dev(qkv)), p(dtab), p(kc), p(vc), p(part), p(stats), p(out), p(vals), p(scs), None)
        q = O.rope(qkv[:heads * hd].reshape(1, heads, hd), table, p_now, style).reshape(heads, hd)
        k = O.rope(qkv[heads * hd:(heads + kvh) * hd].reshape(1, kvh, hd), table, p_now, style).reshape(kvh, hd)
        v = qkv[(heads + kvh) * hd:].reshape(kvh, hd)
        for c, new in ((caches[0], k), (caches[1], v)):
            c[:, p_now] = O.f32_to_f16(new) if kv_type == H.F16 else new
        assert np.array_equal(kc.download(dt, caches[0].shape), caches[0])
        assert np.array_equal(vc.download(dt, caches[1].shape), caches[1])
        want = O.attend_decode(q, caches[0], caches[1], 0, p_now + 1)
        got = out.download(np.float32, (heads, hd))
        assert np.array_equal(bits(got), bits(want))
        ww, ws = O.quantize(O.Q8_0, want, False)
        assert np.array_equal(vals.download(np.uint32, ww.shape), ww)
        assert np.array_equal(scs.download(np.float32, ws.shape).view(np.uint32), ws.view(np.uint32))


@pytest.mark.parametrize("hd,heads,kvh,pos,kv_type,fmt,n", [
    (128, 32, 8, 4096, H.F16, H.Q4_K, 4096), (128, 32, 8, 300, H.F16, H.Q8_0, 4096), (64, 32, 8, 200, H.F16, H.Q4_K, 2048),
    (256, 8, 4, 300, H.F16, H.Q4_K, 2048), (128, 16, 2, 700, H.F32, H.Q4_K, 1024), (128, 16, 4, 130, H.F16, H.Q4_0, 2048)])
def test_attend_step_o_bit_exact(hd, heads, kvh, pos, kv_type, fmt, n):
    # attention + merge + Q8_0 + the o GEMV + residual in one call (the
    # merge and the GEMV in one launch, except q4_0, which takes the three
    # launches), two steps in a row: against the oracle and against
    # vkml_attend_step + vkml_gemv_dot_add on a second copy of the caches
    k = heads * hd
    cap = pos + 67
    chunks = (cap + 127) // 128
    rng = np.random.default_rng(pos + hd + n)
    dt = np.uint16 if kv_type == H.F16 else np.float32
    prior = rng.standard_normal((2, kvh, cap, hd)).astype(np.float32)
    caches = [prior[i].astype(np.float16).view(np.uint16) if kv_type == H.F16 else prior[i] for i in range(2)]
    kc, vc, kc2, vc2 = dev(caches[0]), dev(caches[1]), dev(caches[0]), dev(caches[1])
    table = O.rope_table(cap, hd, 1e6)
    dtab = dev(table)
    v, s_, quant, words, scales = weights(fmt, n, k, pos + 3)
    x0 = rng.standard_normal(n).astype(np.float32)
    x, x2 = dev(x0), dev(x0)
    sync = H.empty(H.lib().vkml_attend_o_sync_bytes())
    H.call("vkml_fill_u32", p(sync), 0, H.lib().vkml_attend_o_sync_bytes() // 4)
    part, stats = H.empty(heads * chunks * hd * 4), H.empty(heads * chunks * 8)
    part2, stats2 = H.empty(heads * chunks * hd * 4), H.empty(heads * chunks * 8)
    op = H.GemvDotParams(1, n, k, fmt, H.F16)
    want_x = x0.copy()
    for step in range(2):
        p_now = pos + step
        qkv = rng.standard_normal((heads + 2 * kvh) * hd).astype(np.float32)
        dq = dev(qkv)
        out, vals, scs = H.empty(k * 4), H.empty(k), H.empty(k // 32 * 4)
        out2, vals2, scs2 = H.empty(k * 4), H.empty(k), H.empty(k // 32 * 4)
        prm = H.AttendStepParams(heads, kvh, hd, cap, 0, p_now, kv_type, chunks, 0, 1, 1.0 / math.sqrt(hd), 0.0)
        H.call("vkml_attend_step_o", prm, p(dq), p(dtab), p(kc), p(vc), p(part), p(stats), p(out), p(vals), p(scs), None,
               op, p(v), p(s_), p(x), p(sync))
        H.call("vkml_attend_step", prm, p(dq), p(dtab), p(kc2), p(vc2), p(part2), p(stats2), p(out2), p(vals2), p(scs2), None)
        H.call("vkml_gemv_dot_add", op, p(vals2), p(v), p(x2), p(s_), p(scs2), p(x2))
        H.call("vkml_attend_o_check", p(sync))  # no wait gave up
        q = O.rope(qkv[:k].reshape(1, heads, hd), table, p_now, 0).reshape(heads, hd)
        kn = O.rope(qkv[k:k + kvh * hd].reshape(1, kvh, hd), table, p_now, 0).reshape(kvh, hd)
        vn = qkv[k + kvh * hd:].reshape(kvh, hd)
        for c, new in ((caches[0], kn), (caches[1], vn)):
            c[:, p_now] = O.f32_to_f16(new) if kv_type == H.F16 else new
        assert np.array_equal(kc.download(dt, caches[0].shape), caches[0])
        assert np.array_equal(vc.download(dt, caches[1].shape), caches[1])
        want = O.attend_decode(q, caches[0], caches[1], 0, p_now + 1)
        assert np.array_equal(bits(out.download(np.float32, (heads, hd))), bits(want))
        ww, ws = O.quantize(O.Q8_0, want.reshape(1, k), False)
        assert np.array_equal(vals.download(np.uint32, ww.shape), ww)
        assert np.array_equal(scs.download(np.float32, ws.shape).view(np.uint32), ws.view(np.uint32))
        want_x = want_x + O.gemv_dot(quant, ww, ws, 1, words, scales, n, k)[0]
        got = x.download(np.float32, n)
        assert np.array_equal(bits(got), bits(want_x))
        assert np.array_equal(bits(got), bits(x2.download(np.float32, n)))


@pytest.mark.parametrize("hd,heads,kvh,pos,kv_type,fmt,n,window,blocks", [
    (128, 32, 8, 4096, H.F16, H.Q4_K, 4096, 0, 2), (128, 32, 8, 300, H.F16, H.Q8_0, 4096, 0, 3),
    (64, 32, 8, 200, H.F16, H.Q4_K, 2048, 0, 2), (256, 8, 4, 300, H.F16, H.Q4_K, 2048, 0, 2),
    (128, 16, 2, 700, H.F32, H.Q4_K, 1024, 0, 2), (128, 16, 4, 130, H.F16, H.Q4_0, 2048, 0, 2),
    (128, 12, 4, 260, H.F16, H.Q4_K, 1536, 0, 2), (64, 8, 8, 0, H.F32, H.Q4_K, 256, 0, 2),
    (128, 16, 4, 500, H.F16, H.Q4_K, 2048, 200, 3)])
def test_attend_step_fused_bit_exact(hd, heads, kvh, pos, kv_type, fmt, n, window, blocks):
    # the chunk pass, the merges (by each head set's last chunk item) and the
    # o GEMV + residual in one launch, four steps in a row cycling through
    # the sync blocks: against the oracle and against vkml_attend_step_o on
    # copies of the caches; q4_0 o weights take the separate launches (with
    # the next block cleared all the same); 12 heads over 4 KV heads take
    # one head a workgroup
    k = heads * hd
    cap = pos + 67
    chunks = (cap + 127) // 128
    rng = np.random.default_rng(pos + hd + n + 1)
    dt = np.uint16 if kv_type == H.F16 else np.float32
    prior = rng.standard_normal((2, kvh, cap, hd)).astype(np.float32)
    caches = [prior[i].astype(np.float16).view(np.uint16) if kv_type == H.F16 else prior[i] for i in range(2)]
    kc, vc, kc2, vc2 = dev(caches[0]), dev(caches[1]), dev(caches[0]), dev(caches[1])
    table = O.rope_table(cap, hd, 1e6)
    dtab = dev(table)
    v, s_, quant, words, scales = weights(fmt, n, k, pos + 5)
    x0 = rng.standard_normal(n).astype(np.float32)
    x, x2 = dev(x0), dev(x0)
    fbytes = H.lib().vkml_attend_fused_sync_bytes(blocks)
    fsync = H.empty(fbytes)
    H.call("vkml_fill_u32", p(fsync), 0, fbytes // 4)
    sync = H.empty(H.lib().vkml_attend_o_sync_bytes())
    H.call("vkml_fill_u32", p(sync), 0, H.lib().vkml_attend_o_sync_bytes() // 4)
    part, stats = H.empty(heads * chunks * hd * 4), H.empty(heads * chunks * 8)
    part2, stats2 = H.empty(heads * chunks * hd * 4), H.empty(heads * chunks * 8)
    st = H.empty(16)
    op = H.GemvDotParams(1, n, k, fmt, H.F16)
    want_x = x0.copy()
    for step in range(4):
        p_now = pos + step
        print(f"fused case hd={hd} heads={heads} kvh={kvh} pos={p_now} n={n} window={window} block={step % blocks}", flush=True)
        H.call("vkml_state_set", p(st), 0, p_now, 0)
        qkv = rng.standard_normal((heads + 2 * kvh) * hd).astype(np.float32)
        dq = dev(qkv)
        out, vals, scs = H.empty(k * 4), H.empty(k), H.empty(k // 32 * 4)
        out2, vals2, scs2 = H.empty(k * 4), H.empty(k), H.empty(k // 32 * 4)
        prm = H.AttendStepParams(heads, kvh, hd, cap, 0, 0, kv_type, chunks, 0, 1, 1.0 / math.sqrt(hd), 0.0, window)
        H.call("vkml_attend_step_fused", prm, p(dq), p(dtab), p(kc), p(vc), p(part), p(stats), p(out), p(vals), p(scs), p(st),
               op, p(v), p(s_), p(x), p(fsync), step % blocks, blocks)
        H.call("vkml_attend_step_o", prm, p(dq), p(dtab), p(kc2), p(vc2), p(part2), p(stats2), p(out2), p(vals2), p(scs2), p(st),
               op, p(v), p(s_), p(x2), p(sync))
        H.call("vkml_attend_fused_check", p(fsync), blocks)  # no wait gave up
        q = O.rope(qkv[:k].reshape(1, heads, hd), table, p_now, 0).reshape(heads, hd)
        kn = O.rope(qkv[k:k + kvh * hd].reshape(1, kvh, hd), table, p_now, 0).reshape(kvh, hd)
        vn = qkv[k + kvh * hd:].reshape(kvh, hd)
        for c, new in ((caches[0], kn), (caches[1], vn)):
            c[:, p_now] = O.f32_to_f16(new) if kv_type == H.F16 else new
        assert np.array_equal(kc.download(dt, caches[0].shape), caches[0])
        assert np.array_equal(vc.download(dt, caches[1].shape), caches[1])
        start = max(0, p_now + 1 - window) if window else 0
        want = O.attend_decode(q, caches[0], caches[1], start, p_now + 1)
        assert np.array_equal(bits(out.download(np.float32, (heads, hd))), bits(want))
        ww, ws = O.quantize(O.Q8_0, want.reshape(1, k), False)
        assert np.array_equal(vals.download(np.uint32, ww.shape), ww)
        assert np.array_equal(scs.download(np.float32, ws.shape).view(np.uint32), ws.view(np.uint32))
        want_x = want_x + O.gemv_dot(quant, ww, ws, 1, words, scales, n, k)[0]
        got = x.download(np.float32, n)
        assert np.array_equal(bits(got), bits(want_x))
        assert np.array_equal(bits(got), bits(x2.download(np.float32, n)))


def test_decode_layers_chained_bit_exact():
    # Two decode layers' attention (one launch: chunks, merges, o GEMV +
    # residual), gate|up (RMSNorm + Q8_0 prologue reading the x the
    # attention launch just wrote, SwiGLU, Q8_0 of h) and down (+ residual,
    # reading h's codes) back to back on the stream with no host wait
    # between them, at cfg5's shapes and position: each kernel reads what
    # the one before it wrote, as in the whole model, and every x and h is
    # checked against the oracle's layer arithmetic.
    hd, heads, kvh, d, ff, pos, ready = 128, 32, 8, 4096, 14336, 4096, 16
    k, cap = heads * hd, pos + 200
    chunks = (cap + 127) // 128
    layers = 2
    rng = np.random.default_rng(77)
    x0 = rng.standard_normal(d).astype(np.float32)
    x = dev(x0)
    fbytes = H.lib().vkml_attend_fused_sync_bytes(layers)
    fsync = H.empty(fbytes)
    H.call("vkml_fill_u32", p(fsync), 0, fbytes // 4)
    part, stats, st = H.empty(heads * chunks * hd * 4), H.empty(heads * chunks * 8), H.empty(16)
    H.call("vkml_state_set", p(st), 0, pos, 0)
    attn, avals, ascs = H.empty(k * 4), H.empty(k), H.empty(k // 32 * 4)
    h, hv, hsc = H.empty(ff * 4), H.empty(ff), H.empty(ff // 32 * 4)
    # every input on the device first: the launches then follow one another
    # on the stream with nothing between them
    L = []
    for layer in range(layers):
        prior = rng.standard_normal((2, kvh, cap, hd)).astype(np.float32)
        caches = [prior[i].astype(np.float16).view(np.uint16) for i in range(2)]
        q = rng.standard_normal((heads, hd)).astype(np.float32)
        qkv = np.concatenate([q.ravel(), rng.standard_normal(2 * kvh * hd).astype(np.float32)])
        nw = rng.standard_normal(d).astype(np.float32)
        L.append(dict(caches=caches, q=q, dqkv=dev(qkv), dk=dev(caches[0]), dv=dev(caches[1]), nw=nw, dnw=dev(nw),
                      o=weights(H.Q4_K, d, k, 100 + 4 * layer), g=weights(H.Q4_K, ff, d, 101 + 4 * layer),
                      u=weights(H.Q4_K, ff, d, 102 + 4 * layer), dn=weights(H.Q4_K, d, ff, 103 + 4 * layer)))
    prm = H.AttendStepParams(heads, kvh, hd, cap, 0, 0, H.F16, chunks, 0, 1, 1.0 / math.sqrt(hd), 0.0, 0, 1, ready)
    H.synchronize()
    for layer, w in enumerate(L):
        H.call("vkml_attend_step_fused", prm, p(w["dqkv"]), None, p(w["dk"]), p(w["dv"]), p(part), p(stats), p(attn), p(avals),
               p(ascs), p(st), H.GemvDotParams(1, d, k, H.Q4_K, H.F16), p(w["o"][0]), p(w["o"][1]), p(x), p(fsync), layer, layers)
        H.call("vkml_gemv_fused", H.GemvFusedParams(ff, d, H.Q4_K, H.F16, 2, 1, 1e-5, 1), p(x), None, p(w["dnw"]), p(w["g"][0]),
               p(w["g"][1]), p(w["u"][0]), p(w["u"][1]), None, p(h), p(hv), p(hsc))
        H.call("vkml_gemv_dot_add", H.GemvDotParams(1, d, ff, H.Q4_K, H.F16), p(hv), p(w["dn"][0]), p(x), p(w["dn"][1]), p(hsc),
               p(x))
    # the oracle's layers: attention, o + residual, ffn norm, SwiGLU, down + residual
    want_x, want_h = x0.copy(), None
    for w in L:
        a = O.attend_decode(w["q"], w["caches"][0], w["caches"][1], 0, pos + 1)
        aw, asw = O.quantize(O.Q8_0, a.reshape(1, k), False)
        _, _, oq, ow, osc = w["o"]
        want_x = want_x + O.gemv_dot(oq, aw, asw, 1, ow, osc, d, k)[0]
        nq, ns = O.quantize(O.Q8_0, O.rms_norm(want_x.reshape(1, d), w["nw"], 1e-5), False)
        _, _, gq, gw, gsc = w["g"]
        _, _, _, uw, usc = w["u"]
        want_h = O.silu(O.gemv_dot(gq, nq, ns, 1, gw, gsc, ff, d)[0]) * O.gemv_dot(gq, nq, ns, 1, uw, usc, ff, d)[0]
        hq, hs = O.quantize(O.Q8_0, want_h.reshape(1, ff), False)
        _, _, dq, dw, dsc = w["dn"]
        want_x = want_x + O.gemv_dot(dq, hq, hs, 1, dw, dsc, d, ff)[0]
    H.call("vkml_attend_fused_check", p(fsync), layers)
    assert np.array_equal(bits(h.download(np.float32, ff)), bits(want_h))
    assert np.array_equal(bits(x.download(np.float32, d)), bits(want_x))


@pytest.mark.parametrize("pos,ready,kv_type", [(4096, 16, H.F16), (300, 2, H.F32), (100, 8, H.F16), (1000, 4, H.F16)])
def test_attend_step_fused_prepared_bit_exact(pos, ready, kv_type):
    # a prepared step (q already rotated, the new key and value already in
    # the caches, as vkml_gemv_rope leaves them) whose first `ready` chunks
    # load before reading the position; the hint may name chunks past the
    # live keys (position 100 with 8), whose rows are then masked out
    hd, heads, kvh, n = 128, 32, 8, 4096
    k, cap = heads * hd, pos + 200
    chunks = (cap + 127) // 128
    rng = np.random.default_rng(pos + ready)
    dt = np.uint16 if kv_type == H.F16 else np.float32
    prior = rng.standard_normal((2, kvh, cap, hd)).astype(np.float32)
    caches = [prior[i].astype(np.float16).view(np.uint16) if kv_type == H.F16 else prior[i] for i in range(2)]
    kc, vc = dev(caches[0]), dev(caches[1])
    v, s_, quant, words, scales = weights(H.Q4_K, n, k, pos + 7)
    x0 = rng.standard_normal(n).astype(np.float32)
    x = dev(x0)
    fbytes = H.lib().vkml_attend_fused_sync_bytes(2)
    fsync = H.empty(fbytes)
    H.call("vkml_fill_u32", p(fsync), 0, fbytes // 4)
    part, stats, st = H.empty(heads * chunks * hd * 4), H.empty(heads * chunks * 8), H.empty(16)
    H.call("vkml_state_set", p(st), 0, pos, 0)
    q = rng.standard_normal((heads, hd)).astype(np.float32)
    qkv = np.concatenate([q.ravel(), rng.standard_normal(2 * kvh * hd).astype(np.float32)])
    out, vals, scs = H.empty(k * 4), H.empty(k), H.empty(k // 32 * 4)
    prm = H.AttendStepParams(heads, kvh, hd, cap, 0, 0, kv_type, chunks, 0, 1, 1.0 / math.sqrt(hd), 0.0, 0, 1, ready)
    H.call("vkml_attend_step_fused", prm, p(dev(qkv)), None, p(kc), p(vc), p(part), p(stats), p(out), p(vals), p(scs), p(st),
           H.GemvDotParams(1, n, k, H.Q4_K, H.F16), p(v), p(s_), p(x), p(fsync), 0, 2)
    H.call("vkml_attend_fused_check", p(fsync), 2)
    want = O.attend_decode(q, caches[0], caches[1], 0, pos + 1)
    assert np.array_equal(bits(out.download(np.float32, (heads, hd))), bits(want))
    ww, ws = O.quantize(O.Q8_0, want.reshape(1, k), False)
    assert np.array_equal(bits(x.download(np.float32, n)), bits(x0 + O.gemv_dot(quant, ww, ws, 1, words, scales, n, k)[0]))
    # nothing was appended: the caches are as they were
    assert np.array_equal(kc.download(dt, caches[0].shape), caches[0])
    assert np.array_equal(vc.download(dt, caches[1].shape), caches[1])


def test_attend_step_fused_reports_a_position_past_its_chunks():
    # launched for 2 chunks (256 keys) at position 300: the step is flagged,
    # every workgroup still ends (the o GEMV's waits stop at the flag), and
    # the check clears the blocks for the next call
    heads, kvh, hd, cap, n = 8, 4, 128, 512, 1024
    rng = np.random.default_rng(3)
    kc = dev(rng.standard_normal((kvh, cap, hd)).astype(np.float16).view(np.uint16))
    vc = dev(rng.standard_normal((kvh, cap, hd)).astype(np.float16).view(np.uint16))
    dtab = dev(O.rope_table(cap, hd, 1e6))
    v, s_, _, _, _ = weights(H.Q4_K, n, heads * hd, 9)
    x = dev(rng.standard_normal(n).astype(np.float32))
    fbytes = H.lib().vkml_attend_fused_sync_bytes(2)
    fsync = H.empty(fbytes)
    H.call("vkml_fill_u32", p(fsync), 0, fbytes // 4)
    part, stats = H.empty(heads * 4 * hd * 4), H.empty(heads * 4 * 8)
    out, vals, scs = H.empty(heads * hd * 4), H.empty(heads * hd), H.empty(heads * hd // 32 * 4)
    st = H.empty(16)
    op = H.GemvDotParams(1, n, heads * hd, H.Q4_K, H.F16)
    dq = dev(rng.standard_normal((heads + 2 * kvh) * hd).astype(np.float32))
    for i, (chunks, pos, ok) in enumerate(((2, 300, False), (3, 300, True), (2, 255, True))):
        print(f"fused chunks={chunks} pos={pos}", flush=True)
        H.call("vkml_state_set", p(st), 0, pos, 0)
        prm = H.AttendStepParams(heads, kvh, hd, cap, 0, 0, H.F16, chunks, 0, 1, 1.0 / math.sqrt(hd), 0.0, 0)
        H.call("vkml_attend_step_fused", prm, p(dq), p(dtab), p(kc), p(vc), p(part), p(stats), p(out), p(vals), p(scs), p(st), op,
               p(v), p(s_), p(x), p(fsync), i % 2, 2)
        if ok:
            H.call("vkml_attend_fused_check", p(fsync), 2)
        else:
            with pytest.raises(H.VkmlError, match="past the keys of the launched chunks"):
                H.call("vkml_attend_fused_check", p(fsync), 2)


def test_attend_step_fused_long_steps_take_separate_launches():
    # past 64 chunks a step runs the chunk pass, the spread merge and the o
    # GEMV apart, bit for bit the one launch's results; a launch sized below
    # the cache (128 chunks of a 134-chunk cache) serves positions up to its
    # chunks and flags one past them, as the one launch does
    hd, heads, kvh, n = 128, 32, 8, 4096
    k, cap, chunks = heads * hd, 17100, 128
    rng = np.random.default_rng(21)
    prior = rng.standard_normal((2, kvh, cap, hd)).astype(np.float32)
    caches = [prior[i].astype(np.float16).view(np.uint16) for i in range(2)]
    kc, vc = dev(caches[0]), dev(caches[1])
    table = O.rope_table(cap, hd, 1e6)
    dtab = dev(table)
    v, s_, quant, words, scales = weights(H.Q4_K, n, k, 23)
    x0 = rng.standard_normal(n).astype(np.float32)
    x = dev(x0)
    fbytes = H.lib().vkml_attend_fused_sync_bytes(2)
    fsync = H.empty(fbytes)
    H.call("vkml_fill_u32", p(fsync), 0, fbytes // 4)
    part, stats, st = H.empty(heads * chunks * hd * 4), H.empty(heads * chunks * 8), H.empty(16)
    op = H.GemvDotParams(1, n, k, H.Q4_K, H.F16)
    want_x = x0.copy()
    for step, p_now in enumerate((12000, 16383)):
        print(f"long fused step pos={p_now} chunks={chunks}", flush=True)
        H.call("vkml_state_set", p(st), 0, p_now, 0)
        qkv = rng.standard_normal((heads + 2 * kvh) * hd).astype(np.float32)
        out, vals, scs = H.empty(k * 4), H.empty(k), H.empty(k // 32 * 4)
        prm = H.AttendStepParams(heads, kvh, hd, cap, 0, 0, H.F16, chunks, 0, 1, 1.0 / math.sqrt(hd), 0.0, 0)
        H.call("vkml_attend_step_fused", prm, p(dev(qkv)), p(dtab), p(kc), p(vc), p(part), p(stats), p(out), p(vals), p(scs),
               p(st), op, p(v), p(s_), p(x), p(fsync), step % 2, 2)
        H.call("vkml_attend_fused_check", p(fsync), 2)
        q = O.rope(qkv[:k].reshape(1, heads, hd), table, p_now, 0).reshape(heads, hd)
        kn = O.rope(qkv[k:k + kvh * hd].reshape(1, kvh, hd), table, p_now, 0).reshape(kvh, hd)
        caches[0][:, p_now] = O.f32_to_f16(kn)
        caches[1][:, p_now] = O.f32_to_f16(qkv[k + kvh * hd:].reshape(kvh, hd))
        want = O.attend_decode(q, caches[0], caches[1], 0, p_now + 1)
        assert np.array_equal(bits(out.download(np.float32, (heads, hd))), bits(want))
        ww, ws = O.quantize(O.Q8_0, want.reshape(1, k), False)
        assert np.array_equal(vals.download(np.uint32, ww.shape), ww)
        want_x = want_x + O.gemv_dot(quant, ww, ws, 1, words, scales, n, k)[0]
        assert np.array_equal(bits(x.download(np.float32, n)), bits(want_x))
    H.call("vkml_state_set", p(st), 0, 16384, 0)
    prm = H.AttendStepParams(heads, kvh, hd, cap, 0, 0, H.F16, chunks, 0, 1, 1.0 / math.sqrt(hd), 0.0, 0)
    H.call("vkml_attend_step_fused", prm, p(dev(rng.standard_normal((heads + 2 * kvh) * hd).astype(np.float32))), p(dtab), p(kc),
           p(vc), p(part), p(stats), p(out), p(vals), p(scs), p(st), op, p(v), p(s_), p(x), p(fsync), 0, 2)
    with pytest.raises(H.VkmlError, match="past the keys of the launched chunks"):
        H.call("vkml_attend_fused_check", p(fsync), 2)


def test_attend_step_fused_rejects_bad_blocks():
    prm = H.AttendStepParams(8, 8, 64, 64, 0, 0, H.F16, 1, 0, 1, 0.125, 0.0, 0)
    op = H.GemvDotParams(1, 256, 512, H.Q4_K, H.F16)
    b = H.empty(1 << 16)
    for block, blocks in ((0, 1), (2, 2)):
        with pytest.raises(H.VkmlError, match="two blocks at least"):
            H.call("vkml_attend_step_fused", prm, p(b), p(b), p(b), p(b), p(b), p(b), p(b), p(b), p(b), p(b), op, p(b), p(b), p(b),
                   p(b), block, blocks)


@pytest.mark.parametrize("fmt,f16", [(H.Q8_0, True), (H.Q8_0, False), (H.Q4_0, True), (H.Q4_1, True), (H.Q4_K, True)])
@pytest.mark.parametrize("k", [96, 4128, 33280])
@pytest.mark.parametrize("m", [1, 3, 12])
def test_int8_gemv_takes_every_k_the_reference_does(fmt, f16, k, m):
    # k a multiple of 32 but not of 64 (an odd last block), and k past the
    # LDS-staged bound (the rows kernel): gemv_dot (m <= 8), matmul_dot
    # (m > 8) and, for one row, gemv_dot_add, bit for bit with the oracle
    if fmt == H.Q4_K and k % 256:
        pytest.skip("q4_K rows are whole 256-value super-blocks")
    n = 72
    v, s_, quant, words, scales = weights(fmt, n, k, k + m, f16_scales=f16)
    a, aw, asc = activation(k, k + 7, m)
    want = (O.gemv_dot if m <= 8 else O.matmul_dot)(quant, aw, asc, m, words, scales, n, k)
    out = H.empty(m * n * 4)
    prm = H.GemvDotParams(m, n, k, fmt, H.F16 if f16 else H.F32)
    call = "vkml_gemv_dot" if m <= 8 else "vkml_matmul_dot"
    H.call(call, prm, p(dev(aw)), p(v), p(out), p(s_), p(dev(asc)))
    assert np.array_equal(bits(out.download(np.float32, (m, n))), bits(want))
    if m == 1:
        res = np.random.default_rng(k).standard_normal(n).astype(np.float32)
        x = dev(res)
        H.call("vkml_gemv_dot_add", prm, p(dev(aw)), p(v), p(x), p(s_), p(dev(asc)), p(x))
        assert np.array_equal(bits(x.download(np.float32, n)), bits(res + want[0]))


# ---------------------------------------------------------------- small ops

def test_argmax_and_step_finish():
    x = np.random.default_rng(11).standard_normal((3, 32768)).astype(np.float32) * 3
    x[0, 5] = x[0, 900] = 100.0
    x[1, :] = np.nan
    x[2, 7] = np.inf
    x[2, 9] = np.nan
    out = H.empty(12)
    H.call("vkml_argmax", 3, 32768, p(dev(x)), p(out))
    assert list(out.download(np.int32, 3)) == [O.argmax(r) for r in x] == [5, 0, 7]
    st, log = H.empty(16), H.empty(64)
    H.call("vkml_state_set", p(st), 1, 10, 0)
    H.call("vkml_step_finish", 32768, p(dev(x[0])), p(st), p(log), 16)
    H.call("vkml_step_finish", 0, None, p(st), p(log), 16)
    assert list(st.download(np.int32, 4)[:3]) == [5, 12, 1]
    assert log.download(np.int32, 1)[0] == 5


@pytest.mark.parametrize("tt", [H.F32, H.F16, H.BF16, H.Q8_0, H.Q4_0, H.Q4_1, H.Q4_K])
def test_embedding_bit_exact(tt):
    vocab, dim = 300, 512
    ids = np.array([0, 299, 5, -1, 300, 17], np.int32)
    if tt in (H.F32, H.F16, H.BF16):
        t = np.random.default_rng(4).standard_normal((vocab, dim)).astype(np.float32)
        if tt == H.F16:
            vals = t.astype(np.float16).view(np.uint16); table = vals.view(np.float16).astype(np.float32)
        elif tt == H.BF16:
            vals = (t.view(np.uint32) >> 16).astype(np.uint16); table = (vals.astype(np.uint32) << 16).view(np.float32)
        else:
            vals = table = t
        want = np.array([table[i] if 0 <= i < vocab else np.zeros(dim, np.float32) for i in ids])
        dv, ds = dev(vals), None
    else:
        dv, ds, quant, words, halves = weights(tt, vocab, dim, 12)
        want = O.embedding_quantized(quant, words, halves, vocab, dim, ids)
    out = H.empty(ids.size * dim * 4)
    H.call("vkml_embedding", H.EmbeddingParams(ids.size * dim, dim, vocab, tt, H.F16), p(dv), p(ds), p(dev(ids)), p(out))
    assert np.array_equal(out.download(np.float32, want.shape).view(np.uint32), want.view(np.uint32))


def test_cast_copy_permute_elementwise():
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.standard_normal(1000).astype(np.float32) * 1e3,
                        np.array([65520.0, 65519.0, 2.0 ** -25, 3 * 2.0 ** -26, np.nan, -np.inf, 1e-40], np.float32)])
    out = H.empty(x.size * 4)
    H.call("vkml_cast", x.size, H.F32, H.F16, p(dev(x)), p(out))
    assert np.array_equal(out.download(np.uint16, x.size), O.f32_to_f16(x))
    h = O.f32_to_f16(x)
    H.call("vkml_cast", x.size, H.F16, H.F32, p(dev(h)), p(out))
    back = out.download(np.float32, x.size)
    ref = O.f16_to_f32(h)
    assert np.array_equal(np.isnan(back), np.isnan(ref)) and np.array_equal(back[~np.isnan(ref)], ref[~np.isnan(ref)])
    # write_rows: rows 3..5 of a [2, 4, 6] word tensor into rows 1..3 of [2, 8, 6]
    src = np.arange(2 * 4 * 6, dtype=np.uint32)
    dst = np.zeros(2 * 8 * 6, np.uint32)
    d = dev(dst)
    H.call("vkml_copy_rows", H.CopyRowsParams(2 * 3 * 6, 3 * 6, 4 * 6, 1 * 6, 8 * 6, 1 * 6), p(dev(src)), p(d))
    want = dst.reshape(2, 8, 6).copy()
    want[:, 1:4] = src.reshape(2, 4, 6)[:, 1:4]
    assert np.array_equal(d.download(np.uint32, want.shape), want)
    # permute [2,3,4] -> dims (2, 0, 1)
    t = np.arange(24, dtype=np.float32).reshape(2, 3, 4)
    prm = H.PermuteParams(3, 24, (H.u32 * 6)(2, 3, 4, 1, 1, 1), (H.u32 * 6)(2, 0, 1, 0, 0, 0))
    H.call("vkml_permute", prm, p(dev(t)), p(out))
    assert np.array_equal(out.download(np.float32, (4, 2, 3)), t.transpose(2, 0, 1))
    a = rng.standard_normal(1000).astype(np.float32)
    b = rng.standard_normal(10).astype(np.float32)
    for op, f in enumerate([np.add, np.subtract, np.multiply, np.divide]):
        H.call("vkml_binary", op, 1000, 10, p(dev(a)), p(dev(b)), p(out))
        assert np.array_equal(out.download(np.float32, 1000), f(a, np.tile(b, 100)).astype(np.float32))
    H.call("vkml_unary", 0, 1000, 0.0, p(dev(a * 30)), p(out))
    assert np.array_equal(bits(out.download(np.float32, 1000)), bits(O.silu(a * 30)))


def test_softmax_and_matmul():
    rng = np.random.default_rng(6)
    x = rng.standard_normal((8, 37)).astype(np.float32)
    out = H.empty(x.nbytes)
    H.call("vkml_softmax", H.SoftmaxParams(8, 37, 0.5, 1, 4, 33, 0, 0.0), p(dev(x)), p(out))
    got = out.download(np.float32, x.shape)
    for r in range(8):
        vis = min(37, r % 4 + 33 + 1)
        e = np.exp(x[r, :vis].astype(np.float64) * 0.5 - (x[r, :vis] * 0.5).max())
        want = np.zeros(37)
        want[:vis] = e / e.sum()
        assert np.allclose(got[r], want, atol=1e-6)
    a = rng.standard_normal((4, 3, 20)).astype(np.float32)
    b = rng.standard_normal((2, 5, 20)).astype(np.float32)  # [2 kv batches, n=5, k=20], transposed, group 2
    out = H.empty(4 * 3 * 5 * 4)
    H.call("vkml_matmul", H.MatmulParams(3, 5, 20, 100, 2, 4, 1, H.F32), p(dev(a)), p(dev(b)), p(out), None)
    want = np.stack([a[z] @ b[z // 2].T for z in range(4)])
    assert np.allclose(out.download(np.float32, want.shape), want, atol=1e-5)


@pytest.mark.parametrize("window,softcap", [(0, 0.0), (300, 0.0), (0, 20.0), (300, 20.0)])
@pytest.mark.parametrize("offset", [900, 1500, 3500])
def test_softmax_register_rows_match_long_rows(window, softcap, offset):
    """Rows of up to 1024, 2048 and 4096 columns take the kernel that holds a
    row in registers (4, 8 or 16 values a thread); longer rows take the one
    that rereads it. Causal rows that see up to offset + 64 keys (past 1024
    and 2048 with the larger offsets, so every register slot holds data) must
    come out bit-identical from every kernel whose width holds them."""
    rng = np.random.default_rng(61)
    rows, q_len = 192, 64
    seen = offset + q_len
    x = (rng.standard_normal((rows, 5000)) * 3).astype(np.float32)
    results = []
    for cols in [c for c in (1024, 2048, 4096) if c >= seen] + [5000]:
        xc = np.ascontiguousarray(x[:, :cols])
        out = H.empty(xc.nbytes)
        H.call("vkml_softmax", H.SoftmaxParams(rows, cols, 0.7, 1, q_len, offset, window, softcap), p(dev(xc)), p(out))
        got = out.download(np.float32, xc.shape)
        assert not got[:, seen:].any()
        results.append(got[:, :seen])
    assert len(results) >= 2
    for got in results[:-1]:
        assert np.array_equal(bits(got), bits(results[-1]))
    for r in (0, 63, 100):
        vis = r % q_len + offset + 1
        lo = vis - window if window and vis > window else 0
        sc = x[r, lo:vis].astype(np.float64) * 0.7
        if softcap:
            sc = softcap * np.tanh(np.clip(sc / softcap, -10, 10))
        e = np.exp(sc - sc.max())
        want = np.zeros(seen)
        want[lo:vis] = e / e.sum()
        assert np.allclose(results[0][r], want, atol=1e-6)


def _float_b(bt, n, k, rng):
    """(device values, device scales, oracle type, oracle values, oracle scales) of a float or quantized [n, k]."""
    if bt in (H.F32, H.F16, H.BF16):
        w = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
        if bt == H.F32:
            b, ot = w, O.T_F32
        elif bt == H.F16:
            b, ot = w.astype(np.float16).view(np.uint16), O.T_F16
        else:
            b, ot = (w.view(np.uint32) >> 16).astype(np.uint16), O.T_BF16
        return dev(b), None, ot, b, None
    dv, ds, quant, words, scales = weights(bt, n, k, int(rng.integers(1 << 30)))
    # q4_K runs as the reference's q4_1 repack, which the oracle holds
    return dv, ds, {O.Q8_0: O.T_Q8, O.Q4_0: O.T_Q4, O.Q4_1: O.T_Q4_1}[quant], words, scales


@pytest.mark.parametrize("bt", [H.F32, H.F16, H.BF16, H.Q8_0, H.Q4_0, H.Q4_1, H.Q4_K])
@pytest.mark.parametrize("m,n,k", [(9, 100, 512), (70, 64, 256), (130, 193, 768)])
def test_matmul_projection_bit_exact(bt, m, n, k):
    """vkml_matmul with a transposed weight (the float path's projections of
    more than 8 rows): each output in matmul.comp's k order, as the oracle."""
    rng = np.random.default_rng(m + n + bt)
    a = rng.standard_normal((m, k)).astype(np.float32)
    dv, ds, ot, ob, osc = _float_b(bt, n, k, rng)
    out = H.empty(m * n * 4)
    H.call("vkml_matmul", H.MatmulParams(m, n, k, 0, 1, 1, 1, bt, H.F16), p(dev(a)), p(dv), p(out), p(ds))
    want = O.matmul_float(ot, a, ob, osc, n, k)
    assert np.array_equal(bits(out.download(np.float32, (m, n))), bits(want))


@pytest.mark.parametrize("kv_type", [H.F16, H.F32])
@pytest.mark.parametrize("rows,keys", [(9, 40), (64, 64), (130, 300), (200, 129)])
def test_matmul_attention_shapes_bit_exact(kv_type, rows, keys):
    """Scores q k^T and probs v as attention_block runs them: a batch per
    query head against its KV head's cache rows (b_group, b_stride), the
    first `keys` rows of a larger cache; k order per output."""
    heads, kvh, hd, cap = 8, 2, 64, keys + 7
    g = heads // kvh
    rng = np.random.default_rng(rows * keys)
    q = rng.standard_normal((heads, rows, hd)).astype(np.float32)
    dt = np.float16 if kv_type == H.F16 else np.float32
    kc = rng.standard_normal((kvh, cap, hd)).astype(dt)
    vc = rng.standard_normal((kvh, cap, hd)).astype(dt)
    ot = O.T_F16 if kv_type == H.F16 else O.T_F32
    kb = kc.view(np.uint16) if kv_type == H.F16 else kc
    vb = vc.view(np.uint16) if kv_type == H.F16 else vc
    scores = H.empty(heads * rows * keys * 4)
    H.call("vkml_matmul", H.MatmulParams(rows, keys, hd, cap * hd, g, heads, 1, kv_type, H.F16), p(dev(q)), p(dev(kb)),
           p(scores), None)
    got = scores.download(np.float32, (heads, rows, keys))
    for h in range(heads):
        want = O.matmul_float(ot, q[h], np.ascontiguousarray(kb[h // g, :keys]), None, keys, hd)
        assert np.array_equal(bits(got[h]), bits(want)), h
    probs = rng.random((heads, rows, keys)).astype(np.float32)
    out = H.empty(heads * rows * hd * 4)
    H.call("vkml_matmul", H.MatmulParams(rows, hd, keys, cap * hd, g, heads, 0, kv_type, H.F16), p(dev(probs)), p(dev(vb)),
           p(out), None)
    got = out.download(np.float32, (heads, rows, hd))
    for h in range(heads):
        # b [k, n] in k order equals b^T [n, k] in k order
        want = O.matmul_float(ot, probs[h], np.ascontiguousarray(vb[h // g, :keys].T), None, hd, keys)
        assert np.array_equal(bits(got[h]), bits(want)), h


@pytest.mark.parametrize("bt", [H.F32, H.F16])
def test_matmul_vec4_and_scalar_loads_agree(bt):
    """The same product with a's rows whole aligned vec4s (the vec4 tile
    loads) and with a 4 bytes off alignment (scalar loads): bit-identical,
    and both the oracle's k order, for scores (b transposed) and probs . v."""
    heads, kvh, hd, rows, keys = 4, 2, 64, 70, 132
    cap, g = keys + 4, 2
    rng = np.random.default_rng(bt + 91)
    dt = np.float16 if bt == H.F16 else np.float32
    ot = O.T_F16 if bt == H.F16 else O.T_F32
    kc = rng.standard_normal((kvh, cap, hd)).astype(dt)
    kb = kc.view(np.uint16) if bt == H.F16 else kc
    for transposed, m, n, k in ((1, rows, keys, hd), (0, rows, hd, keys)):
        a = rng.standard_normal((heads, m, k)).astype(np.float32)
        shifted = dev(np.concatenate([np.zeros(1, np.float32), a.ravel()]))
        aligned = dev(a)
        outs = []
        for ptr in (p(aligned), C.c_void_p(p(shifted).value + 4)):
            out = H.empty(heads * m * n * 4)
            H.call("vkml_matmul", H.MatmulParams(m, n, k, cap * hd, g, heads, transposed, bt, H.F16), ptr, p(dev(kb)), p(out), None)
            outs.append(out.download(np.float32, (heads, m, n)))
        assert np.array_equal(bits(outs[0]), bits(outs[1]))
        for h in range(heads):
            b = kb[h // g, :n] if transposed else kb[h // g, :k].T
            want = O.matmul_float(ot, a[h], np.ascontiguousarray(b), None, n, k)
            assert np.array_equal(bits(outs[0][h]), bits(want)), h


@pytest.mark.parametrize("rows,first", [(130, 0), (64, 70), (200, 3)])
def test_matmul_causal_skip_changes_nothing(rows, first):
    """The causal skip: scores on and below the diagonal (row r sees keys
    0 .. first + r) as the full product's, and probs . v with the masked
    probabilities 0 identical to the full sum over every key."""
    heads, kvh, hd = 4, 2, 64
    keys, cap, g = first + rows, first + rows + 5, 2
    rng = np.random.default_rng(rows + first)
    q = rng.standard_normal((heads, rows, hd)).astype(np.float32)
    kc = rng.standard_normal((kvh, cap, hd)).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal((kvh, cap, hd)).astype(np.float16).view(np.uint16)
    full, skip = H.empty(heads * rows * keys * 4), H.empty(heads * rows * keys * 4)
    dq, dk = dev(q), dev(kc)
    H.call("vkml_matmul", H.MatmulParams(rows, keys, hd, cap * hd, g, heads, 1, H.F16, H.F16, 0, 0), p(dq), p(dk), p(full), None)
    H.call("vkml_matmul", H.MatmulParams(rows, keys, hd, cap * hd, g, heads, 1, H.F16, H.F16, 1, first), p(dq), p(dk), p(skip), None)
    a, b = full.download(np.float32, (heads, rows, keys)), skip.download(np.float32, (heads, rows, keys))
    seen = np.arange(keys)[None, :] <= np.arange(rows)[:, None] + first
    assert np.array_equal(bits(a[:, seen]), bits(b[:, seen]))
    probs = rng.random((heads, rows, keys)).astype(np.float32) * seen
    dp = dev(probs)
    o_full, o_skip = H.empty(heads * rows * hd * 4), H.empty(heads * rows * hd * 4)
    H.call("vkml_matmul", H.MatmulParams(rows, hd, keys, cap * hd, g, heads, 0, H.F16, H.F16, 0, 0), p(dp), p(dev(vc)), p(o_full), None)
    H.call("vkml_matmul", H.MatmulParams(rows, hd, keys, cap * hd, g, heads, 0, H.F16, H.F16, 1, first), p(dp), p(dev(vc)), p(o_skip), None)
    assert np.array_equal(bits(o_full.download(np.float32, (heads, rows, hd))), bits(o_skip.download(np.float32, (heads, rows, hd))))


@pytest.mark.parametrize("rows", [1, 5, 8])
def test_gemv_batched_scores_bit_exact(rows):
    """Up to 8 queries' scores through gemv.comp's order, one batch per
    query head against its KV head (gemv's z, b_group, b_stride)."""
    heads, kvh, hd, keys, cap = 8, 2, 128, 77, 90
    g = heads // kvh
    rng = np.random.default_rng(rows)
    q = rng.standard_normal((heads, rows, hd)).astype(np.float32)
    kc = rng.standard_normal((kvh, cap, hd)).astype(np.float16).view(np.uint16)
    out = H.empty(heads * rows * keys * 4)
    H.call("vkml_gemv", H.GemvParams(rows, keys, hd, H.F16, H.F16, cap * hd, g, heads), p(dev(q)), p(dev(kc)), p(out), None)
    got = out.download(np.float32, (heads, rows, keys))
    for h in range(heads):
        want = O.gemv_float(O.T_F16, q[h], np.ascontiguousarray(kc[h // g, :keys]), None, keys, hd)
        assert np.array_equal(bits(got[h]), bits(want)), h


@pytest.mark.parametrize("kv_type", [H.F16, H.F32])
@pytest.mark.parametrize("style", [0, 1])
def test_rope_kv_prompt_bit_exact(kv_type, style):
    """A prompt's rope + heads-first q + KV append in one launch, as the
    reference's rope, permute, cast and write_rows (llama.cpp:320-355)."""
    heads, kvh, hd, cap, pos, t = 8, 2, 64, 40, 3, 13
    width = (heads + 2 * kvh) * hd
    stride = width + 32
    rng = np.random.default_rng(4 + style)
    rows = rng.standard_normal((t, stride)).astype(np.float32)
    table = O.rope_table(cap, hd, 1e4)
    dt = np.uint16 if kv_type == H.F16 else np.float32
    kc, vc = H.empty(kvh * cap * hd * 4), H.empty(kvh * cap * hd * 4)
    H.call("vkml_fill_u32", kc.p, 0, kvh * cap * hd)
    H.call("vkml_fill_u32", vc.p, 0, kvh * cap * hd)
    q = H.empty(heads * t * hd * 4)
    H.call("vkml_rope_kv_prompt", H.RopeKvParams(heads, kvh, hd, cap, pos, style, kv_type, 1), t, stride, p(dev(rows)),
           p(dev(table)), p(q), p(kc), p(vc))
    qr = O.rope(np.ascontiguousarray(rows[:, :heads * hd]).reshape(t, heads, hd), table, pos, style)
    kr = O.rope(np.ascontiguousarray(rows[:, heads * hd:(heads + kvh) * hd]).reshape(t, kvh, hd), table, pos, style)
    vr = rows[:, (heads + kvh) * hd:width].reshape(t, kvh, hd)
    assert np.array_equal(bits(q.download(np.float32, (heads, t, hd))), bits(qr.transpose(1, 0, 2)))
    kg = kc.download(dt, (kvh, cap, hd))
    vg = vc.download(dt, (kvh, cap, hd))
    cast = (lambda x: O.f32_to_f16(x)) if kv_type == H.F16 else (lambda x: x)
    assert np.array_equal(kg[:, pos:pos + t], cast(kr.transpose(1, 0, 2)))
    assert np.array_equal(vg[:, pos:pos + t], cast(vr.transpose(1, 0, 2)))
    assert not kg[:, :pos].any() and not kg[:, pos + t:].any()


def test_graph_replay_advances_the_state():
    st, log = H.empty(16), H.empty(64)
    logits = np.zeros(1000, np.float32)
    logits[123] = 1.0
    dl = dev(logits)
    H.call("vkml_state_set", p(st), 0, 0, 0)
    H.call("vkml_graph_begin")
    H.call("vkml_step_finish", 1000, p(dl), p(st), p(log), 16)
    g = H.u64()
    H.call("vkml_graph_end", H.C.byref(g))
    for _ in range(5):
        H.call("vkml_graph_launch", g.value)
    H.synchronize()
    assert list(st.download(np.int32, 4)[:3]) == [123, 5, 5]
    assert list(log.download(np.int32, 5)) == [123] * 5
    H.call("vkml_graph_destroy", g.value)
