"""The matrix-core form of decode attention (vkml_attend_fast,
vkml_attend_step_fast): the tolerance option beside the bit-exact kernels.

It does not keep the reference's order of f32 operations (attend.comp:97-168,
attend_merge.comp:25-39), so its outputs are held to a bound against
float64 attention instead of the oracle's bits. The bound: scores are
q.k with q split in two f16 terms (relative error 2^-22 of |q| per element)
against f16 keys, summed in f32, so a score is off by at most about
2^-21 * sum_d |q_d k_d| (scale included); softmax weights carry that
error as a relative one (times 1 + |s|), and the weights are split in two
f16 terms against f16 values (2^-22), accumulated in f32 over at most a few
thousand terms. With K, V ~ N(0, 1) and hd <= 128 this stays below
TOL * max|v| with TOL = 2e-5 on every shape here (the exact kernels'
results sit about 1e-7 from float64 on the same inputs).

The Q8_0 codes and scales the merge publishes must be the quantizer's
(quantize.comp:102-114) bit for bit on the kernel's own f32 output, and the
one-launch step's o projection + residual must equal vkml_gemv_dot_add on
that output bit for bit.
"""
import math

import numpy as np
import pytest

import oracle as O
from vkml_amd import hip as H
from vkml_amd import synth

pytestmark = pytest.mark.gpu

TOL = 2e-5


def attention_f64(q, kc, vc, kv_start, kv_len, group, softcap=0.0):
    """float64 softmax(q k^T / sqrt(hd)) v over keys kv_start .. kv_len - 1."""
    heads, hd = q.shape
    k = kc.view(np.float16).astype(np.float64)
    v = vc.view(np.float16).astype(np.float64)
    out = np.empty((heads, hd))
    for h in range(heads):
        kvh = h // group
        s = k[kvh, kv_start:kv_len] @ q[h].astype(np.float64) / math.sqrt(hd)
        if softcap:
            s = softcap * np.tanh(np.clip(s / softcap, -10.0, 10.0))
        p = np.exp(s - s.max())
        out[h] = p @ v[kvh, kv_start:kv_len] / p.sum()
    return out


def within(got, want, vmax, what):
    err = np.max(np.abs(got.astype(np.float64) - want))
    assert err <= TOL * vmax, f"{what}: max |err| {err:.3g} above {TOL * vmax:.3g}"
    return err


SHAPES = [
    # (heads, kv_heads, hd, kv_start, kv_len, capacity)
    (4, 4, 64, 0, 1, 64),
    (8, 2, 64, 0, 5, 64),
    (32, 8, 128, 0, 127, 200),
    (32, 8, 128, 0, 128, 128),
    (32, 8, 128, 3, 129, 300),
    (16, 2, 128, 0, 1000, 1024),
    (32, 8, 64, 0, 4097, 4100),
    (32, 4, 128, 0, 2048, 2048),
    (32, 32, 128, 7, 999, 1000),
    (24, 8, 64, 0, 333, 400),
    # past 64 chunks the merge takes two levels (segments of 32 chunks)
    (8, 2, 64, 5, 9000, 9100),
    # past two items a CU, runs of chunks an item, streamed (3, 4 and 9
    # chunks a run; the last run short, its last chunk partial)
    (32, 8, 128, 0, 20000, 20000),
    (32, 8, 128, 0, 32768, 32768),
    (16, 4, 64, 100, 70000, 70100),
]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("softcap", [0.0, 30.0])
def test_fast_attention_within_bound_of_f64(shape, softcap):
    H.init()
    heads, kvh, hd, start, kv_len, cap = shape
    group = heads // kvh
    rng = np.random.default_rng(1 + kv_len + hd)
    print(f"attend_fast shape {shape} softcap {softcap}", flush=True)
    q = rng.standard_normal((heads, hd)).astype(np.float32)
    kc = rng.standard_normal((kvh, cap, hd)).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal((kvh, cap, hd)).astype(np.float16).view(np.uint16)
    chunks = (kv_len - start + 127) // 128
    prm = H.AttendParams(start, kv_len, cap, heads, kvh, hd, H.F16, chunks, 1.0 / math.sqrt(hd), softcap)
    sync = H.empty(int(H.lib().vkml_attend_fused_sync_bytes(1)))
    H.call("vkml_fill_u32", sync.p, 0, sync.nbytes // 4)
    dq, dk, dv = H.to_device(q), H.to_device(kc), H.to_device(vc)
    part, stats = H.empty(heads * chunks * hd * 4), H.empty(heads * chunks * 8)
    out, vals, scs = H.empty(heads * hd * 4), H.empty(heads * hd), H.empty(heads * hd // 32 * 4)
    want = attention_f64(q, kc, vc, start, kv_len, group, softcap)
    vmax = np.abs(vc.view(np.float16)).max()
    for rep in range(2):  # the arrival counters reset themselves between calls
        H.call("vkml_fill_u32", out.p, 0x7FC00000, heads * hd)
        H.call("vkml_attend_fast", prm, dq.p, dk.p, dv.p, part.p, stats.p, out.p, vals.p, scs.p, sync.p, None)
        got = out.download(np.float32, (heads, hd))
        within(got, want, vmax, f"rep {rep}")
        ww, ws = O.quantize(O.Q8_0, got, False)
        assert np.array_equal(vals.download(np.uint32, ww.shape), ww)
        assert np.array_equal(scs.download(np.float32, ws.shape).view(np.uint32), ws.view(np.uint32))
    assert not sync.download(np.uint32, sync.nbytes // 4).any(), "counters left non-zero"
    H.synchronize()


def test_exact_kernel_is_within_the_same_bound():
    """The bound is not loose for the exact form either: the bit-exact
    kernels on one of the shapes above sit well inside it."""
    H.init()
    heads, kvh, hd, start, kv_len, cap = 32, 8, 128, 0, 1000, 1024
    rng = np.random.default_rng(7)
    q = rng.standard_normal((heads, hd)).astype(np.float32)
    kc = rng.standard_normal((kvh, cap, hd)).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal((kvh, cap, hd)).astype(np.float16).view(np.uint16)
    want = attention_f64(q, kc, vc, start, kv_len, heads // kvh)
    exact = O.attend_decode(q, kc, vc, start, kv_len)
    err = np.max(np.abs(exact - want))
    assert err <= TOL * np.abs(vc.view(np.float16)).max() / 10, err


@pytest.mark.parametrize("hd,positions,cap", [(128, [4096, 4100, 4223], 4352), (64, [511, 512, 700], 4352),
                                               (128, [32000, 32767, 20000], 32768)])
def test_fast_step_with_o_projection(hd, positions, cap):
    """vkml_attend_step_fast at the decode state's position (a prepared
    step: q rotated, the new row appended) with the q4_K o GEMV + residual
    in the same launch, over four calls cycling through the sync blocks and
    a chunk tier below the cache's; the o projection equals
    vkml_gemv_dot_add on the published Q8_0 output. Near 32K keys the
    items are runs of chunks."""
    H.init()
    heads, kvh = 32, 8
    n = heads * hd
    rng = np.random.default_rng(hd)
    kc = rng.standard_normal((kvh, cap, hd)).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal((kvh, cap, hd)).astype(np.float16).view(np.uint16)
    blocks = synth.q4_k_blocks(rng, n * heads * hd // 256).reshape(n, heads * hd // 256, 144)
    codes = np.ascontiguousarray(blocks[:, :, 16:]).reshape(n, heads * hd // 2)
    hdr = np.ascontiguousarray(blocks[:, :, :16])
    dk, dv, dcodes, dhdr = H.to_device(kc), H.to_device(vc), H.to_device(codes), H.to_device(hdr)
    nblk = 4
    sync = H.empty(int(H.lib().vkml_attend_fused_sync_bytes(nblk)))
    H.call("vkml_fill_u32", sync.p, 0, sync.nbytes // 4)
    state = H.empty(16)
    op = H.GemvDotParams(1, n, heads * hd, H.Q4_K, H.F16)
    for i, pos in enumerate(positions + [positions[0]]):
        tier = 8
        while tier * 128 < pos + 1:
            tier *= 2
        chunks = min(tier, (cap + 127) // 128)
        print(f"attend_step_fast hd {hd} position {pos} tier {tier} block {i % nblk}", flush=True)
        qkv = rng.standard_normal((heads + 2 * kvh) * hd).astype(np.float32)
        x0 = rng.standard_normal(n).astype(np.float32)
        dqkv, dx = H.to_device(qkv), H.to_device(x0)
        part, stats = H.empty(heads * chunks * hd * 4), H.empty(heads * chunks * 8)
        out, vals, scs = H.empty(heads * hd * 4), H.empty(heads * hd), H.empty(heads * hd // 32 * 4)
        H.call("vkml_state_set", state.p, 0, pos, 0)
        prm = H.AttendStepParams(heads, kvh, hd, cap, 0, pos, H.F16, chunks, 0, 1, 1.0 / math.sqrt(hd), 0.0, 0, 1,
                                 tier // 2 if tier > 8 else 0)
        assert H.lib().vkml_attend_step_fast_supported(prm, op) == 1
        H.call("vkml_attend_step_fast", prm, dqkv.p, dk.p, dv.p, part.p, stats.p, out.p, vals.p, scs.p, state.p, op,
               dcodes.p, dhdr.p, dx.p, sync.p, i % nblk, nblk)
        H.call("vkml_attend_fused_check", sync.p, nblk)
        got = out.download(np.float32, (heads, hd))
        want = attention_f64(qkv[:heads * hd].reshape(heads, hd), kc, vc, 0, pos + 1, heads // kvh)
        within(got, want, np.abs(vc.view(np.float16)).max(), f"position {pos}")
        ww, ws = O.quantize(O.Q8_0, got, False)
        assert np.array_equal(vals.download(np.uint32, ww.shape), ww)
        dx2, dww, dws = H.to_device(x0), H.to_device(ww), H.to_device(ws)
        H.call("vkml_gemv_dot_add", op, dww.p, dcodes.p, dx2.p, dhdr.p, dws.p, dx2.p)
        assert np.array_equal(dx.download(np.uint32, n), dx2.download(np.uint32, n)), f"o projection at {pos}"
    H.synchronize()


def test_fast_step_reports_a_position_past_its_chunks():
    """A launch sized for fewer chunks than the position needs sets the
    error flag that vkml_attend_fused_check reports (nothing faults)."""
    H.init()
    heads, kvh, hd, cap = 32, 8, 128, 2048
    n = heads * hd
    rng = np.random.default_rng(3)
    kc = np.zeros((kvh, cap, hd), np.uint16)
    vc = np.zeros((kvh, cap, hd), np.uint16)
    blocks = synth.q4_k_blocks(rng, n * n // 256).reshape(n, n // 256, 144)
    dcodes = H.to_device(np.ascontiguousarray(blocks[:, :, 16:]).reshape(n, n // 2))
    dhdr = H.to_device(np.ascontiguousarray(blocks[:, :, :16]))
    dk, dv = H.to_device(kc), H.to_device(vc)
    sync = H.empty(int(H.lib().vkml_attend_fused_sync_bytes(2)))
    H.call("vkml_fill_u32", sync.p, 0, sync.nbytes // 4)
    state = H.empty(16)
    H.call("vkml_state_set", state.p, 0, 1500, 0)
    dqkv = H.to_device(rng.standard_normal((heads + 2 * kvh) * hd).astype(np.float32))
    dx = H.to_device(np.zeros(n, np.float32))
    part, stats = H.empty(heads * 8 * hd * 4), H.empty(heads * 8 * 8)
    out, vals, scs = H.empty(n * 4), H.empty(n), H.empty(n // 32 * 4)
    prm = H.AttendStepParams(heads, kvh, hd, cap, 0, 0, H.F16, 8, 0, 1, 1.0 / math.sqrt(hd), 0.0, 0, 1, 0)
    op = H.GemvDotParams(1, n, n, H.Q4_K, H.F16)
    H.call("vkml_attend_step_fast", prm, dqkv.p, dk.p, dv.p, part.p, stats.p, out.p, vals.p, scs.p, state.p, op,
           dcodes.p, dhdr.p, dx.p, sync.p, 0, 2)
    with pytest.raises(H.VkmlError, match="past the keys"):
        H.call("vkml_attend_fused_check", sync.p, 2)
    H.synchronize()


def prompt_attention_f64(q, kc, vc, first, group, softcap=0.0):
    """float64 causal attention of a prompt: query i sees keys 0 .. first + i."""
    heads, t, hd = q.shape
    k = kc.view(np.float16).astype(np.float64)
    v = vc.view(np.float16).astype(np.float64)
    out = np.empty((t, heads, hd))
    keys = first + t
    mask = np.arange(keys)[None, :] > (first + np.arange(t))[:, None]
    for h in range(heads):
        s = q[h].astype(np.float64) @ k[h // group, :keys].T / math.sqrt(hd)
        if softcap:
            s = softcap * np.tanh(np.clip(s / softcap, -10.0, 10.0))
        s[mask] = -np.inf
        p = np.exp(s - s.max(axis=1, keepdims=True))
        out[:, h] = (p @ v[h // group, :keys]) / p.sum(axis=1, keepdims=True)
    return out


PROMPT_SHAPES = [
    # (heads, kv_heads, hd, first, t, capacity)
    (32, 8, 128, 0, 1, 64),
    (32, 8, 128, 0, 17, 64),
    (32, 8, 128, 0, 300, 512),
    (32, 8, 128, 100, 64, 200),
    (8, 2, 64, 0, 1000, 1024),
    (16, 2, 128, 5, 130, 200),
    (32, 8, 128, 0, 2048, 2048),
]


@pytest.mark.parametrize("shape", PROMPT_SHAPES)
@pytest.mark.parametrize("softcap", [0.0, 30.0])
def test_prompt_fast_attention_within_bound_of_f64(shape, softcap):
    """vkml_attend_prompt_fast against float64 causal attention, under the
    same bound as the decode form (every product exact, sums in f32)."""
    H.init()
    heads, kvh, hd, first, t, cap = shape
    print(f"attend_prompt_fast shape {shape} softcap {softcap}", flush=True)
    rng = np.random.default_rng(11 + t + first + hd)
    q = rng.standard_normal((heads, t, hd)).astype(np.float32)
    kc = rng.standard_normal((kvh, cap, hd)).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal((kvh, cap, hd)).astype(np.float16).view(np.uint16)
    prm = H.AttendPromptParams(heads, kvh, hd, cap, t, first, H.F16, 1.0 / math.sqrt(hd), softcap)
    assert H.lib().vkml_attend_prompt_fast_supported(prm) == 1
    dq, dk, dv, out = H.to_device(q), H.to_device(kc), H.to_device(vc), H.empty(t * heads * hd * 4)
    H.call("vkml_attend_prompt_fast", prm, dq.p, dk.p, dv.p, out.p)
    got = out.download(np.float32, (t, heads, hd))
    want = prompt_attention_f64(q, kc, vc, first, heads // kvh, softcap)
    err = within(got, want, np.abs(vc.view(np.float16)).max(), f"shape {shape}")
    print(f"max |err| {err:.3g}", flush=True)
    H.synchronize()


def test_prompt_fast_attention_rejects_what_it_does_not_take():
    H.init()
    for prm, msg in ((H.AttendPromptParams(32, 8, 128, 64, 65, 0, H.F16, 0.1, 0.0), "do not fit"),
                     (H.AttendPromptParams(32, 8, 128, 64, 8, 0, H.F32, 0.1, 0.0), "f16"),
                     (H.AttendPromptParams(12, 4, 128, 64, 8, 0, H.F16, 0.1, 0.0), "multiple of 4"),
                     (H.AttendPromptParams(32, 8, 256, 64, 8, 0, H.F16, 0.1, 0.0), "64 or 128")):
        assert H.lib().vkml_attend_prompt_fast_supported(prm) == 0
        b = H.empty(1 << 16)
        with pytest.raises(H.VkmlError, match=msg):
            H.call("vkml_attend_prompt_fast", prm, b.p, b.p, b.p, b.p)
