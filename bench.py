#!/usr/bin/env python3
"""Batch-1 decode benchmark of vkml-mi355x on one MI355X (BASELINE.json's
metric on its config 5): a Mistral-7B-shaped model (32 layers, hidden 4096,
32/8 heads, head_dim 128, FFN 14336, vocab 32768, q4_K weights and a q6_K
output matrix, seeded synthetic values), its f16 KV cache prefilled with
4096 random-token positions, then greedy decoding. A step is one decode
token; the timed steps replay the captured decode graph back to back with
the weights and cache resident in HBM, and the host reads the tokens once
at the end.

Prints one JSON line: tokens/s, the whole step's algorithmic HBM rate (GGUF
bytes of every weight plus the KV rows read) against 8 TB/s, a roofline
entry for the dominant kernel, and the CPU oracle's decode rate on the host
cores as a reported baseline.

"parity" holds the timed run against the oracle's own run of the same
model and prompt (tests/golden/headline_cfg5.npz, written by
tests/golden/make_headline_fixture.py: its 4096-token prompt pass and 256
greedy steps, nothing handed over from the GPU): the GPU's prompt logits
bit for bit, and every timed greedy id. The CPU baseline's oracle, which
continues from the GPU's KV cache, must also pick the timed run's first
tokens. "fast_attention" reports the same decode with the matrix-core
attention option, which is not the reference's order of f32 operations:
its rate, its attention launch, and how many of its ids equal the oracle's.

Under "configs" the line also carries BASELINE.json's other measured
configs: cfg2's isolated GEMVs and cfg4's decode attention (each launched
back to back over rotating distinct copies of at least 512 MB, so no cache
holds the operands; best and median per launch over the rotations), and
cfg3's decode rate with its 512-token prefill on the matrix cores.

The dominant kernel, the one taking the largest share of a step's time, is
the one attention launch a layer (k_attend_fused: the chunk pass over the
f16 caches, the merges, and the o GEMV + residual add). Its average launch
duration is measured here with two HIP events on the library's stream around
back-to-back launches at the step's exact shape, at the middle position of
the timed run, over 32 distinct KV caches and o matrices (873 MB, more than
any cache holds), the way the step goes from one layer to the next. The
fused gate/up GEMV, the kernel moving the most bytes (66 MB of q4_K weights
a layer, with the ffn RMSNorm and the activation's Q8_0 in its prologue and
SwiGLU and h's Q8_0 in its epilogue), gets a second entry measured the same
way over 32 distinct weight pairs (2.1 GB). A per-kernel table of extra
eager steps (HIP events around each launch, so with launch gaps) goes to
stderr.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "vkml-framework_amd", "python"))

import numpy as np  # noqa: E402

PEAK_HBM = 8000.0  # GB/s, MI355X HBM3E
PEAK_INT8_TOPS = 5000.0  # dense int8 MFMA, TOP/s
PROMPT = 4096

# HBM bytes one launch of each roofline kernel moves (reads + writes):
# FETCH_SIZE and WRITE_SIZE passes of rocprofv3 over `bench.py
# --roofline-only`, each scaled by the same counter's reading for a 256 MiB
# device copy; the readings and commands are in
# profiles/attend_step_cfg5_hbm_traffic.md and
# profiles/gate_up_cfg5_hbm_traffic.md. Each figure holds only for the
# kernel sources it was taken on: its hash is the SHA-256 (first 16 hex
# digits) of those files, and the line reports no traffic when they have
# changed since.
GATE_UP_TRAFFIC = 67_212_366
GATE_UP_TRAFFIC_SOURCES = "558e79baed80feb0"
TRAFFIC_FILES = ("vkml-framework_amd/csrc/gemv.hpp", "vkml-framework_amd/csrc/k_gemv.hip", "vkml-framework_amd/csrc/device.hpp")
ATTEND_TRAFFIC = 28_566_713
ATTEND_TRAFFIC_SOURCES = "4a8995ea2854df48"
ATTEND_TRAFFIC_POSITION = 4224  # the launch's shape the figure was taken at (position; 35 chunks, 32 loading early)
ATTEND_FILES = ("vkml-framework_amd/csrc/k_attend.hip", "vkml-framework_amd/csrc/attend.hpp", "vkml-framework_amd/csrc/gemv.hpp",
                "vkml-framework_amd/csrc/device.hpp")

# The oracle's own runs of the headline workloads (tests/golden/make_headline_fixture.py):
# its prompt logits and every greedy id, against which each timed run is checked.
GOLDEN = os.path.join(ROOT, "tests", "golden")

# The roofline entry's attention launch is timed at the configured cfg5
# workload's middle position (4096-token prompt, 256 steps), whatever --steps is.
ROOFLINE_STEPS = 256

# GGUF-native bytes per weight (q4_K 144 B / 256, q6_K 210 B / 256).
Q4K, Q6K = 144 / 256, 210 / 256


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def fixture(cfg):
    """The oracle's headline run for cfg ("cfg5", "cfg3"), or None if absent."""
    path = os.path.join(GOLDEN, f"headline_{cfg}.npz")
    return np.load(path) if os.path.exists(path) else None


def against_fixture(fx, prompt_logits, first, tokens):
    """The GPU run against the oracle's own: the prompt's logits bit for bit,
    the first greedy id and every timed id (as many as the fixture holds)."""
    if fx is None:
        return None
    ids = fx["ids"]
    n = min(len(tokens), len(ids) - 1)
    got = [int(t) for t in tokens[:n]]
    want = [int(t) for t in ids[1:n + 1]]
    differ = [i for i in range(n) if got[i] != want[i]]
    bits = bool(np.array_equal(np.asarray(prompt_logits, np.float32).view(np.uint32), fx["prompt_logits"].view(np.uint32)))
    return {"prompt_logits_bit_identical": bits, "first_id_equal": int(first) == int(ids[0]),
            "timed_ids_checked": n, "timed_ids_equal": n - len(differ), "first_difference": differ[0] if differ else None,
            "all_equal": bits and int(first) == int(ids[0]) and not differ and n == len(tokens)}


def sources_hash(files=TRAFFIC_FILES):
    import hashlib
    h = hashlib.sha256()
    for f in files:
        with open(os.path.join(ROOT, f), "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()[:16]


def host_cores():
    """(threads the CPU baseline uses, the host's logical CPUs): the box's
    share of its host is 16 threads for one GPU, whatever the host has."""
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    return min(16, avail), os.cpu_count() or avail


def algorithmic_bytes(spec):
    """Per-token bytes: every weight once (GGUF-native sizes), the embedding
    row, and per-position KV bytes read by attention."""
    d, ff, L = spec.hidden, spec.ffn, spec.n_layers
    qd, kvd = spec.heads * spec.head_dim, spec.kv_heads * spec.head_dim
    per_layer = {"qkv": (qd + 2 * kvd) * d * Q4K, "o": d * qd * Q4K, "gate_up": 2 * ff * d * Q4K, "down": d * ff * Q4K}
    weights = L * sum(per_layer.values()) + spec.vocab * d * Q6K + d * Q4K
    kv_per_position = L * 2 * kvd * 2  # k and v rows, f16
    return weights, kv_per_position, per_layer


class _Events:
    """hipEvent timing on the library's stream (libamdhip64 through ctypes)."""

    def __init__(self):
        import ctypes as C
        self.C = C
        self.hip = None
        for name in ("libamdhip64.so", os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "lib", "libamdhip64.so")):
            try:
                self.hip = C.CDLL(name)
                break
            except OSError:
                continue
        if self.hip is None:
            raise RuntimeError("libamdhip64.so not found")
        self.hip.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
        self.hip.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        self.hip.hipEventSynchronize.argtypes = [C.c_void_p]
        self.hip.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        self.hip.hipEventDestroy.argtypes = [C.c_void_p]
        self.a, self.b = C.c_void_p(), C.c_void_p()
        for e in (self.a, self.b):
            if self.hip.hipEventCreate(C.byref(e)) != 0:
                raise RuntimeError("hipEventCreate failed")

    def elapsed_ms(self, stream, fn):
        C = self.C
        self.hip.hipEventRecord(self.a, stream)
        fn()
        self.hip.hipEventRecord(self.b, stream)
        self.hip.hipEventSynchronize(self.b)
        ms = C.c_float()
        self.hip.hipEventElapsedTime(C.byref(ms), self.a, self.b)
        return ms.value

    def close(self):
        self.hip.hipEventDestroy(self.a)
        self.hip.hipEventDestroy(self.b)


def time_gate_up(spec, layers=32, rounds=3):
    """Average duration of vkml_gemv_fused at the step's gate/up call (q4_K
    gate and up [ffn, hidden]; f32 residual stream in, RMSNorm + Q8_0 in the
    prologue; SwiGLU and Q8_0 of h in the epilogue), over `layers` distinct
    weight pairs launched back to back, `rounds` times, between two events.
    Weight values do not change the kernel's work; the buffers are filled
    with fixed patterns (f16 scales finite)."""
    from vkml_amd import hip as H
    n, k = spec.ffn, spec.hidden
    codes, hdr = n * k // 2, n * k // 256 * 16

    def buf(nbytes, word):
        b = H.Buffer(nbytes)
        H.call("vkml_fill_u32", b.p, word, (nbytes + 3) // 4)
        return b

    mats = [(buf(codes, 0x5A3C96E1), buf(hdr, 0x2C1F2C00), buf(codes, 0x3C5A1E96), buf(hdr, 0x2C0F2C00)) for _ in range(layers)]
    x, nw = buf(k * 4, 0x3F000000), buf(k * 4, 0x3F800000)
    out, hq, hs = buf(n * 4, 0), buf(n, 0), buf(n // 32 * 4, 0)
    prm = H.GemvFusedParams(n, k, H.Q4_K, H.F16, 2, 1, 1e-5, 1)

    def launches():
        for _ in range(rounds):
            for g, gs, u, us in mats:
                H.call("vkml_gemv_fused", prm, x.p, None, nw.p, g.p, gs.p, u.p, us.p, None, out.p, hq.p, hs.p)

    ev = _Events()
    try:
        launches()  # warm
        H.synchronize()
        ms = ev.elapsed_ms(H.stream(), launches)
    finally:
        ev.close()
        for m in mats:
            for b in m:
                b.close()
        for b in (x, nw, out, hq, hs):
            b.close()
    weight_bytes = 2 * (codes + hdr)
    io_bytes = 2 * k * 4 + n * 4 + n + n // 32 * 4  # x and the norm weight in; h, its codes and scales out
    return ms * 1e3 / (layers * rounds), weight_bytes + io_bytes


def attention_shape(prompt, steps):
    """The decode step's one attention launch a layer at the middle of the
    timed positions: (position, cache rows, chunks launched, chunks that
    load before reading the position), as src/llama.cpp sizes them (chunks
    of 128 keys in power-of-two tiers from 8; a tier above the smallest
    lets its lower half load early)."""
    position = prompt + steps // 2
    rows = prompt + steps + 1
    chunks = (rows + 127) // 128
    tier = 8
    while tier * 128 < position + 1:
        tier *= 2
    launched = min(chunks, tier)
    ready = min(tier // 2, launched) if tier > 8 else 0
    return position, rows, launched, ready


def time_attention_step(spec, prompt=PROMPT, steps=256, layers=32, rounds=3, fast=False):
    """Average duration of vkml_attend_step_fused as the decode step
    launches it (k_attend_fused: the chunk pass over the f16 caches, the
    merges, and the o GEMV + residual add of q4_K o weights), over `layers`
    distinct KV caches and o matrices launched back to back (873 MB, more
    than any cache holds), `rounds` times, between two HIP events, at the
    middle position of the timed run. The caches and weights hold fixed
    patterns (finite f16 values). Algorithmic bytes of one launch: the K
    and V rows of positions 0 .. position (f16), the o matrix (GGUF q4_K),
    q in, and the residual read and written; the chunk partials (split-K
    overhead) are not counted. With fast, vkml_attend_step_fast (the
    matrix-core attention option) instead."""
    import math
    from vkml_amd import hip as H
    heads, kvh, hd, d = spec.heads, spec.kv_heads, spec.head_dim, spec.hidden
    position, rows, chunks, ready = attention_shape(prompt, steps)
    cache = kvh * rows * hd * 2
    o_codes, o_hdr = d * heads * hd // 2, d * heads * hd // 256 * 16
    caches = [(filled(cache, 0x3C003800 + i), filled(cache, 0x38003C00 + i)) for i in range(layers)]
    mats = [(filled(o_codes, 0x5A3C96E1 + i), filled(o_hdr, 0x2C1F2C00)) for i in range(layers)]
    qkv = filled((heads + 2 * kvh) * hd * 4, 0x3F000000)
    x = filled(d * 4, 0x3F000000)
    part, stats = filled(heads * chunks * hd * 4, 0), filled(heads * chunks * 8, 0)
    attn, aq, as_ = filled(heads * hd * 4, 0), filled(heads * hd, 0), filled(heads * hd // 32 * 4, 0)
    st = filled(16, 0)
    H.call("vkml_state_set", st.p, 0, position, 0)
    fbytes = H.lib().vkml_attend_fused_sync_bytes(layers)
    fsync = filled(fbytes, 0)
    prm = H.AttendStepParams(heads, kvh, hd, rows, 0, 0, H.F16, chunks, 0, 1, 1.0 / math.sqrt(hd), 0.0, 0, 1, ready)
    op = H.GemvDotParams(1, d, heads * hd, H.Q4_K, H.F16)

    def launches():
        for _ in range(rounds):
            for li in range(layers):
                if fast:
                    H.call("vkml_attend_step_fast", prm, qkv.p, caches[li][0].p, caches[li][1].p, part.p, stats.p, attn.p,
                           aq.p, as_.p, st.p, op, mats[li][0].p, mats[li][1].p, x.p, fsync.p, li, layers)
                else:
                    H.call("vkml_attend_step_fused", prm, qkv.p, None, caches[li][0].p, caches[li][1].p, part.p, stats.p,
                           attn.p, aq.p, as_.p, st.p, op, mats[li][0].p, mats[li][1].p, x.p, fsync.p, li, layers)

    ev = _Events()
    try:
        launches()  # warm
        H.synchronize()
        ms = ev.elapsed_ms(H.stream(), launches)
        H.call("vkml_attend_fused_check", fsync.p, layers)
    finally:
        ev.close()
        for pair in caches + mats:
            for b in pair:
                b.close()
        for b in (qkv, x, part, stats, attn, aq, as_, st, fsync):
            b.close()
    alg = 2 * kvh * (position + 1) * hd * 2 + d * heads * hd * 144 // 256 + heads * hd * 4 + 2 * d * 4
    return ms * 1e3 / (layers * rounds), alg, {"position": position, "chunks": chunks, "ready_chunks": ready}


def roofline_only(spec):
    """The dominant kernels' measurements alone, then a device copy of 256
    MiB (hipMemcpy device to device, the runtime's copy kernel) launched
    three times: per dispatch it reads and writes exactly 268,435,456 bytes,
    the known size against which a counter's reading is scaled."""
    from vkml_amd import hip as H
    H.init()
    att_us, att_bytes, shape = time_attention_step(spec, rounds=1)
    log(f"attend_step_fused at position {shape['position']}: {att_us:.2f} us a launch, "
        f"{att_bytes / (att_us * 1e-6) / 1e9:.0f} GB/s ({att_bytes} algorithmic bytes)")
    fast_us, _, _ = time_attention_step(spec, rounds=1, fast=True)
    log(f"attend_step_fast at position {shape['position']}: {fast_us:.2f} us a launch, "
        f"{att_bytes / (fast_us * 1e-6) / 1e9:.0f} GB/s")
    dom_us, dom_bytes = time_gate_up(spec, layers=32, rounds=1)
    log(f"gemv_fused gate/up: {dom_us:.2f} us a launch, {dom_bytes / (dom_us * 1e-6) / 1e9:.0f} GB/s "
        f"({dom_bytes} algorithmic bytes)")
    copy_256mib()


def copy_256mib():
    """hipMemcpy device to device of 256 MiB, three times: the runtime's copy
    kernel reads and writes exactly 268,435,456 bytes a dispatch, the known
    size a hardware counter's reading is scaled by."""
    from vkml_amd import hip as H
    n = 256 << 20
    src, dst = H.Buffer(n), H.Buffer(n)
    H.call("vkml_fill_u32", src.p, 0x01020304, n // 4)
    for _ in range(3):
        H.call("vkml_memcpy_d2d", dst.p, src.p, n)
    H.synchronize()
    src.close()
    dst.close()
    log(f"copy: 3 x {n} bytes")


def rotation_times(n_copies, launch, rotations=5):
    """Per-launch microseconds of each of `rotations` passes over n_copies
    back-to-back launches (launch(i) issues copy i's), between HIP events on
    the library's stream, after one untimed pass: (best, median)."""
    from vkml_amd import hip as H
    ev = _Events()
    try:
        for i in range(n_copies):
            launch(i)
        H.synchronize()
        per = []
        for _ in range(rotations):
            ms = ev.elapsed_ms(H.stream(), lambda: [launch(i) for i in range(n_copies)])
            per.append(ms * 1e3 / n_copies)
    finally:
        ev.close()
    per.sort()
    return per[0], per[len(per) // 2]


def filled(nbytes, word):
    from vkml_amd import hip as H
    b = H.Buffer(nbytes)
    H.call("vkml_fill_u32", b.p, word, (nbytes + 3) // 4)
    return b


def bench_gemv_cfg2(min_bytes=512 << 20):
    """cfg2: y = W x for W 4096x4096, 14336x4096 and 4096x14336 in Q8_0 and
    Q4_K, x f32. Two figures each: the GEMV kernel on the Q8_0 activation
    (the decode step's unit of work), and the op on the f32 x as
    matmul_transposed runs it for one row (k <= 4096: the Q8_0 of x inside
    the GEMV, one launch; else the activation quantized, then the GEMV).
    Algorithmic bytes are the GGUF-native weight bytes plus x in and y out."""
    from vkml_amd import hip as H
    out = []
    for fmt in ("q8_0", "q4_K"):
        for n, k in ((4096, 4096), (14336, 4096), (4096, 14336)):
            if fmt == "q8_0":
                codes, scales, bt, wbytes = n * k, n * k // 32 * 2, H.Q8_0, n * k * 34 // 32
                patt = (0x7F81C03E, 0x1C231C17)
            else:
                codes, scales, bt, wbytes = n * k // 2, n * k // 256 * 16, H.Q4_K, n * k * 144 // 256
                patt = (0x5A3C96E1, 0x2C1F2C00)
            copies = max(2, -(-min_bytes // (codes + scales)))
            mats = [(filled(codes, patt[0] + i), filled(scales, patt[1])) for i in range(copies)]
            x, xq, xs, y = filled(k * 4, 0x3F000000), filled(k, 0), filled(k // 32 * 4, 0), filled(n * 4, 0)
            dp = H.GemvDotParams(1, n, k, bt, H.F16)
            qp = H.QuantizeParams(k // 32, H.F32, H.Q8_0, H.F32)
            H.call("vkml_quantize", qp, x.p, xq.p, xs.p)
            kern = rotation_times(copies, lambda i: H.call("vkml_gemv_dot", dp, xq.p, mats[i][0].p, y.p, mats[i][1].p, xs.p))

            fp = H.GemvFusedParams(n, k, bt, H.F16, 0, 2, 0.0, 0)

            def op(i):
                if k <= 4096:
                    H.call("vkml_gemv_fused", fp, x.p, None, None, mats[i][0].p, mats[i][1].p, None, None, None, y.p, None, None)
                else:
                    H.call("vkml_quantize", qp, x.p, xq.p, xs.p)
                    H.call("vkml_gemv_dot", dp, xq.p, mats[i][0].p, y.p, mats[i][1].p, xs.p)
            opt = rotation_times(copies, op)
            alg = wbytes + 4 * k + 4 * n
            out.append({"format": fmt, "n": n, "k": k, "bytes": alg,
                        "kernel_us": {"best": round(kern[0], 3), "median": round(kern[1], 3)},
                        "kernel_frac": round(alg / (kern[0] * 1e-6) / 1e9 / PEAK_HBM, 4),
                        "op_us": {"best": round(opt[0], 3), "median": round(opt[1], 3)},
                        "op_frac": round(alg / (opt[0] * 1e-6) / 1e9 / PEAK_HBM, 4)})
            log(f"cfg2 {fmt} {n}x{k}: gemv {kern[0]:.2f} us ({alg / (kern[0] * 1e-6) / 1e9:.0f} GB/s), "
                f"f32 x to y {opt[0]:.2f} us ({'one launch' if k <= 4096 else 'quantize + gemv'})")
            for m in mats:
                for b in m:
                    b.close()
            for b in (x, xq, xs, y):
                b.close()
    return out


def bench_attention_cfg4(min_bytes=512 << 20, lengths=(4096, 16384, 32768)):
    """cfg4: decode attention of 32 query heads on 8 KV heads, head_dim 128,
    over f16 caches of T = 4096, 16384 and 32768 positions: the exact chunk
    pass and merge (vkml_attend + vkml_attend_merge), and the matrix-core
    form (vkml_attend_fast: items, merges by the last item, one launch).
    Algorithmic bytes: K and V (4096 T) plus q in and the output out."""
    import math
    from vkml_amd import hip as H
    heads, kvh, hd = 32, 8, 128
    out = []
    for T in lengths:
        cache = kvh * T * hd * 2
        copies = max(2, -(-min_bytes // (2 * cache)))
        caches = [(filled(cache, 0x3C003800 + i), filled(cache, 0x38003C00 + i)) for i in range(copies)]
        chunks = (T + 127) // 128
        q = filled(heads * hd * 4, 0x3F000000)
        part, stats, o = filled(heads * chunks * hd * 4, 0), filled(heads * chunks * 8, 0), filled(heads * hd * 4, 0)
        prm = H.AttendParams(0, T, T, heads, kvh, hd, H.F16, chunks, 1.0 / math.sqrt(hd), 0.0)

        def call(i):
            H.call("vkml_attend", prm, q.p, caches[i][0].p, caches[i][1].p, part.p, stats.p, None)
            H.call("vkml_attend_merge", prm, part.p, stats.p, o.p, None, None)
        best, med = rotation_times(copies, call)
        sync = filled(H.lib().vkml_attend_fused_sync_bytes(1), 0)

        def call_fast(i):
            H.call("vkml_attend_fast", prm, q.p, caches[i][0].p, caches[i][1].p, part.p, stats.p, o.p, None, None, sync.p, None)
        fbest, fmed = rotation_times(copies, call_fast)
        sync.close()
        alg = 2 * cache + 2 * heads * hd * 4
        out.append({"positions": T, "bytes": alg, "us": {"best": round(best, 3), "median": round(med, 3)},
                    "frac": round(alg / (best * 1e-6) / 1e9 / PEAK_HBM, 4),
                    "fast_us": {"best": round(fbest, 3), "median": round(fmed, 3)},
                    "fast_frac": round(alg / (fbest * 1e-6) / 1e9 / PEAK_HBM, 4)})
        log(f"cfg4 attention at {T}: exact {best:.2f} us ({alg / (best * 1e-6) / 1e9:.0f} GB/s), "
            f"matrix-core {fbest:.2f} us ({alg / (fbest * 1e-6) / 1e9:.0f} GB/s)")
        for c in caches:
            for b in c:
                b.close()
        for b in (q, part, stats, o):
            b.close()
    return out


def bench_cfg3(L, steps=128, prompt_len=512):
    """cfg3: the Llama-3.2-1B-shaped model (16 layers, tied q6_K vocabulary
    of 128256) with a 512-token prompt prefilled on the matrix cores, then
    `steps` greedy decode tokens timed back to back."""
    from vkml_amd import synth
    spec = synth.CONFIGS["cfg3"]
    path = os.path.join(synth.scratch_dir(), f"vkml_bench_cfg3_{os.getpid()}.gguf")
    synth.write_model(spec, path, seed=4)
    try:
        model = L.Llama(path, prompt_len + steps + 1, kv_f16=True)
        prompt = np.random.default_rng(4).integers(0, spec.vocab, prompt_len).astype(np.int32)
        pre = prefill_rates(model, spec, prompt, [prompt_len], L)
        model.rewind(0)
        prompt_logits = model.forward(prompt)
        first = int(np.argmax(prompt_logits))
        model.generate_greedy(first, 8)
        model.rewind(prompt_len)
        L.synchronize()
        t0 = time.perf_counter()
        tokens = model.generate_greedy(first, steps)
        secs = time.perf_counter() - t0
        parity = against_fixture(fixture("cfg3"), prompt_logits, first, tokens)
        d, ff, layers = spec.hidden, spec.ffn, spec.n_layers
        qd, kvd = spec.heads * spec.head_dim, spec.kv_heads * spec.head_dim
        weights = layers * ((qd + 2 * kvd) * d + d * qd + 3 * ff * d) * Q4K + spec.vocab * d * Q6K + d * Q6K
        kv = layers * 2 * kvd * 2 * (prompt_len + (steps + 1) / 2)
        tok_s = steps / secs
        gbs = (weights + kv) * tok_s / 1e9
        log(f"cfg3 decode: {tok_s:.1f} tokens/s, {gbs:.0f} GB/s algorithmic")
        model.close()
        return {"decode_tokens_per_s": round(tok_s, 1), "ms_per_token": round(secs * 1e3 / steps, 4),
                "bytes_per_token": round(weights + kv), "hbm_gb_s": round(gbs, 1), "hbm_frac": round(gbs / PEAK_HBM, 4),
                "prefill": pre[0] if pre else None, "parity": parity}
    finally:
        os.remove(path)


def bench_fast_attention(L, path, spec, prompt, steps, context, fx):
    """The same run with LlamaOptions::fast_attention (attention on the
    matrix cores, not the reference's f32 order): the prompt's prefill time
    (its attention by vkml_attend_prompt_fast), tokens/s over `steps`
    greedy steps from the same prompt, its attention launch at the roofline
    entry's shape, and how many of its ids equal the oracle's (the int8
    activations carry any last-bit change on, so they part after a while)."""
    model = L.Llama(path, context, kv_f16=True, fast_attention=True)
    try:
        model.forward(prompt)  # warm
        model.rewind(0)
        L.synchronize()
        t0 = time.perf_counter()
        first = int(np.argmax(model.forward(prompt)))  # the prompt's attention on the matrix cores too
        L.synchronize()
        prefill_s = time.perf_counter() - t0
        model.generate_greedy(first, 8)
        model.rewind(len(prompt))
        L.synchronize()
        t0 = time.perf_counter()
        tokens = model.generate_greedy(first, steps)
        secs = time.perf_counter() - t0
    finally:
        model.close()
    att_us, att_bytes, shape = time_attention_step(spec, len(prompt), ROOFLINE_STEPS, fast=True)
    out = {"tokens_per_s": round(steps / secs, 2), "ms_per_step": round(secs * 1e3 / steps, 4),
           "prefill": {"tokens": len(prompt), "ms": round(prefill_s * 1e3, 2), "tokens_per_s": round(len(prompt) / prefill_s, 1)},
           "attention_launch_us": round(att_us, 3), "attention_gb_s": round(att_bytes / (att_us * 1e-6) / 1e9, 1),
           "attention_frac": round(att_bytes / (att_us * 1e-6) / 1e9 / PEAK_HBM, 4), "shape": shape}
    if fx is not None:
        ids = [int(t) for t in fx["ids"][1:steps + 1]]
        differ = [i for i, (a, b) in enumerate(zip(tokens, ids)) if int(a) != b]
        out["ids_equal_to_oracle"] = len(ids) - len(differ)
        out["first_difference"] = differ[0] if differ else None
    log(f"fast attention: prefill of {len(prompt)} tokens {prefill_s * 1e3:.1f} ms; {out['tokens_per_s']} tokens/s; "
        f"attention launch {att_us:.2f} us; "
        f"ids equal to the oracle's: {out.get('ids_equal_to_oracle')} of {steps}")
    return out


def bench_long_position(L, path, spec, position=32696, steps=64):
    """The cfg5 model decoding at positions 32696..32760 (Llama::advance to
    the position: the cache rows below hold zeros, which costs the same to
    attend over), with the exact and the matrix-core attention: the step at
    a 32k context."""
    out = {"positions": [position, position + steps]}
    for fast in (False, True):
        model = L.Llama(path, position + steps + 8, kv_f16=True, fast_attention=fast)
        try:
            model.advance(position)
            model.generate_greedy(3, 8)
            model.rewind(position)
            L.synchronize()
            t0 = time.perf_counter()
            model.generate_greedy(3, steps)
            secs = time.perf_counter() - t0
        finally:
            model.close()
        weights, kv_pos, _ = algorithmic_bytes(spec)
        step_bytes = weights + kv_pos * (position + (steps + 1) / 2)
        key = "matrix_core" if fast else "exact"
        out[key] = {"tokens_per_s": round(steps / secs, 1), "hbm_gb_s": round(step_bytes * steps / secs / 1e9, 1)}
        log(f"cfg5 decode at positions {position}..{position + steps} ({key} attention): {steps / secs:.1f} tokens/s")
    return out


def bench_short_position(L, path, contexts=(1024, 32768), prompt_len=512, steps=64):
    """The cfg5 model decoding at positions 512.. with caches of different
    lengths: a step launches the attention chunks its position needs, so
    the rate should not fall with the cache's length."""
    prompt = np.random.default_rng(5).integers(0, 32768, prompt_len).astype(np.int32)
    out = {}
    for ctx in contexts:
        model = L.Llama(path, ctx, kv_f16=True)
        first = int(np.argmax(model.forward(prompt)))
        model.generate_greedy(first, 8)
        model.rewind(prompt_len)
        L.synchronize()
        t0 = time.perf_counter()
        model.generate_greedy(first, steps)
        secs = time.perf_counter() - t0
        model.close()
        out[f"context_{ctx}"] = round(steps / secs, 1)
        log(f"cfg5 decode at positions {prompt_len}..{prompt_len + steps} with a {ctx}-row cache: {steps / secs:.1f} tokens/s")
    return {"tokens_per_s": out, "positions": [prompt_len, prompt_len + steps]}


def matrix_macs(spec):
    """Multiply-accumulates of one token's layer projections (q|k|v, o,
    gate, up, down) over all layers: matmul_dot's work per prompt row."""
    qkv = (spec.heads + 2 * spec.kv_heads) * spec.head_dim * spec.hidden
    o = spec.hidden * spec.heads * spec.head_dim
    ffn = 3 * spec.ffn * spec.hidden
    return spec.n_layers * (qkv + o + ffn)


def prefill_rates(model, spec, prompt, lengths, L):
    """Prompts of the given lengths at once from position 0 (the cache rows
    they write are the decode run's, which is over): a warm-up pass, a timed
    pass, and a HIP-event profile pass. MFMA utilisation is matmul_dot's
    int8 operations (2 per multiply-accumulate) over its event time (with
    matmul_dot_add's, the o and down projections), against the 5.0 POP/s
    dense int8 peak."""
    out = []
    for n in [n for n in lengths if 1 < n <= len(prompt)]:
        toks = prompt[:n]
        model.rewind(0)
        model.forward(toks)
        model.rewind(0)
        L.synchronize()
        t0 = time.perf_counter()
        model.forward(toks)
        L.synchronize()
        secs = time.perf_counter() - t0
        model.rewind(0)
        L.set_profiling(True)
        L.reset_profile()
        model.forward(toks)
        L.synchronize()
        prof = L.profile()
        L.set_profiling(False)
        by_kernel = {}
        for name, calls, ms in prof:
            k = name.split(":")[0]
            c, t = by_kernel.get(k, (0, 0.0))
            by_kernel[k] = (c + calls, t + ms)
        # the o and down projections take matmul_dot_add (the residual add in the store)
        mm_ms = sum(by_kernel.get(k, (0, 0.0))[1] for k in ("matmul_dot", "matmul_dot_add"))
        ops = 2.0 * n * matrix_macs(spec)
        tops = ops / (mm_ms * 1e-3) / 1e12 if mm_ms else None
        top = sorted(by_kernel.items(), key=lambda kv: -kv[1][1])[:8]
        log(f"prefill {n} tokens: {secs * 1e3:.1f} ms, {n / secs:.0f} tokens/s; matmul_dot {mm_ms:.2f} ms "
            f"({tops or 0:.0f} TOP/s int8, {100 * (tops or 0) / PEAK_INT8_TOPS:.1f}% of peak)")
        for k, (c, t) in top:
            log(f"    {k:<20} calls {c:>6}  {t:9.3f} ms")
        out.append({"tokens": n, "ms": round(secs * 1e3, 3), "tokens_per_s": round(n / secs, 1),
                    "matmul_dot_ms": round(mm_ms, 3),
                    "mfma": {"kernel": "matmul_dot (v_mfma_i32_16x16x32_i8)", "achieved": round(tops, 1) if tops else None,
                             "peak": PEAK_INT8_TOPS, "unit": "TOP/s", "frac": round(tops / PEAK_INT8_TOPS, 4) if tops else None},
                    "kernels_ms": {k: round(t, 3) for k, (c, t) in top}})
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--prompt", type=int, default=PROMPT)
    ap.add_argument("--profile-steps", type=int, default=16)
    ap.add_argument("--cpu-tokens", type=int, default=3, help="decode tokens the CPU oracle is timed on (0: skip)")
    ap.add_argument("--layers", type=int, default=0, help="override the layer count (for quick local checks only)")
    ap.add_argument("--no-graphs", action="store_true",
                    help="launch every kernel from the host instead of replaying the captured step (for profilers "
                         "that cannot follow graph launches; the kernels are the same)")
    ap.add_argument("--prefill", type=int, nargs="*", default=[512, 4096],
                    help="prompt lengths whose prefill rate is measured after the decode run (none: skip)")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the cfg2, cfg3 and cfg4 measurements")
    ap.add_argument("--roofline-only", action="store_true",
                    help="run only the dominant kernel's timed launches and a 256 MiB device copy of known size, "
                         "for hardware-counter passes (FETCH_SIZE, WRITE_SIZE) that scale the kernel's HBM bytes "
                         "by what the copy reads")
    ap.add_argument("--cfg4", type=int, nargs="+", default=None, metavar="POSITIONS",
                    help="run only cfg4's attention at these cache lengths (4096 16384 32768) and the 256 MiB device "
                         "copy, printing cfg4's JSON entries: the command the cfg4 profiles are taken with")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported (every GPU box here has one). "
              "A second GPU would hold a replica (independent sequences) or a tensor-parallel shard; see DESIGN.md.",
              file=sys.stderr)
        sys.exit(2)

    from vkml_amd import synth
    from vkml_amd import llama as L

    spec = synth.CONFIGS["cfg5"]
    if args.roofline_only:
        roofline_only(spec)
        return
    if args.cfg4:
        from vkml_amd import hip as H
        H.init()
        print(json.dumps({"cfg4_attention": bench_attention_cfg4(lengths=args.cfg4)}), flush=True)
        copy_256mib()
        return
    if args.layers:
        spec = synth.ModelSpec(spec.name, args.layers, spec.hidden, spec.heads, spec.kv_heads, spec.head_dim, spec.ffn,
                               spec.vocab, spec.theta, max_positions=spec.max_positions)
    context = args.prompt + max(args.steps, args.profile_steps, args.warmup) + 1
    path = os.path.join(synth.scratch_dir(), f"vkml_bench_cfg5_{os.getpid()}.gguf")
    t0 = time.time()
    synth.write_model(spec, path, seed=6)
    log(f"model written in {time.time() - t0:.1f} s ({os.path.getsize(path) / 1e9:.2f} GB)")
    try:
        t0 = time.time()
        model = L.Llama(path, context, kv_f16=True, use_graphs=not args.no_graphs)
        log(f"loaded in {time.time() - t0:.1f} s; kv cache {model.kv_cache_bytes / 1e6:.0f} MB")
        prompt = np.random.default_rng(6).integers(0, spec.vocab, args.prompt).astype(np.int32)
        t0 = time.time()
        logits = model.forward(prompt)
        log(f"prefill {args.prompt} tokens in {time.time() - t0:.1f} s")
        first = int(np.argmax(logits))
        prompt_logits = logits.copy()

        # Warm-up, then rewind so the timed steps see positions 4096.. as configured.
        if args.warmup:
            model.generate_greedy(first, args.warmup)
            model.rewind(args.prompt)
        L.synchronize()
        t0 = time.perf_counter()
        tokens = model.generate_greedy(first, args.steps)  # returns after the device is done
        elapsed = time.perf_counter() - t0
        ms_per_step = elapsed * 1e3 / args.steps
        tok_s = args.steps / elapsed
        weights, kv_pos, per_layer = algorithmic_bytes(spec)
        positions = np.arange(args.prompt + 1, args.prompt + args.steps + 1)
        step_bytes = weights + kv_pos * positions.mean()
        hbm = step_bytes / (ms_per_step * 1e-3) / 1e9
        log(f"decode {args.steps} tokens: {ms_per_step:.3f} ms/token, {tok_s:.1f} tokens/s, {hbm:.0f} GB/s algorithmic")

        # Per-kernel HIP-event profile of extra steps (eager launches on the same stream).
        model.rewind(args.prompt)
        L.set_profiling(True)
        L.reset_profile()
        model.generate_greedy(first, args.profile_steps)
        L.synchronize()
        prof = L.profile()
        L.set_profiling(False)
        n_layers = spec.n_layers
        kv_mean = args.prompt + (args.profile_steps + 1) / 2
        launch_bytes = {
            "gemv_rope:qkv": per_layer["qkv"], "gemv_fused:gate_up": per_layer["gate_up"],
            "gemv_dot_add:down": per_layer["down"], "gemv_dot:lm_head": spec.vocab * spec.hidden * Q6K,
            "attend_fused:attention": kv_pos / n_layers * kv_mean + per_layer["o"],
        }
        rows = []
        for name, calls, ms in prof:
            avg_us = ms * 1e3 / max(calls, 1)
            b = launch_bytes.get(name)
            rows.append({"kernel": name, "calls": calls, "avg_us": round(avg_us, 3),
                         "gb_s": round(b / (avg_us * 1e-6) / 1e9, 1) if b else None})
        log("per-label HIP-event profile of eager steps (includes launch gaps):")
        for r in sorted(rows, key=lambda r: -r["calls"] * r["avg_us"])[:14]:
            log(f"  {r['kernel']:<28} calls {r['calls']:>6}  avg {r['avg_us']:9.2f} us  {r['gb_s'] or '':>8} GB/s")
        busy_ms = sum(ms for _, _, ms in prof) / args.profile_steps if args.profile_steps else None
        att_us, att_bytes, att_shape = time_attention_step(spec, args.prompt, ROOFLINE_STEPS)
        att_rate = att_bytes / (att_us * 1e-6) / 1e9
        log(f"attend_step_fused (chunks, merge, o GEMV + residual) back to back at position {att_shape['position']}: "
            f"{att_us:.2f} us a launch, {att_rate:.0f} GB/s")
        gu_us, gu_bytes = time_gate_up(spec)
        gu_rate = gu_bytes / (gu_us * 1e-6) / 1e9
        log(f"gemv_fused (norm + gate/up + swiglu + q8_0) back to back: {gu_us:.2f} us a launch, {gu_rate:.0f} GB/s")

        headline = args.prompt == PROMPT and not args.layers
        fx_parity = against_fixture(fixture("cfg5"), prompt_logits, first, tokens) if headline else None
        if fx_parity:
            log(f"against the oracle's own run: prompt logits {'bit-identical' if fx_parity['prompt_logits_bit_identical'] else 'DIFFER'}, "
                f"{fx_parity['timed_ids_equal']} of {fx_parity['timed_ids_checked']} timed ids equal")
        fast = bench_fast_attention(L, path, spec, prompt, args.steps, context, fixture("cfg5") if headline else None)

        pre = prefill_rates(model, spec, prompt, args.prefill, L) if args.prefill else None

        cpu, parity = None, None
        if args.cpu_tokens > 0:
            # The oracle continues from the GPU's cache: rows 0 .. prompt - 1
            # hold the prompt's keys and values (the prefill passes above
            # rewrote them with the same prompt).
            sys.path.insert(0, os.path.join(ROOT, "oracle"))
            import oracle as O
            threads, nproc = host_cores()
            O.set_threads(threads)
            t0 = time.time()
            ref = O.Model(path, context, kv_f16=True)
            for layer in range(spec.n_layers):
                k, v = model.read_kv_cache(layer)
                ref.set_kv(layer, k, v)
            ref.set_position(args.prompt)
            log(f"oracle loaded with the GPU's KV cache in {time.time() - t0:.1f} s")
            t0 = time.perf_counter()
            cpu_tokens, nxt = [], first
            for i in range(args.cpu_tokens):
                nxt = int(O.argmax(ref.forward(np.array([nxt], np.int32))))
                cpu_tokens.append(nxt)
            cpu_s = time.perf_counter() - t0
            parity = cpu_tokens == [int(t) for t in tokens[:args.cpu_tokens]]
            cpu = {"value": round(args.cpu_tokens / cpu_s, 4), "unit": "tokens/s", "cores": threads, "host_cpus": nproc,
                   "kind": "port",
                   "sample": f"{args.cpu_tokens} greedy decode tokens of the same model at positions {args.prompt}.. from the "
                             f"GPU's KV cache (CPU oracle, the reference's int8 path, {threads} threads of the box's "
                             f"{nproc} logical CPUs, {cpu_s:.1f} s)",
                   "tokens": cpu_tokens}
            ref.close()
            log(f"cpu oracle: {cpu['value']} tokens/s on {threads} threads; tokens {cpu_tokens} "
                f"{'equal' if parity else 'DIFFER FROM'} the GPU's {[int(t) for t in tokens[:args.cpu_tokens]]}")

        configs = None
        if not args.no_configs:
            configs = {"cfg2_gemv": bench_gemv_cfg2(), "cfg4_attention": bench_attention_cfg4()}
            model.close()
            model = None
            configs["cfg5_short_position"] = bench_short_position(L, path)
            configs["cfg5_long_position"] = bench_long_position(L, path, spec)
            configs["cfg3"] = bench_cfg3(L)

        gu_traffic = GATE_UP_TRAFFIC if sources_hash() == GATE_UP_TRAFFIC_SOURCES else None
        att_traffic = (ATTEND_TRAFFIC if ATTEND_TRAFFIC and sources_hash(ATTEND_FILES) == ATTEND_TRAFFIC_SOURCES
                       and att_shape["position"] == ATTEND_TRAFFIC_POSITION else None)
        result = {
            "metric": "batch-1 decode tokens/s + achieved HBM GB/s (% of 8 TB/s), 1xMI355X",
            "value": round(tok_s, 2),
            "unit": "tokens/s",
            "n_gpus": 1,
            "steps": args.steps,
            "warmup": args.warmup,
            "ms_per_step": round(ms_per_step, 4),
            "higher_is_better": True,
            "scaling": "weak",
            "vs_baseline": None,
            "dtype": "int8",
            "data": "synthetic",
            "config": {"workload": "cfg5: Mistral-7B-shaped decoder, q4_K weights + q6_K output (GGUF), f16 KV prefilled "
                                   f"with {args.prompt} random-token positions, {args.steps} greedy decode steps, batch 1",
                       "layers": spec.n_layers, "hidden": spec.hidden, "heads": spec.heads, "kv_heads": spec.kv_heads,
                       "head_dim": spec.head_dim, "ffn": spec.ffn, "vocab": spec.vocab, "seq_len": args.prompt},
            "hbm_gb_s": round(hbm, 1),
            "hbm_frac": round(hbm / PEAK_HBM, 4),
            "bytes_per_step": round(step_bytes),
            "gpu_busy_ms_per_step": round(busy_ms, 4) if busy_ms is not None else None,
            "roofline": {"bound": "hbm",
                         "kernel": "attend_step_fused (k_attend_fused: chunk pass, merges, o GEMV + residual; one launch a layer)",
                         "achieved": round(att_rate, 1), "peak": PEAK_HBM, "unit": "GB/s",
                         "frac": round(att_rate / PEAK_HBM, 4), "traffic": att_traffic,
                         "traffic_over_algorithmic": round(att_traffic / att_bytes, 4) if att_traffic else None,
                         "traffic_sources": sources_hash(ATTEND_FILES),
                         "bytes_per_launch": round(att_bytes), "avg_launch_us": round(att_us, 3), "shape": att_shape},
            "roofline_gate_up": {"bound": "hbm",
                                 "kernel": "gemv_fused gate/up (k_gemv_dot<q4_K, f16, 8 lanes, swiglu, norm, q8_0 out>)",
                                 "achieved": round(gu_rate, 1), "peak": PEAK_HBM, "unit": "GB/s",
                                 "frac": round(gu_rate / PEAK_HBM, 4), "traffic": gu_traffic,
                                 "traffic_over_algorithmic": round(gu_traffic / gu_bytes, 4) if gu_traffic else None,
                                 "traffic_sources": sources_hash(),
                                 "bytes_per_launch": round(gu_bytes), "avg_launch_us": round(gu_us, 3)},
            "cpu_baseline": cpu,
            "parity": (fx_parity["all_equal"] if fx_parity else parity) if parity is not False else False,
            "parity_detail": {"oracle_fixture": fx_parity, "cpu_baseline_tokens_equal": parity},
            "fast_attention": fast,
            "prefill": pre,
            "configs": configs,
            "tokens_head": [int(t) for t in tokens[:8]],
        }
        print(json.dumps(result), flush=True)
        if model is not None:
            model.close()
    finally:
        try:
            os.remove(path)
        except OSError:
            pass


if __name__ == "__main__":
    main()
