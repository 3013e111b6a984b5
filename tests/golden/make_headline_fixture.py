"""Writes the headline runs' fixtures: the CPU oracle's own prompt and
greedy decode on the seeded cfg5 and cfg3 models, as bench.py and the
full-size GPU tests run them.

    python tests/golden/make_headline_fixture.py cfg5   # about an hour on 8 threads
    python tests/golden/make_headline_fixture.py cfg3

Each run writes tests/golden/headline_<cfg>.npz:
- prompt_logits: the last prompt row's logits (float32, whole);
- ids: the first greedy token (argmax of prompt_logits), then one per decode
  step (steps + 1 ids);
- step_sha: per decode step, the first 8 bytes of SHA-256 over that step's
  float32 logits (little-endian bytes), as uint64, so a bit-identical run
  is checked on every logit of every step;
- fixed_idx / fixed_logits: every step's logits at 256 fixed indices, and
  top_idx / top_logits: its 16 largest, for tolerance checks of paths that
  do not keep the reference's order of f32 operations;
- max_abs: every step's largest |logit|.

The model files and prompts are the ones bench.py and
tests/test_gpu_fullsize.py build: synth.write_model(spec, seed) and
numpy.random.default_rng(seed).integers(0, vocab, prompt) with seed 6 (cfg5,
4096 prompt tokens, 256 steps) or 4 (cfg3, 512 prompt tokens, 128 steps),
f16 KV cache. The oracle is test infrastructure (oracle/); it restates the
reference's Llama::run (src/models/llama.cpp:299-406) and its int8 kernels.
"""
import argparse
import hashlib
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for sub in ("oracle", os.path.join("vkml-framework_amd", "python")):
    sys.path.insert(0, os.path.join(ROOT, sub))

import oracle as O  # noqa: E402
from vkml_amd import synth  # noqa: E402

RUNS = {"cfg5": (6, 4096, 256), "cfg3": (4, 512, 128)}
FIXED = 256
TOP = 16


def logits_sha(x) -> int:
    return int.from_bytes(hashlib.sha256(np.ascontiguousarray(x, "<f4").tobytes()).digest()[:8], "little")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("config", choices=sorted(RUNS))
    ap.add_argument("--threads", type=int, default=os.cpu_count() or 1)
    ap.add_argument("--steps", type=int, default=0, help="fewer decode steps (0: the headline's)")
    args = ap.parse_args()
    seed, prompt_len, steps = RUNS[args.config]
    steps = args.steps or steps
    spec = synth.CONFIGS[args.config]
    O.set_threads(args.threads)
    path = os.path.join(synth.scratch_dir(), f"vkml_fixture_{args.config}_{os.getpid()}.gguf")
    synth.write_model(spec, path, seed=seed)
    try:
        prompt = np.random.default_rng(seed).integers(0, spec.vocab, prompt_len).astype(np.int32)
        ref = O.Model(path, prompt_len + steps + 1, kv_f16=True)
        t0 = time.time()
        print(f"{args.config}: prompt of {prompt_len} tokens on {args.threads} threads", flush=True)
        prompt_logits = ref.forward(prompt)
        print(f"{args.config}: prompt done in {time.time() - t0:.0f} s", flush=True)
        fixed_idx = np.sort(np.random.default_rng(1000 + seed).choice(spec.vocab, FIXED, replace=False)).astype(np.int32)
        ids = [int(O.argmax(prompt_logits))]
        sha, fixed, top_i, top_v, max_abs = [], [], [], [], []
        for i in range(steps):
            lg = ref.forward(np.array([ids[-1]], np.int32))
            ids.append(int(O.argmax(lg)))
            sha.append(logits_sha(lg))
            fixed.append(lg[fixed_idx])
            order = np.argsort(-lg, kind="stable")[:TOP]
            top_i.append(order.astype(np.int32))
            top_v.append(lg[order])
            max_abs.append(float(np.abs(lg).max()))
            if i % 8 == 7 or i == steps - 1:
                print(f"{args.config}: step {i + 1}/{steps} at {time.time() - t0:.0f} s", flush=True)
        ref.close()
        out = os.path.join(HERE, f"headline_{args.config}.npz")
        np.savez_compressed(out, prompt_logits=prompt_logits.astype(np.float32), ids=np.array(ids, np.int32),
                            step_sha=np.array(sha, np.uint64), fixed_idx=fixed_idx,
                            fixed_logits=np.array(fixed, np.float32), top_idx=np.array(top_i, np.int32),
                            top_logits=np.array(top_v, np.float32), max_abs=np.array(max_abs, np.float32),
                            seed=np.int32(seed), prompt_len=np.int32(prompt_len))
        print(f"wrote {out}", flush=True)
    finally:
        os.remove(path)


if __name__ == "__main__":
    main()
