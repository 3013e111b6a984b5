"""Seeded synthetic models and weight blocks of BASELINE.json's configs.

Values come from numpy's PCG64 generator (np.random.default_rng(seed)), one
stream per tensor (seed, tensor index), so any tensor can be rebuilt alone.

Block recipes (the ones the isolated GEMV config names, scaled so a layer's
weights have a realistic spread):
- q8_0: codes uniform over -127..127, f16 scale |N(0, 0.01)|.
- q4_K: 4-bit codes and 6-bit sub-block scales and mins uniform (random
  bytes); f16 d = |N(0,1)| * 0.01 / 63, f16 dmin = |N(0,1)| * 0.01 * 7.5 / 63,
  so d * sc * q has a spread near 0.02 and sub-blocks are centred on average.
- q6_K: 6-bit codes uniform (random ql/qh bytes), int8 sub-block scales
  uniform over -128..127, f16 d = |N(0,1)| * 0.02 / 1365 (spread near 0.02).
- f32: N(0, 0.02) (the plumbing config), norm weights 1.0.
"""
from __future__ import annotations

import dataclasses
import os

import numpy as np

from . import gguf


@dataclasses.dataclass
class ModelSpec:
    name: str
    n_layers: int
    hidden: int
    heads: int
    kv_heads: int
    head_dim: int
    ffn: int
    vocab: int
    theta: float
    eps: float = 1e-5
    max_positions: int = 32768
    tied: bool = False
    matrix_type: int = gguf.Q4_K   # attention and FFN matrices
    embed_type: int = gguf.Q4_K    # token_embd
    output_type: int = gguf.Q6_K   # output (ignored when tied)
    sliding_window: int = 0        # llama.attention.sliding_window (every layer), 0: none
    attn_softcap: float = 0.0      # llama.attn_logit_softcapping, 0: none
    final_softcap: float = 0.0     # llama.final_logit_softcapping, 0: none


# BASELINE.json configs 1, 3 and 5.
CONFIGS = {
    "cfg1": ModelSpec("tiny-llama-f32", 2, 256, 4, 2, 64, 688, 4096, 10000.0, max_positions=2048,
                      matrix_type=gguf.F32, embed_type=gguf.F32, output_type=gguf.F32),
    "cfg3": ModelSpec("llama-3.2-1b-shaped", 16, 2048, 32, 8, 64, 8192, 128256, 500000.0,
                      max_positions=131072, tied=True, embed_type=gguf.Q6_K),
    "cfg5": ModelSpec("mistral-7b-shaped", 32, 4096, 32, 8, 128, 14336, 32768, 1000000.0,
                      max_positions=32768),
}


def _rng(seed: int, index: int) -> np.random.Generator:
    return np.random.default_rng([seed, index])


def _f16_bits(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def _random_bytes(rng: np.random.Generator, rows: int, width: int) -> np.ndarray:
    """A fresh [rows, width] uint8 array of uniform random bytes: raw 64-bit
    outputs (little-endian) of an SFC64 stream seeded from rng, several
    times faster than rng.bytes for the gigabytes a 7B-shaped model needs."""
    n = rows * width
    sfc = np.random.SFC64(int(rng.integers(0, 2**63)))
    raw = sfc.random_raw((n + 7) // 8)
    return raw.view(np.uint8)[:n].reshape(rows, width)


def q8_0_blocks(rng: np.random.Generator, n_blocks: int) -> np.ndarray:
    out = np.empty((n_blocks, 34), np.uint8)
    out[:, 0:2] = _f16_bits(np.abs(rng.standard_normal(n_blocks) * 0.01)).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = rng.integers(-127, 128, (n_blocks, 32), dtype=np.int8).view(np.uint8)
    return out


def q4_k_blocks(rng: np.random.Generator, n_blocks: int) -> np.ndarray:
    out = _random_bytes(rng, n_blocks, 144)
    d = np.abs(rng.standard_normal(n_blocks)) * (0.01 / 63)
    dmin = np.abs(rng.standard_normal(n_blocks)) * (0.01 * 7.5 / 63)
    out[:, 0:2] = _f16_bits(d).view(np.uint8).reshape(-1, 2)
    out[:, 2:4] = _f16_bits(dmin).view(np.uint8).reshape(-1, 2)
    return out


def q6_k_blocks(rng: np.random.Generator, n_blocks: int) -> np.ndarray:
    out = _random_bytes(rng, n_blocks, 210)
    d = np.abs(rng.standard_normal(n_blocks)) * (0.02 / 1365)
    out[:, 208:210] = _f16_bits(d).view(np.uint8).reshape(-1, 2)
    return out


def matrix(ggml_type: int, rows: int, cols: int, seed: int, index: int) -> np.ndarray:
    """A [rows, cols] matrix in ggml_type, as the bytes (or f32 values) of the file."""
    rng = _rng(seed, index)
    if ggml_type == gguf.F32:
        return (rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    if ggml_type == gguf.F16:
        return (rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.02)).astype(np.float16)
    values, _ = gguf.BLOCK[ggml_type]
    n = rows * cols // values
    make = {gguf.Q8_0: q8_0_blocks, gguf.Q4_K: q4_k_blocks, gguf.Q6_K: q6_k_blocks}[ggml_type]
    return make(rng, n).reshape(rows, -1)


def write_model(spec: ModelSpec, path: str, seed: int = 6) -> str:
    """Writes spec as a GGUF "llama" file with seeded weights."""
    w = gguf.Writer()
    w.add("general.architecture", "llama")
    w.add("general.name", spec.name)
    w.add("llama.context_length", spec.max_positions)
    w.add("llama.embedding_length", spec.hidden)
    w.add("llama.block_count", spec.n_layers)
    w.add("llama.feed_forward_length", spec.ffn)
    w.add("llama.attention.head_count", spec.heads)
    w.add("llama.attention.head_count_kv", spec.kv_heads)
    w.add("llama.attention.key_length", spec.head_dim)
    w.add("llama.attention.value_length", spec.head_dim)
    w.add("llama.attention.layer_norm_rms_epsilon", float(spec.eps))
    w.add("llama.rope.freq_base", float(spec.theta))
    if spec.sliding_window:
        w.add("llama.attention.sliding_window", int(spec.sliding_window))
    if spec.attn_softcap:
        w.add("llama.attn_logit_softcapping", float(spec.attn_softcap))
    if spec.final_softcap:
        w.add("llama.final_logit_softcapping", float(spec.final_softcap))
    d, qd, kvd = spec.hidden, spec.heads * spec.head_dim, spec.kv_heads * spec.head_dim
    ones = np.ones(d, np.float32)
    index = 0

    def mat(name, t, rows, cols):
        nonlocal index
        index += 1
        w.tensor(name, (rows, cols), t, matrix(t, rows, cols, seed, index))

    mat("token_embd.weight", spec.embed_type, spec.vocab, d)
    w.tensor("output_norm.weight", (d,), gguf.F32, ones)
    if not spec.tied:
        mat("output.weight", spec.output_type, spec.vocab, d)
    for l in range(spec.n_layers):
        p = f"blk.{l}."
        w.tensor(p + "attn_norm.weight", (d,), gguf.F32, ones)
        mat(p + "attn_q.weight", spec.matrix_type, qd, d)
        mat(p + "attn_k.weight", spec.matrix_type, kvd, d)
        mat(p + "attn_v.weight", spec.matrix_type, kvd, d)
        mat(p + "attn_output.weight", spec.matrix_type, d, qd)
        w.tensor(p + "ffn_norm.weight", (d,), gguf.F32, ones)
        mat(p + "ffn_gate.weight", spec.matrix_type, spec.ffn, d)
        mat(p + "ffn_up.weight", spec.matrix_type, spec.ffn, d)
        mat(p + "ffn_down.weight", spec.matrix_type, d, spec.ffn)
    w.write(path)
    return path


def scratch_dir() -> str:
    """A directory for large generated files: RAM-backed when there is one."""
    for d in ("/dev/shm", os.environ.get("TMPDIR", "/tmp"), "/tmp"):
        if d and os.path.isdir(d) and os.access(d, os.W_OK):
            return d
    return "."
