"""numpy binding of the CPU oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker. The product never imports it.
Each function forwards to the C restatement in vkml_oracle.c / oracle_model.c,
which cite the reference file:line they follow.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

Q8_0, Q4_0, Q4_1 = 0, 1, 2
GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q4_1, GGML_Q8_0, GGML_Q4_K, GGML_Q6_K, GGML_BF16 = 0, 1, 2, 3, 8, 12, 14, 30
T_F32, T_F16, T_BF16, T_Q8, T_Q4, T_Q4_1 = 0, 1, 2, 3, 4, 5

_lib = None


def build() -> None:
    """Compile liboracle.so with its Makefile (gcc, -ffp-contract=off)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


def _p(a):
    return a.ctypes.data_as(C.c_void_p) if a is not None else None


def _declare(L):
    vp, i64, i32, f32 = C.c_void_p, C.c_int64, C.c_int, C.c_float
    sig = {
        "orc_last_error": (C.c_char_p, []),
        "orc_set_threads": (None, [i32]),
        "orc_f16_to_f32": (f32, [C.c_uint16]),
        "orc_f32_to_f16": (C.c_uint16, [f32]),
        "orc_cast_f32_to_f16": (None, [vp, vp, i64]),
        "orc_cast_f16_to_f32": (None, [vp, vp, i64]),
        "orc_dequantize_ggml": (i64, [i32, vp, i64, vp]),
        "orc_ggml_row_bytes": (i64, [i32, i64]),
        "orc_load_quantized": (i32, [i32, vp, i64, i64, vp, vp]),
        "orc_load_q8": (i32, [i32, vp, i64, i64, vp, vp]),
        "orc_quantize": (None, [i32, i32, vp, i64, i64, vp, vp]),
        "orc_dequantize": (None, [i32, i32, vp, vp, i64, i64, vp]),
        "orc_gemv_dot": (None, [i32, i32, vp, vp, i64, vp, vp, i64, i64, vp]),
        "orc_matmul_dot": (None, [i32, i32, vp, vp, i64, vp, vp, i64, i64, vp]),
        "orc_gemv_float": (None, [i32, i32, vp, i64, vp, vp, i64, i64, vp]),
        "orc_matmul_float": (None, [i32, i32, vp, i64, vp, vp, i64, i64, vp]),
        "orc_rms_norm": (None, [vp, vp, i64, i64, f32, vp]),
        "orc_rope_table": (None, [i64, i64, f32, vp]),
        "orc_rope": (None, [vp, vp, i64, i64, i64, i64, i64, i64, i32, vp]),
        "orc_expf_array": (None, [vp, vp, i64]),
        "orc_silu": (None, [vp, vp, i64]),
        "orc_binary": (None, [i32, vp, vp, i64, i64, vp]),
        "orc_argmax": (C.c_int32, [vp, i64]),
        "orc_embedding_quantized": (None, [i32, vp, vp, i64, i64, vp, i64, vp]),
        "orc_attend_decode": (None, [vp, i64, vp, vp, i32, i64, i64, i64, i64, i64, f32, vp]),
        "orc_attention_prefill": (None, [vp, i64, i64, vp, vp, i32, i64, i64, i64, i64, i64, f32, vp]),
        "orc_attention_sliding": (None, [vp, i64, i64, vp, vp, vp, vp, i32, i64, i64, i64, i64, i64, i64, f32, vp]),
        "orc_model_load_ex": (vp, [C.c_char_p, i64, i32, i32, i64]),
        "orc_model_load_opts": (vp, [C.c_char_p, i64, i32, i32, i64, i64, f32, f32]),
        "orc_token_logprobs": (f32, [vp, i64, i32, i32, vp, vp]),
        "orc_model_set_attention_noise": (None, [vp, i32]),
        "orc_model_ring": (i64, [vp]),
        "orc_model_load": (vp, [C.c_char_p, i64, i32, i32]),
        "orc_model_free": (None, [vp]),
        "orc_model_forward": (i32, [vp, vp, i64, vp]),
        "orc_model_forward_all": (i32, [vp, vp, i64, vp]),
        "orc_model_set_max_score_bytes": (None, [vp, i64]),
        "orc_model_position": (i64, [vp]),
        "orc_model_set_position": (i32, [vp, i64]),
        "orc_model_rewind": (i64, [vp, i64]),
        "orc_model_reset": (None, [vp]),
        "orc_model_vocab": (i64, [vp]),
        "orc_model_dims": (None, [vp, vp]),
        "orc_model_k_cache": (vp, [vp, i32]),
        "orc_model_v_cache": (vp, [vp, i32]),
        "orc_model_set_kv": (i32, [vp, i32, vp, vp]),
        "orc_model_reference_f64": (i32, [C.c_char_p, vp, i64, vp]),
        "orc_sampler_new": (vp, [f32, i32, f32, C.c_uint64, f32, f32, f32, f32]),
        "orc_sampler_free": (None, [vp]),
        "orc_sampler_sample": (i32, [vp, vp, i64, vp, i64]),
        "orc_sampler_draw_u64": (C.c_uint64, [vp]),
        "orc_sampler_draw_uniform": (C.c_double, [vp, C.c_double]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))


def last_error() -> str:
    return lib().orc_last_error().decode()


def f32_to_f16(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, np.uint16)
    lib().orc_cast_f32_to_f16(_p(x), _p(y), x.size)
    return y


def f16_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    y = np.empty(h.shape, np.float32)
    lib().orc_cast_f16_to_f32(_p(h), _p(y), h.size)
    return y


def dequantize_ggml(ggml_type: int, blocks: bytes) -> np.ndarray:
    b = np.frombuffer(bytes(blocks), np.uint8)
    per = {GGML_Q8_0: (32, 34), GGML_Q4_0: (32, 18), GGML_Q4_1: (32, 20), GGML_Q4_K: (256, 144), GGML_Q6_K: (256, 210)}
    values, size = per[ggml_type]
    out = np.empty(len(b) // size * values, np.float32)
    n = lib().orc_dequantize_ggml(ggml_type, _p(b), len(b), _p(out))
    if n < 0:
        raise ValueError("oracle: cannot decode type %d" % ggml_type)
    return out


def load_quantized(ggml_type: int, data: bytes, rows: int, cols: int):
    """(quant, words uint32, halves uint16) as Gguf::load_quantized repacks them."""
    d = np.frombuffer(bytes(data), np.uint8)
    q8 = ggml_type == GGML_Q8_0
    words = np.empty(rows * cols // (4 if q8 else 8), np.uint32)
    pairs = ggml_type in (GGML_Q4_1, GGML_Q4_K)
    halves = np.empty(rows * cols // 32 * (2 if pairs else 1), np.uint16)
    quant = lib().orc_load_quantized(ggml_type, _p(d), rows, cols, _p(words), _p(halves))
    if quant < 0:
        raise ValueError("oracle: cannot load type %d" % ggml_type)
    return quant, words, halves


def load_q8(ggml_type: int, data: bytes, rows: int, cols: int):
    d = np.frombuffer(bytes(data), np.uint8)
    words = np.empty(rows * cols // 4, np.uint32)
    halves = np.empty(rows * cols // 32, np.uint16)
    if lib().orc_load_q8(ggml_type, _p(d), rows, cols, _p(words), _p(halves)) < 0:
        raise ValueError("oracle: cannot requantize type %d" % ggml_type)
    return words, halves


def quantize(quant: int, x, f16_scales: bool):
    """quantize.comp: (words uint32, scales f32 or uint16 f16 bits)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = (1, x.size) if x.ndim == 1 else x.shape
    words = np.empty(rows * cols // (4 if quant == Q8_0 else 8), np.uint32)
    n_scales = rows * cols // 32 * (2 if quant == Q4_1 else 1)
    scales = np.empty(n_scales, np.uint16 if f16_scales else np.float32)
    lib().orc_quantize(quant, int(f16_scales), _p(x), rows, cols, _p(words), _p(scales))
    return words, scales


def dequantize(quant: int, words, scales, rows: int, cols: int) -> np.ndarray:
    words = np.ascontiguousarray(words, dtype=np.uint32)
    scales = np.ascontiguousarray(scales)
    out = np.empty((rows, cols), np.float32)
    lib().orc_dequantize(quant, int(scales.dtype == np.uint16), _p(words), _p(scales), rows, cols, _p(out))
    return out


def gemv_dot(quant, a_words, a_scales, M, b_words, b_scales, N, K) -> np.ndarray:
    a_words = np.ascontiguousarray(a_words, dtype=np.uint32)
    a_scales = np.ascontiguousarray(a_scales, dtype=np.float32)
    b_words = np.ascontiguousarray(b_words, dtype=np.uint32)
    b_scales = np.ascontiguousarray(b_scales)
    out = np.empty((M, N), np.float32)
    lib().orc_gemv_dot(quant, int(b_scales.dtype == np.uint16), _p(a_words), _p(a_scales), M,
                       _p(b_words), _p(b_scales), N, K, _p(out))
    return out


def matmul_dot(quant, a_words, a_scales, M, b_words, b_scales, N, K) -> np.ndarray:
    a_words = np.ascontiguousarray(a_words, dtype=np.uint32)
    a_scales = np.ascontiguousarray(a_scales, dtype=np.float32)
    b_words = np.ascontiguousarray(b_words, dtype=np.uint32)
    b_scales = np.ascontiguousarray(b_scales)
    out = np.empty((M, N), np.float32)
    lib().orc_matmul_dot(quant, int(b_scales.dtype == np.uint16), _p(a_words), _p(a_scales), M,
                         _p(b_words), _p(b_scales), N, K, _p(out))
    return out


def gemv_float(b_type, a, b, b_scales, N, K) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32).reshape(-1, K)
    b = np.ascontiguousarray(b)
    sc = None if b_scales is None else np.ascontiguousarray(b_scales)
    f16 = int(sc is not None and sc.dtype == np.uint16)
    out = np.empty((a.shape[0], N), np.float32)
    lib().orc_gemv_float(b_type, f16, _p(a), a.shape[0], _p(b), _p(sc), N, K, _p(out))
    return out


def matmul_float(b_type, a, b, b_scales, N, K) -> np.ndarray:
    """matmul.comp with b [N, K] transposed: a [M, K] f32, sums in k order."""
    a = np.ascontiguousarray(a, dtype=np.float32).reshape(-1, K)
    b = np.ascontiguousarray(b)
    sc = None if b_scales is None else np.ascontiguousarray(b_scales)
    f16 = int(sc is not None and sc.dtype == np.uint16)
    out = np.empty((a.shape[0], N), np.float32)
    lib().orc_matmul_float(b_type, f16, _p(a), a.shape[0], _p(b), _p(sc), N, K, _p(out))
    return out


def attention_prefill(q, k_cache, v_cache, kv_len: int, max_score_bytes: int = 64 << 20, softcap: float = 0.0) -> np.ndarray:
    """q [heads, q_len, hd] f32; caches [kv_heads, capacity, hd] f32 or uint16
    (f16 bits); query i at key position kv_len - q_len + i."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    heads, q_len, hd = q.shape
    kv_heads, capacity = k_cache.shape[0], k_cache.shape[1]
    f16 = int(k_cache.dtype == np.uint16)
    k = np.ascontiguousarray(k_cache)
    v = np.ascontiguousarray(v_cache)
    out = np.empty((heads, q_len, hd), np.float32)
    lib().orc_attention_prefill(_p(q), heads, q_len, _p(k), _p(v), f16, kv_heads, capacity, hd, kv_len,
                                max_score_bytes, softcap, _p(out))
    return out


def attention_sliding(q, k, v, k_ring, v_ring, start: int, window: int, softcap: float = 0.0,
                      max_score_bytes: int = 64 << 20) -> np.ndarray:
    """detail::sliding_attention: q [heads, t, hd] f32 at positions start..;
    k, v [kv_heads, t, hd] in the rings' type (f32, or f16 bits as uint16),
    appended in place to k_ring / v_ring [kv_heads, ring, hd]."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    heads, t, hd = q.shape
    kv_heads, ring = k_ring.shape[0], k_ring.shape[1]
    f16 = int(k_ring.dtype == np.uint16)
    k, v = np.ascontiguousarray(k), np.ascontiguousarray(v)
    assert k_ring.flags.c_contiguous and v_ring.flags.c_contiguous
    out = np.empty((heads, t, hd), np.float32)
    lib().orc_attention_sliding(_p(q), heads, t, _p(k), _p(v), _p(k_ring), _p(v_ring), f16, kv_heads, ring, hd, start,
                                window, max_score_bytes, softcap, _p(out))
    return out


def rms_norm(x, w, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = (1, x.size) if x.ndim == 1 else x.shape
    out = np.empty_like(x)
    lib().orc_rms_norm(_p(x), _p(w), rows, cols, eps, _p(out))
    return out


def rope_table(positions: int, head_dim: int, theta: float) -> np.ndarray:
    t = np.empty((positions, head_dim // 2, 2), np.float32)
    lib().orc_rope_table(positions, head_dim, theta, _p(t))
    return t


def rope(x, table, start_pos: int, style: int = 0) -> np.ndarray:
    """x [..., seq, heads, dim]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    seq, heads, dim = x.shape[-3:]
    rows = x.size // dim
    table = np.ascontiguousarray(table, dtype=np.float32)
    out = np.empty_like(x)
    lib().orc_rope(_p(x), _p(table), rows, heads, seq, dim, table.shape[1], start_pos, style, _p(out))
    return out


def expf(x) -> np.ndarray:
    """The exp the oracle and the GPU kernels share (orc_expf)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().orc_expf_array(_p(x), _p(y), x.size)
    return y


def silu(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().orc_silu(_p(x), _p(y), x.size)
    return y


def argmax(x) -> int:
    x = np.ascontiguousarray(x, dtype=np.float32)
    return int(lib().orc_argmax(_p(x), x.size))


def embedding_quantized(quant, words, halves, vocab, dim, ids) -> np.ndarray:
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    words = np.ascontiguousarray(words, dtype=np.uint32)
    halves = np.ascontiguousarray(halves, dtype=np.uint16)
    out = np.empty((ids.size, dim), np.float32)
    lib().orc_embedding_quantized(quant, _p(words), _p(halves), vocab, dim, _p(ids), ids.size, _p(out))
    return out


def attend_decode(q, k_cache, v_cache, kv_start: int, kv_len: int, softcap: float = 0.0) -> np.ndarray:
    """q [heads, hd] f32; caches [kv_heads, capacity, hd] f32 or uint16 (f16 bits)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    heads, hd = q.shape[0], q.shape[-1]
    kv_heads, capacity = k_cache.shape[0], k_cache.shape[1]
    f16 = int(k_cache.dtype == np.uint16)
    k = np.ascontiguousarray(k_cache)
    v = np.ascontiguousarray(v_cache)
    out = np.empty((heads, hd), np.float32)
    lib().orc_attend_decode(_p(q), heads, _p(k), _p(v), f16, kv_heads, capacity, hd, kv_start, kv_len,
                            softcap, _p(out))
    return out


class Model:
    """orc_model: the reference's Llama::run restated on the CPU."""

    def __init__(self, gguf_path: str, context: int, kv_f16: bool = True, int_dot: bool = True,
                 sliding_extra_rows: int = 1024, sliding_window: int = 0, attn_softcap: float = 0.0,
                 final_softcap: float = 0.0):
        self._h = lib().orc_model_load_opts(gguf_path.encode(), context, int(kv_f16), int(int_dot), sliding_extra_rows,
                                            int(sliding_window), float(attn_softcap), float(final_softcap))
        if not self._h:
            raise RuntimeError(last_error())
        self.vocab = int(lib().orc_model_vocab(self._h))
        dims = np.zeros(8, np.int64)
        lib().orc_model_dims(self._h, _p(dims))
        (_, self.hidden, self.ffn, self.layers, self.heads, self.kv_heads, self.head_dim, self.context) = (int(x) for x in dims)
        self.kv_f16 = bool(kv_f16)
        self.ring = int(lib().orc_model_ring(self._h))  # rows of each cache

    def forward(self, tokens) -> np.ndarray:
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.empty(self.vocab, np.float32)
        if lib().orc_model_forward(self._h, _p(t), t.size, _p(out)) != 0:
            raise RuntimeError(last_error())
        return out

    def set_attention_noise(self, ulps: int) -> None:
        """Test instrumentation: decode attention outputs moved by up to
        `ulps` ulps before they are quantized (0: off)."""
        lib().orc_model_set_attention_noise(self._h, int(ulps))

    def forward_all(self, tokens) -> np.ndarray:
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.empty((t.size, self.vocab), np.float32)
        if lib().orc_model_forward_all(self._h, _p(t), t.size, _p(out)) != 0:
            raise RuntimeError(last_error())
        return out

    def set_max_score_bytes(self, n: int) -> None:
        lib().orc_model_set_max_score_bytes(self._h, int(n))

    @property
    def position(self) -> int:
        return int(lib().orc_model_position(self._h))

    def set_position(self, position: int) -> None:
        if lib().orc_model_set_position(self._h, position) != 0:
            raise RuntimeError("position %d outside the context" % position)

    def rewind(self, position: int) -> int:
        r = lib().orc_model_rewind(self._h, position)
        if r < 0:
            raise RuntimeError(last_error())
        return int(r)

    def reset(self) -> None:
        lib().orc_model_reset(self._h)

    def kv_cache(self, layer: int):
        """Layer `layer`'s caches [kv_heads, context, head_dim] as the model
        holds them (f16 bits as uint16, or f32), copied."""
        k = lib().orc_model_k_cache(self._h, layer)
        v = lib().orc_model_v_cache(self._h, layer)
        n = self.kv_heads * self.ring * self.head_dim
        t = C.c_uint16 if self.kv_f16 else C.c_float
        shape = (self.kv_heads, self.ring, self.head_dim)
        return tuple(np.ctypeslib.as_array(C.cast(p, C.POINTER(t)), (n,)).reshape(shape).copy() for p in (k, v))

    def set_kv(self, layer: int, k, v) -> None:
        """Layer `layer`'s caches from k and v (the kv_cache layout)."""
        dt = np.uint16 if self.kv_f16 else np.float32
        shape = (self.kv_heads, self.ring, self.head_dim)
        k, v = np.ascontiguousarray(k, dt), np.ascontiguousarray(v, dt)
        assert k.shape == shape and v.shape == shape, (k.shape, shape)
        if lib().orc_model_set_kv(self._h, layer, _p(k), _p(v)) != 0:
            raise RuntimeError("set_kv: layer %d" % layer)

    def close(self) -> None:
        if self._h:
            lib().orc_model_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def reference_f64(gguf_path: str, tokens) -> np.ndarray:
    t = np.ascontiguousarray(tokens, dtype=np.int32)
    # vocab from a throwaway load is wasteful; read it from the forward's size instead.
    m = Model(gguf_path, max(1, t.size), kv_f16=False)
    vocab = m.vocab
    m.close()
    out = np.empty(vocab, np.float64)
    if lib().orc_model_reference_f64(gguf_path.encode(), _p(t), t.size, _p(out)) != 0:
        raise RuntimeError(last_error())
    return out


def token_logprobs(logits, token: int, top: int):
    """(logprob, top ids, top logprobs) of the reference's token_logprobs."""
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    ti = np.zeros(max(top, 1), np.int32)
    tl = np.zeros(max(top, 1), np.float32)
    lp = lib().orc_token_logprobs(_p(lg), lg.size, int(token), int(top), _p(ti), _p(tl))
    k = min(top, lg.size)
    return float(lp), ti[:k].copy(), tl[:k].copy()


class Sampler:
    """orc_sampler: the reference's Sampler (src/io/sampling.cpp:17-139)."""

    def __init__(self, temperature=0.0, top_k=0, top_p=1.0, seed=0, repetition_penalty=1.0, min_p=0.0,
                 frequency_penalty=0.0, presence_penalty=0.0):
        self._h = lib().orc_sampler_new(temperature, top_k, top_p, seed, repetition_penalty, min_p,
                                        frequency_penalty, presence_penalty)

    def sample(self, logits, previous=()) -> int:
        lg = np.ascontiguousarray(logits, dtype=np.float32)
        pv = np.ascontiguousarray(previous, dtype=np.int32)
        return int(lib().orc_sampler_sample(self._h, _p(lg), lg.size, _p(pv), pv.size))

    def draw_u64(self) -> int:
        return int(lib().orc_sampler_draw_u64(self._h))

    def draw_uniform(self, total: float) -> float:
        return float(lib().orc_sampler_draw_uniform(self._h, total))

    def close(self) -> None:
        if self._h:
            lib().orc_sampler_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
