"""ctypes binding of libvkml.so's C API (include/vkml_llama.h): vkml::Llama
from Python. Raises when the in-tree library is missing."""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from .hip import LIB_DIR

LIB_PATH = os.path.join(LIB_DIR, "libvkml.so")

i32, i64, u32, u64, vp = C.c_int32, C.c_int64, C.c_uint32, C.c_uint64, C.c_void_p


class Options(C.Structure):
    _fields_ = [("kv_cache_f16", i32), ("quantize", i32), ("integer_dot", i32), ("use_graphs", i32),
                ("device_name", C.c_char_p), ("prompt_score_bytes", i64), ("sliding_extra_rows", i64),
                ("fast_attention", i32), ("sliding_window", i64), ("attn_logit_softcap", C.c_float),
                ("final_logit_softcap", C.c_float)]


class SamplingOptions(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_k", i32), ("top_p", C.c_float), ("repetition_penalty", C.c_float),
                ("min_p", C.c_float), ("frequency_penalty", C.c_float), ("presence_penalty", C.c_float), ("seed", u64)]


class Config(C.Structure):
    _fields_ = [(n, i64) for n in ("vocab_size", "hidden_size", "intermediate_size", "num_layers", "num_heads",
                                   "num_kv_heads", "head_dim", "max_positions")] + \
               [("rms_norm_eps", C.c_float), ("rope_theta", C.c_float), ("tie_word_embeddings", i32), ("rope_interleaved", i32)]


P = C.POINTER
SIGNATURES = {
    "vkml_llama_default_options": (None, [P(Options)]),
    "vkml_llama_load": (C.c_int, [C.c_char_p, i64, P(Options), P(vp)]),
    "vkml_llama_free": (None, [vp]),
    "vkml_llama_shutdown": (C.c_int, []),
    "vkml_llama_get_config": (C.c_int, [vp, P(Config)]),
    "vkml_llama_read_config": (C.c_int, [C.c_char_p, P(Config)]),
    "vkml_llama_context_length": (i64, [vp]),
    "vkml_llama_position": (i64, [vp]),
    "vkml_llama_kv_cache_bytes": (i64, [vp]),
    "vkml_llama_forward": (C.c_int, [vp, vp, i64, vp]),
    "vkml_llama_forward_all": (C.c_int, [vp, vp, i64, vp]),
    "vkml_llama_generate_greedy": (C.c_int, [vp, i32, i64, vp]),
    "vkml_llama_reset": (C.c_int, [vp]),
    "vkml_llama_rewind": (C.c_int, [vp, i64, P(i64)]),
    "vkml_llama_advance": (C.c_int, [vp, i64]),
    "vkml_llama_read_kv_cache": (C.c_int, [vp, i64, vp, vp, u64]),
    "vkml_llama_set_profiling": (C.c_int, [i32]),
    "vkml_llama_profile": (C.c_int, [vp, u32, vp, vp, u32, P(u32)]),
    "vkml_llama_reset_profile": (C.c_int, []),
    "vkml_llama_synchronize": (C.c_int, []),
    "vkml_sampling_default_options": (None, [vp]),
    "vkml_sampler_create": (C.c_int, [vp, P(vp)]),
    "vkml_sampler_free": (None, [vp]),
    "vkml_sampler_sample": (C.c_int, [vp, vp, i64, vp, i64, vp]),
    "vkml_session_create": (C.c_int, [vp, vp, i64, P(vp)]),
    "vkml_session_free": (None, [vp]),
    "vkml_session_generate": (C.c_int, [vp, vp, i64, vp, i64, vp, i64, vp, vp]),
    "vkml_session_cached": (i64, [vp, vp, i64]),
    "vkml_session_generate_logprobs": (C.c_int, [vp, vp, i64, vp, i64, i32, vp, i64, vp, vp, vp, vp, vp]),
    "vkml_session_score": (C.c_int, [vp, vp, i64, i32, vp, vp, vp]),
    "vkml_token_logprobs": (C.c_int, [vp, i64, i32, i32, vp, vp, vp]),
}

_lib = None


class VkmlError(RuntimeError):
    pass


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise VkmlError(f"{LIB_PATH} is missing: build it (python -c 'import __graft_entry__ as g; g.build()')")
        _lib = C.CDLL(LIB_PATH)
        _lib.vkml_llama_last_error.restype = C.c_char_p
        _lib.vkml_llama_last_error.argtypes = []
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(_lib, name)
            fn.restype = res
            fn.argtypes = args
    return _lib


def _check(status: int) -> None:
    if status != 0:
        raise VkmlError(lib().vkml_llama_last_error().decode())


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(vp)


class Llama:
    def __init__(self, path: str, context: int, kv_f16: bool = False, quantize: int = -1, integer_dot: bool = True,
                 use_graphs: bool = True, prompt_score_bytes: int = 0, sliding_extra_rows: int = -1,
                 fast_attention: bool = False, sliding_window: int = 0, attn_softcap: float = 0.0, final_softcap: float = 0.0):
        o = Options()
        lib().vkml_llama_default_options(C.byref(o))
        o.kv_cache_f16, o.quantize, o.integer_dot = int(kv_f16), int(quantize), int(integer_dot)
        o.use_graphs = int(use_graphs)
        if prompt_score_bytes:
            o.prompt_score_bytes = int(prompt_score_bytes)
        if sliding_extra_rows >= 0:
            o.sliding_extra_rows = int(sliding_extra_rows)
        o.fast_attention = int(fast_attention)
        o.sliding_window = int(sliding_window)
        o.attn_logit_softcap, o.final_logit_softcap = float(attn_softcap), float(final_softcap)
        self._h = vp()
        _check(lib().vkml_llama_load(path.encode(), int(context), C.byref(o), C.byref(self._h)))
        cfg = Config()
        _check(lib().vkml_llama_get_config(self._h, C.byref(cfg)))
        self.config = {f: getattr(cfg, f) for f, _ in Config._fields_}
        self.vocab = int(cfg.vocab_size)
        self.kv_f16 = kv_f16

    def forward(self, tokens) -> np.ndarray:
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.empty(self.vocab, np.float32)
        _check(lib().vkml_llama_forward(self._h, _ptr(t), t.size, _ptr(out)))
        return out

    def forward_all(self, tokens) -> np.ndarray:
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.empty((t.size, self.vocab), np.float32)
        _check(lib().vkml_llama_forward_all(self._h, _ptr(t), t.size, _ptr(out)))
        return out

    def generate_greedy(self, first: int, count: int) -> np.ndarray:
        out = np.empty(max(int(count), 0), np.int32)
        _check(lib().vkml_llama_generate_greedy(self._h, int(first), int(count), _ptr(out)))
        return out

    @property
    def position(self) -> int:
        return int(lib().vkml_llama_position(self._h))

    @property
    def context_length(self) -> int:
        return int(lib().vkml_llama_context_length(self._h))

    @property
    def kv_cache_bytes(self) -> int:
        return int(lib().vkml_llama_kv_cache_bytes(self._h))

    def reset(self) -> None:
        _check(lib().vkml_llama_reset(self._h))

    def rewind(self, position: int) -> int:
        out = i64()
        _check(lib().vkml_llama_rewind(self._h, int(position), C.byref(out)))
        return int(out.value)

    def advance(self, position: int) -> None:
        """Llama::advance: skip to position without running the tokens between."""
        _check(lib().vkml_llama_advance(self._h, int(position)))

    def read_kv_cache(self, layer: int):
        c = self.config
        rows = int(lib().vkml_llama_kv_cache_bytes(self._h)) // (2 * c["num_layers"] * c["num_kv_heads"] * c["head_dim"] * (2 if self.kv_f16 else 4))
        shape = (c["num_kv_heads"], rows, c["head_dim"])
        dt = np.uint16 if self.kv_f16 else np.float32
        k, v = np.empty(shape, dt), np.empty(shape, dt)
        _check(lib().vkml_llama_read_kv_cache(self._h, int(layer), _ptr(k), _ptr(v), k.nbytes))
        return k, v

    def close(self) -> None:
        if self._h:
            lib().vkml_llama_free(self._h)
            self._h = vp()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def read_config(path: str) -> dict:
    """LlamaConfig::from_gguf: a GGUF file's model config, from its header."""
    cfg = Config()
    _check(lib().vkml_llama_read_config(path.encode(), C.byref(cfg)))
    return {f: getattr(cfg, f) for f, _ in Config._fields_}


def set_profiling(on: bool) -> None:
    _check(lib().vkml_llama_set_profiling(int(on)))


def reset_profile() -> None:
    _check(lib().vkml_llama_reset_profile())


def synchronize() -> None:
    _check(lib().vkml_llama_synchronize())


def profile() -> list[tuple[str, int, float]]:
    count = u32()
    _check(lib().vkml_llama_profile(None, 0, None, None, 0, C.byref(count)))
    n = count.value
    stride = 64
    names = C.create_string_buffer(stride * max(n, 1))
    calls = np.zeros(max(n, 1), np.uint64)
    ms = np.zeros(max(n, 1), np.float64)
    _check(lib().vkml_llama_profile(names, stride, _ptr(calls), _ptr(ms), n, C.byref(count)))
    raw = names.raw
    return [(raw[i * stride:(i + 1) * stride].split(b"\0")[0].decode(), int(calls[i]), float(ms[i])) for i in range(n)]


def shutdown() -> None:
    _check(lib().vkml_llama_shutdown())


class Sampler:
    """vkml::Sampler (host code: no device needed)."""

    def __init__(self, **options):
        o = SamplingOptions()
        lib().vkml_sampling_default_options(C.byref(o))
        for k, v in options.items():
            setattr(o, k, v)
        self._h = vp()
        _check(lib().vkml_sampler_create(C.byref(o), C.byref(self._h)))

    def sample(self, logits, previous=()) -> int:
        lg = np.ascontiguousarray(logits, dtype=np.float32)
        pv = np.ascontiguousarray(previous, dtype=np.int32)
        out = i32()
        _check(lib().vkml_sampler_sample(self._h, _ptr(lg), lg.size, _ptr(pv), pv.size, C.byref(out)))
        return int(out.value)

    def close(self) -> None:
        if self._h:
            lib().vkml_sampler_free(self._h)
            self._h = vp()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def token_logprobs(logits, token: int, top: int):
    """vkml::token_logprobs (host code): (logprob, top ids, top logprobs)."""
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    lp = np.empty(1, np.float32)
    ti = np.empty(max(top, 1), np.int32)
    tl = np.empty(max(top, 1), np.float32)
    _check(lib().vkml_token_logprobs(_ptr(lg), lg.size, int(token), int(top), _ptr(lp), _ptr(ti), _ptr(tl)))
    return float(lp[0]), ti[:top].copy(), tl[:top].copy()


class Session:
    """vkml::Session: requests against one model, reusing its KV cache."""

    STOP, LENGTH = 0, 1

    def __init__(self, model: Llama, stop=()):
        st = np.ascontiguousarray(stop, dtype=np.int32)
        self.model = model
        self._h = vp()
        _check(lib().vkml_session_create(model._h, _ptr(st), st.size, C.byref(self._h)))

    def generate(self, prompt, sampler: Sampler, max_tokens: int):
        """(reply tokens, finish: STOP or LENGTH)."""
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        cap = max(max_tokens, 0) if max_tokens >= 0 else self.model.context_length
        out = np.empty(max(cap, 1), np.int32)
        n, fin = i64(), i32()
        _check(lib().vkml_session_generate(self._h, _ptr(p), p.size, sampler._h, int(max_tokens), _ptr(out), cap,
                                           C.byref(n), C.byref(fin)))
        return out[:n.value].copy(), int(fin.value)

    def generate_logprobs(self, prompt, sampler: Sampler, max_tokens: int, top: int):
        """(reply tokens, finish, logprobs [n], top ids [n, top], top logprobs [n, top])."""
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        cap = max(max_tokens, 0) if max_tokens >= 0 else self.model.context_length
        out = np.empty(max(cap, 1), np.int32)
        lp = np.empty(max(cap, 1), np.float32)
        ti = np.empty((max(cap, 1), max(top, 1)), np.int32)
        tl = np.empty((max(cap, 1), max(top, 1)), np.float32)
        n, fin = i64(), i32()
        _check(lib().vkml_session_generate_logprobs(self._h, _ptr(p), p.size, sampler._h, int(max_tokens), int(top), _ptr(out),
                                                    cap, C.byref(n), C.byref(fin), _ptr(lp), _ptr(ti), _ptr(tl)))
        k = n.value
        return out[:k].copy(), int(fin.value), lp[:k].copy(), ti[:k, :top].copy(), tl[:k, :top].copy()

    def score(self, prompt, top: int):
        """(logprobs [n] (NaN first), top ids [n, top], top logprobs [n, top])."""
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        lp = np.empty(p.size, np.float32)
        ti = np.empty((p.size, max(top, 1)), np.int32)
        tl = np.empty((p.size, max(top, 1)), np.float32)
        _check(lib().vkml_session_score(self._h, _ptr(p), p.size, int(top), _ptr(lp), _ptr(ti), _ptr(tl)))
        return lp, ti[:, :top].copy(), tl[:, :top].copy()

    @property
    def cached(self) -> np.ndarray:
        n = lib().vkml_session_cached(self._h, None, 0)
        out = np.empty(max(n, 1), np.int32)
        lib().vkml_session_cached(self._h, _ptr(out), n)
        return out[:n].copy()

    def close(self) -> None:
        if self._h:
            lib().vkml_session_free(self._h)
            self._h = vp()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
