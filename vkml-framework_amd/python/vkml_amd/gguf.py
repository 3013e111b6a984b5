"""GGUF v3 writing, for synthetic models and test fixtures.

The format is llama.cpp's, as the reference reads it (src/io/gguf.cpp:310-387)
and its tests write it (tests/support/gguf_writer.hpp:46-148): magic, version,
tensor and metadata counts, typed key-value metadata, tensor infos with
dimensions fastest first, then tensor data at general.alignment (32).
"""
from __future__ import annotations

import struct
from typing import Iterable

import numpy as np

F32, F16, Q4_0, Q4_1, Q8_0, Q4_K, Q6_K, BF16 = 0, 1, 2, 3, 8, 12, 14, 30
BLOCK = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q4_0: (32, 18), Q4_1: (32, 20), Q8_0: (32, 34),
         Q4_K: (256, 144), Q6_K: (256, 210)}

_T_U32, _T_I32, _T_F32, _T_BOOL, _T_STR, _T_ARR, _T_U64 = 4, 5, 6, 7, 8, 9, 10


def row_bytes(ggml_type: int, cols: int) -> int:
    values, size = BLOCK[ggml_type]
    if cols % values:
        raise ValueError(f"{cols} columns are not whole blocks of {values}")
    return cols // values * size


def read(path: str):
    """(metadata dict, {name: (shape, ggml_type, uint8 data view)}) of a GGUF v2/v3 file."""
    buf = np.memmap(path, np.uint8, mode="r")
    pos = 0

    def take(fmt):
        nonlocal pos
        vals = struct.unpack_from("<" + fmt, buf, pos)
        pos += struct.calcsize("<" + fmt)
        return vals[0] if len(vals) == 1 else vals

    def string():
        nonlocal pos
        n = take("Q")
        s = bytes(buf[pos:pos + n]).decode()
        pos += n
        return s

    scalar = {0: "B", 1: "b", 2: "H", 3: "h", 4: "I", 5: "i", 6: "f", 7: "B", 10: "Q", 11: "q", 12: "d"}

    def value(t):
        if t in scalar:
            v = take(scalar[t])
            return bool(v) if t == 7 else v
        if t == 8:
            return string()
        if t == 9:
            et, n = take("I"), take("Q")
            return [value(et) for _ in range(n)]
        raise ValueError(f"GGUF value type {t}")

    if bytes(buf[:4]) != b"GGUF":
        raise ValueError(f"{path}: not a GGUF file")
    pos = 4
    version, n_tensors, n_kv = take("I"), take("Q"), take("Q")
    if version not in (2, 3):
        raise ValueError(f"{path}: GGUF version {version}")
    meta = {}
    for _ in range(n_kv):
        key = string()
        meta[key] = value(take("I"))
    infos = []
    for _ in range(n_tensors):
        name = string()
        dims = take("I")
        shape = tuple(reversed([take("Q") for _ in range(dims)]))
        infos.append((name, shape, take("I"), take("Q")))
    align = int(meta.get("general.alignment", 32))
    start = (pos + align - 1) // align * align
    tensors = {}
    for name, shape, t, off in infos:
        n = int(np.prod(shape))
        size = row_bytes(t, shape[-1]) * (n // shape[-1])
        tensors[name] = (shape, t, buf[start + off:start + off + size])
    return meta, tensors


class Writer:
    def __init__(self, alignment: int = 32):
        self.alignment = alignment
        self.kv: list[tuple[str, int, object]] = []
        self.tensors: list[tuple[str, tuple[int, ...], int, bytes | np.ndarray]] = []

    def add(self, key: str, value) -> None:
        if isinstance(value, bool):
            self.kv.append((key, _T_BOOL, value))
        elif isinstance(value, int):
            self.kv.append((key, _T_U32 if 0 <= value < 2**32 else _T_U64, value))
        elif isinstance(value, float):
            self.kv.append((key, _T_F32, value))
        elif isinstance(value, str):
            self.kv.append((key, _T_STR, value))
        else:
            raise TypeError(key)

    def tensor(self, name: str, shape: Iterable[int], ggml_type: int, data) -> None:
        """shape row-major (outermost first); data bytes or a uint8/float array."""
        shape = tuple(int(s) for s in shape)
        if isinstance(data, np.ndarray):
            data = np.ascontiguousarray(data)
        n = int(np.prod(shape)) if shape else 1
        want = row_bytes(ggml_type, shape[-1]) * (n // shape[-1])
        got = data.nbytes if isinstance(data, np.ndarray) else len(data)
        if got != want:
            raise ValueError(f"{name}: {got} bytes for {shape} of type {ggml_type}, want {want}")
        self.tensors.append((name, shape, ggml_type, data))

    @staticmethod
    def _str(s: str) -> bytes:
        b = s.encode()
        return struct.pack("<Q", len(b)) + b

    def _value(self, t: int, v) -> bytes:
        if t == _T_U32:
            return struct.pack("<I", v)
        if t == _T_U64:
            return struct.pack("<Q", v)
        if t == _T_F32:
            return struct.pack("<f", v)
        if t == _T_BOOL:
            return struct.pack("<B", int(v))
        if t == _T_STR:
            return self._str(v)
        raise TypeError(t)

    def write(self, path: str) -> None:
        head = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(self.tensors), len(self.kv)))
        for key, t, v in self.kv:
            head += self._str(key) + struct.pack("<I", t) + self._value(t, v)
        offset = 0
        offsets = []
        for name, shape, ggml_type, data in self.tensors:
            offsets.append(offset)
            head += self._str(name) + struct.pack("<I", len(shape))
            for d in reversed(shape):
                head += struct.pack("<Q", d)
            head += struct.pack("<IQ", ggml_type, offset)
            size = data.nbytes if isinstance(data, np.ndarray) else len(data)
            offset += (size + self.alignment - 1) // self.alignment * self.alignment
        pad = (-len(head)) % self.alignment
        with open(path, "wb") as f:
            f.write(head)
            f.write(b"\0" * pad)
            for (name, shape, ggml_type, data), off in zip(self.tensors, offsets):
                size = data.nbytes if isinstance(data, np.ndarray) else len(data)
                f.write(memoryview(data).cast("B") if isinstance(data, np.ndarray) else data)
                f.write(b"\0" * ((-size) % self.alignment))
