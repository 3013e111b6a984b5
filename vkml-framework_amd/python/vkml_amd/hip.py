"""ctypes binding of libvkml_hip.so (include/vkml_hip.h): the kernels and
runtime of the MI355X build, callable from Python with numpy arrays.

Loading fails loudly when the in-tree library is missing: there is no
fallback to any other implementation.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

PKG = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
LIB_DIR = os.path.join(PKG, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libvkml_hip.so")

F32, F16, BF16, Q8_0, Q4_0, Q4_1, Q4_K, I32 = 0, 1, 2, 3, 4, 5, 6, 7

u32, i32, f32, u64, vp = C.c_uint32, C.c_int32, C.c_float, C.c_uint64, C.c_void_p


class DeviceInfo(C.Structure):
    _fields_ = [("name", C.c_char * 256), ("arch", C.c_char * 64), ("driver", C.c_char * 64),
                ("global_memory_bytes", u64), ("compute_units", u32), ("wave_size", u32),
                ("max_threads_per_block", u32), ("max_block_dims", u32 * 3), ("max_grid_dims", u32 * 3),
                ("lds_bytes_per_block", u32), ("l2_bytes", u32), ("clock_khz", u32), ("memory_clock_khz", u32),
                ("memory_bus_bits", u32), ("integer_dot_product", i32), ("timestamps", i32),
                ("timestamp_period_ns", C.c_double)]


class KernelTime(C.Structure):
    _fields_ = [("name", C.c_char * 48), ("calls", u64), ("milliseconds", C.c_double)]


def _struct(name, fields):
    return type(name, (C.Structure,), {"_fields_": [(f, t) for f, t in fields]})


QuantizeParams = _struct("QuantizeParams", [("blocks", u32), ("src_type", u32), ("quant", u32), ("scale_type", u32)])
DequantizeParams = _struct("DequantizeParams", [("count", u32), ("quant", u32), ("scale_type", u32), ("cols", u32)])
GemvDotParams = _struct("GemvDotParams", [("m", u32), ("n", u32), ("k", u32), ("b_type", u32), ("scale_type", u32)])
GemvParams = _struct("GemvParams", [("m", u32), ("n", u32), ("k", u32), ("b_type", u32), ("scale_type", u32),
                                    ("b_stride", u32), ("b_group", u32), ("batches", u32)])
MatmulParams = _struct("MatmulParams", [("m", u32), ("n", u32), ("k", u32), ("b_stride", u32), ("b_group", u32),
                                        ("batches", u32), ("b_transposed", u32), ("b_type", u32), ("scale_type", u32),
                                        ("causal", u32), ("causal_offset", u32)])
RmsNormParams = _struct("RmsNormParams", [("rows", u32), ("cols", u32), ("eps", f32)])
SoftmaxParams = _struct("SoftmaxParams", [("rows", u32), ("cols", u32), ("scale", f32), ("causal", u32),
                                          ("q_len", u32), ("offset", u32), ("window", u32), ("softcap", f32),
                                          ("ring", u32)])
RopeParams = _struct("RopeParams", [("pairs", u32), ("half_dim", u32), ("dim", u32), ("heads", u32), ("seq", u32),
                                    ("start_pos", u32), ("copies", u32), ("style", u32)])
CopyRowsParams = _struct("CopyRowsParams", [("count", u32), ("block", u32), ("src_stride", u32), ("src_start", u32),
                                            ("dst_stride", u32), ("dst_start", u32)])
PermuteParams = _struct("PermuteParams", [("rank", u32), ("count", u32), ("in_shape", u32 * 6), ("dims", u32 * 6)])
EmbeddingParams = _struct("EmbeddingParams", [("count", u32), ("dim", u32), ("vocab", u32), ("table_type", u32),
                                              ("scale_type", u32)])
DecodeState = _struct("DecodeState", [("token", i32), ("position", i32), ("steps", i32), ("reserved", i32)])
AttendParams = _struct("AttendParams", [("kv_start", u32), ("kv_len", u32), ("capacity", u32), ("heads", u32),
                                        ("kv_heads", u32), ("head_dim", u32), ("kv_type", u32), ("chunks", u32),
                                        ("scale", f32), ("softcap", f32)])
RopeKvParams = _struct("RopeKvParams", [("heads", u32), ("kv_heads", u32), ("head_dim", u32), ("capacity", u32),
                                        ("position", u32), ("style", u32), ("kv_type", u32), ("rotate", u32)])
GemvFusedParams = _struct("GemvFusedParams", [("n", u32), ("k", u32), ("b_type", u32), ("scale_type", u32),
                                              ("epilogue", u32), ("norm", u32), ("eps", f32), ("quantize_out", u32)])
AttendStepParams = _struct("AttendStepParams", [("heads", u32), ("kv_heads", u32), ("head_dim", u32), ("capacity", u32),
                                                ("kv_start", u32), ("position", u32), ("kv_type", u32), ("chunks", u32),
                                                ("rope_style", u32), ("rotate", u32), ("scale", f32), ("softcap", f32),
                                                ("window", u32), ("prepared", u32), ("ready_chunks", u32)])
AttendPromptParams = _struct("AttendPromptParams", [("heads", u32), ("kv_heads", u32), ("head_dim", u32), ("capacity", u32),
                                                    ("t", u32), ("first", u32), ("kv_type", u32), ("scale", f32),
                                                    ("softcap", f32)])
GemvRopeParams = _struct("GemvRopeParams", [("n", u32), ("k", u32), ("b_type", u32), ("scale_type", u32), ("eps", f32),
                                            ("row0", u32), ("heads", u32), ("kv_heads", u32), ("head_dim", u32),
                                            ("capacity", u32), ("kv_type", u32), ("rotate", u32)])

P = C.POINTER
# name -> argtypes (all return int status unless noted)
SIGNATURES = {
    "vkml_abi_version": [],
    "vkml_init": [C.c_char_p],
    "vkml_shutdown": [],
    "vkml_is_initialized": [],
    "vkml_get_device_info": [P(DeviceInfo)],
    "vkml_malloc": [u64, P(vp)],
    "vkml_free": [vp],
    "vkml_host_malloc": [u64, P(vp)],
    "vkml_host_free": [vp],
    "vkml_memcpy_h2d": [vp, vp, u64],
    "vkml_memcpy_d2h": [vp, vp, u64],
    "vkml_memcpy_d2d": [vp, vp, u64],
    "vkml_fill_u32": [vp, u32, u64],
    "vkml_submit": [P(u64)],
    "vkml_wait": [u64],
    "vkml_completed": [P(u64)],
    "vkml_synchronize": [],
    "vkml_stream": [],
    "vkml_set_profiling": [C.c_int],
    "vkml_get_profiling": [],
    "vkml_set_profile_tag": [C.c_char_p],
    "vkml_profile": [P(KernelTime), u32, P(u32)],
    "vkml_reset_profile": [],
    "vkml_graph_begin": [],
    "vkml_graph_end": [P(u64)],
    "vkml_graph_launch": [u64],
    "vkml_graph_destroy": [u64],
    "vkml_quantize": [P(QuantizeParams), vp, vp, vp],
    "vkml_swiglu_quantize": [u32, vp, vp, vp, vp],
    "vkml_dequantize": [P(DequantizeParams), vp, vp, vp],
    "vkml_gemv_dot": [P(GemvDotParams), vp, vp, vp, vp, vp],
    "vkml_gemv_dot_add": [P(GemvDotParams), vp, vp, vp, vp, vp, vp],
    "vkml_matmul_dot": [P(GemvDotParams), vp, vp, vp, vp, vp],
    "vkml_matmul_dot_add": [P(GemvDotParams), vp, vp, vp, vp, vp, vp],
    "vkml_gemv_dot_swiglu": [P(GemvDotParams), vp, vp, vp, vp, vp, vp, vp],
    "vkml_gemv": [P(GemvParams), vp, vp, vp, vp],
    "vkml_matmul": [P(MatmulParams), vp, vp, vp, vp],
    "vkml_rms_norm": [P(RmsNormParams), vp, vp, vp],
    "vkml_rms_norm_quantize": [P(RmsNormParams), vp, vp, vp, vp, vp],
    "vkml_softmax": [P(SoftmaxParams), vp, vp],
    "vkml_argmax": [u32, u32, vp, vp],
    "vkml_rope": [P(RopeParams), vp, vp, vp],
    "vkml_cast": [u32, u32, u32, vp, vp],
    "vkml_copy_rows": [P(CopyRowsParams), vp, vp],
    "vkml_permute": [P(PermuteParams), vp, vp],
    "vkml_binary": [u32, u32, u32, vp, vp, vp],
    "vkml_unary": [u32, u32, f32, vp, vp],
    "vkml_embedding": [P(EmbeddingParams), vp, vp, vp, vp],
    "vkml_attend": [P(AttendParams), vp, vp, vp, vp, vp, vp],
    "vkml_attend_merge": [P(AttendParams), vp, vp, vp, vp, vp],
    "vkml_rope_kv_append": [P(RopeKvParams), vp, vp, vp, vp, vp, vp],
    "vkml_rope_kv_prompt": [P(RopeKvParams), u32, u32, vp, vp, vp, vp, vp],
    "vkml_gemv_fused": [P(GemvFusedParams), vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp],
    "vkml_gemv_rope": [P(GemvRopeParams), vp, vp, vp, vp, vp, vp, vp, vp, vp],
    "vkml_attend_step": [P(AttendStepParams), vp, vp, vp, vp, vp, vp, vp, vp, vp, vp],
    "vkml_attend_step_o": [P(AttendStepParams), vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, P(GemvDotParams), vp, vp, vp, vp],
    "vkml_attend_o_check": [vp],
    "vkml_attend_fused_sync_bytes": [u32],
    "vkml_attend_step_fused": [P(AttendStepParams), vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, P(GemvDotParams), vp, vp, vp, vp, u32, u32],
    "vkml_attend_fused_check": [vp, u32],
    "vkml_attend_fused_status": [vp, u32, P(u32)],
    "vkml_attend_o_status": [vp, P(u32)],
    "vkml_set_wait_limit": [u32],
    "vkml_attend_step_fused_supported": [P(AttendStepParams), P(GemvDotParams)],
    "vkml_attend_prompt_fast": [P(AttendPromptParams), vp, vp, vp, vp],
    "vkml_attend_prompt_fast_supported": [P(AttendPromptParams)],
    "vkml_attend_fast": [P(AttendParams), vp, vp, vp, vp, vp, vp, vp, vp, vp, vp],
    "vkml_attend_step_fast": [P(AttendStepParams), vp, vp, vp, vp, vp, vp, vp, vp, vp, P(GemvDotParams), vp, vp, vp, vp, u32, u32],
    "vkml_attend_step_fast_supported": [P(AttendStepParams), P(GemvDotParams)],
    "vkml_attend_step_noalloc": [P(AttendStepParams), vp, vp, vp, vp, vp, vp, vp, vp],
    "vkml_attend_o_sync_bytes": [],
    "vkml_state_set": [vp, i32, i32, i32],
    "vkml_embedding_state": [P(EmbeddingParams), vp, vp, vp, vp],
    "vkml_step_finish": [u32, vp, vp, vp, u32],
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
        _lib.vkml_last_error.restype = C.c_char_p
        _lib.vkml_last_error.argtypes = []
        for name, args in SIGNATURES.items():
            fn = getattr(_lib, name)
            fn.argtypes = args
            fn.restype = C.c_int
        _lib.vkml_stream.restype = C.c_void_p
        _lib.vkml_attend_o_sync_bytes.restype = C.c_uint64
        _lib.vkml_attend_fused_sync_bytes.restype = C.c_uint64
    return _lib


def check(status: int) -> None:
    if status != 0:
        raise VkmlError(f"vkml error {status}: {lib().vkml_last_error().decode()}")


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args))


def init(device: str = "") -> None:
    if not lib().vkml_is_initialized():
        call("vkml_init", device.encode())


def shutdown() -> None:
    call("vkml_shutdown")


def device_info() -> DeviceInfo:
    info = DeviceInfo()
    call("vkml_get_device_info", C.byref(info))
    return info


def synchronize() -> None:
    call("vkml_synchronize")


def stream() -> int:
    """The library's hipStream_t (an integer handle), or 0 before vkml_init."""
    return lib().vkml_stream() or 0


class Buffer:
    """Device memory from vkml_malloc, freed on close or collection."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        self.ptr = vp()
        call("vkml_malloc", max(self.nbytes, 4), C.byref(self.ptr))

    @property
    def p(self):
        return self.ptr

    def upload(self, arr: np.ndarray) -> "Buffer":
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes, (arr.nbytes, self.nbytes)
        call("vkml_memcpy_h2d", self.ptr, arr.ctypes.data_as(vp), arr.nbytes)
        return self

    def download(self, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype)
        assert out.nbytes <= self.nbytes
        call("vkml_memcpy_d2h", out.ctypes.data_as(vp), self.ptr, out.nbytes)
        return out

    def close(self) -> None:
        if self.ptr:
            try:
                lib().vkml_free(self.ptr)
            finally:
                self.ptr = vp()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def to_device(arr: np.ndarray) -> Buffer:
    arr = np.ascontiguousarray(arr)
    return Buffer(arr.nbytes).upload(arr)


def empty(nbytes: int) -> Buffer:
    return Buffer(nbytes)


def profile() -> list[tuple[str, int, float]]:
    count = u32()
    call("vkml_profile", None, 0, C.byref(count))
    rows = (KernelTime * max(count.value, 1))()
    call("vkml_profile", rows, count.value, C.byref(count))
    return [(r.name.decode(), int(r.calls), float(r.milliseconds)) for r in rows[:count.value]]
