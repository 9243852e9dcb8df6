"""ctypes binding of the C ABI in include/vc_hip.h (libvc_hip.so).

This is the same binding a Python-side FFI of the reference would add; tests
use it to drive every entry point directly. Loading fails loudly when the
library has not been built.
"""

from __future__ import annotations

import contextlib
import ctypes
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "libvc_hip.so"

OK = 0
ERRORS = {1: ValueError, 2: IndexError, 3: OverflowError, 4: RuntimeError, 5: RuntimeError, 6: MemoryError}
ADD, SUB, MUL, DIV = 0, 1, 2, 3
NEG, RELU, SIGMOID, RELU_GRAD, EXP, LOG = 0, 1, 2, 3, 4, 5
SUM, MAX, ARGMAX = 0, 1, 2

_vp = ctypes.c_void_p
_sz = ctypes.c_size_t
_szp = ctypes.POINTER(ctypes.c_size_t)
_i = ctypes.c_int
_f = ctypes.c_float

# Fused elementwise programs (vc_hip_map).
MAP_ADD, MAP_SUB, MAP_MUL, MAP_DIV, MAP_NEG, MAP_STEP = range(6)
MAP_SLOTS, MAP_CODE, MAP_INPUTS, MAP_CONSTANTS, MAP_OUTPUTS, MAP_SUMS = 16, 32, 8, 8, 4, 2


class MapProgram(ctypes.Structure):
    _fields_ = [("inputs", _vp * MAP_INPUTS), ("n_inputs", _sz), ("constants", _f * MAP_CONSTANTS),
                ("n_constants", _sz), ("code", ctypes.c_uint32 * MAP_CODE), ("n_code", _sz),
                ("outputs", _vp * MAP_OUTPUTS), ("output_slots", ctypes.c_ubyte * MAP_OUTPUTS), ("n_outputs", _sz),
                ("sums", _vp * MAP_SUMS), ("sum_slots", ctypes.c_ubyte * MAP_SUMS), ("n_sums", _sz),
                ("rows", _sz), ("cols", _sz)]


def map_word(op: int, a: int, b: int, dst: int) -> int:
    """One instruction of a vc_hip_map program: slot[dst] = slot[a] op slot[b]."""
    return op | a << 8 | b << 16 | dst << 24


def map_program(inputs, constants, code, outputs, sums, rows, cols) -> MapProgram:
    """A vc_hip_map program. inputs: device pointers; constants: floats;
    code: (op, a, b, dst) tuples; outputs and sums: (device pointer, slot) pairs."""
    p = MapProgram()
    for j, ptr in enumerate(inputs):
        p.inputs[j] = ptr
    p.n_inputs = len(inputs)
    for j, v in enumerate(constants):
        p.constants[j] = v
    p.n_constants = len(constants)
    for k, ins in enumerate(code):
        p.code[k] = map_word(*ins)
    p.n_code = len(code)
    for j, (ptr, slot) in enumerate(outputs):
        p.outputs[j] = ptr
        p.output_slots[j] = slot
    p.n_outputs = len(outputs)
    for j, (ptr, slot) in enumerate(sums):
        p.sums[j] = ptr
        p.sum_slots[j] = slot
    p.n_sums = len(sums)
    p.rows, p.cols = rows, cols
    return p

_SIGNATURES = {
    "vc_hip_available": ([], _i),
    "vc_hip_device_name": ([], ctypes.c_char_p),
    "vc_hip_last_error": ([], ctypes.c_char_p),
    "vc_hip_gemm_kernel": ([], ctypes.c_char_p),
    "vc_hip_set_gemm_kernel": ([ctypes.c_char_p], _i),
    "vc_hip_alloc": ([_sz, ctypes.POINTER(_vp)], _i),
    "vc_hip_release": ([_vp], _i),
    "vc_hip_upload": ([_vp, _vp, _sz], _i),
    "vc_hip_download": ([_vp, _vp, _sz], _i),
    "vc_hip_mirror_scalar": ([_vp, ctypes.POINTER(_vp)], _i),
    "vc_hip_mirror_read": ([_vp, ctypes.POINTER(ctypes.c_float)], _i),
    "vc_hip_mirror_release": ([_vp], _i),
    "vc_hip_copy": ([_vp, _vp, _sz], _i),
    "vc_hip_synchronize": ([], _i),
    "vc_hip_stream_idle": ([ctypes.POINTER(_i)], _i),
    "vc_hip_pool_stats_get": ([_vp], _i),
    "vc_hip_pool_trim": ([], _i),
    "vc_hip_colsum_finish": ([_vp, _vp], _i),
    "vc_hip_colsum_size": ([_vp, _szp], _i),
    "vc_hip_colsum_release": ([_vp], _i),
    "vc_hip_fill": ([_vp, _sz, _f], _i),
    "vc_hip_binary": ([_vp, _szp, _szp, _sz, _vp, _szp, _szp, _sz, _vp, _szp, _sz, _i], _i),
    "vc_hip_binary_scalar": ([_vp, _sz, _f, _i, _vp, _i], _i),
    "vc_hip_unary": ([_vp, _vp, _sz, _i], _i),
    "vc_hip_axpy": ([_vp, _vp, _sz, _f], _i),
    "vc_hip_axpy_batch": ([ctypes.POINTER(_vp), ctypes.POINTER(_vp), ctypes.POINTER(_vp), _szp, _sz, _f], _i),
    "vc_hip_axpy_batch_colsum": ([ctypes.POINTER(_vp), ctypes.POINTER(_vp), ctypes.POINTER(_vp),
                                  ctypes.POINTER(_vp), _szp, _sz, _f], _i),
    "vc_hip_relu_backward": ([_vp, _vp, _vp, _sz], _i),
    "vc_hip_sigmoid_backward": ([_vp, _vp, _vp, _sz], _i),
    "vc_hip_exp_backward": ([_vp, _vp, _vp, _sz], _i),
    "vc_hip_log_backward": ([_vp, _vp, _vp, _sz], _i),
    "vc_hip_div_backward": ([_vp, _vp, _szp, _szp, _sz, _vp, _szp, _szp, _sz, _szp, _sz, _vp, _vp], _i),
    "vc_hip_map": ([ctypes.POINTER(MapProgram)], _i),
    "vc_hip_matmul": ([_vp, _vp, _vp, _sz, _sz, _sz, _szp, _szp, _sz, _i, _i], _i),
    "vc_hip_matmul_relu_mask": ([_vp, _vp, _vp, _sz, _sz, _sz, _szp, _szp, _sz, _i, _i, _vp], _i),
    "vc_hip_matmul_relu_mask_colsum": ([_vp, _vp, _vp, _sz, _sz, _sz, _i, _i, _vp, _vp], _i),
    "vc_hip_matmul_relu_mask_colsum_pending": ([_vp, _vp, _vp, _sz, _sz, _sz, _i, _i, _vp, _vp,
                                                ctypes.POINTER(_vp)], _i),
    "vc_hip_matmul_bias_relu": ([_vp, _vp, _vp, _sz, _sz, _sz, _vp, _i], _i),
    "vc_hip_matmul_bias_relu_bits": ([_vp, _vp, _vp, _sz, _sz, _sz, _vp, _vp, ctypes.POINTER(_i)], _i),
    "vc_hip_matmul_relu_bits": ([_vp, _vp, _vp, _sz, _sz, _sz, _i, _i, _vp], _i),
    "vc_hip_matmul_relu_bits_colsum_pending": ([_vp, _vp, _vp, _sz, _sz, _sz, _i, _i, _vp, _vp,
                                                ctypes.POINTER(_vp)], _i),
    "vc_hip_matmul_reduce": ([_vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz, _i, _i], _i),
    "vc_hip_transpose_last2": ([_vp, _vp, _sz, _sz, _sz], _i),
    "vc_hip_reduce_sum": ([_vp, _sz, _vp], _i),
    "vc_hip_reduce_axis": ([_vp, _vp, _sz, _sz, _sz, _i], _i),
    "vc_hip_reduce_axis_noalloc": ([_vp, _vp, _sz, _sz, _sz, _i], _i),
    "vc_hip_scatter_axis": ([_vp, _vp, _vp, _sz, _sz, _sz], _i),
    "vc_hip_xent_forward": ([_vp, _vp, _sz, _sz, _vp, _vp], _i),
    "vc_hip_xent_forward_published": ([_vp, _vp, _sz, _sz, _vp, _vp, ctypes.POINTER(_vp)], _i),
    "vc_hip_xent_forward_argmax": ([_vp, _vp, _sz, _sz, _vp, _vp, _vp, ctypes.POINTER(_vp)], _i),
    "vc_hip_xent_backward": ([_vp, _vp, _vp, _vp, _sz, _sz, _vp], _i),
    "vc_hip_xent_backward_value": ([_vp, _vp, _vp, _f, _sz, _sz, _vp], _i),
    "vc_hip_xent_backward_colsum": ([_vp, _vp, _vp, _vp, _f, _sz, _sz, _vp, _vp], _i),
    "vc_hip_xent_backward_colsum_pending": ([_vp, _vp, _vp, _vp, _f, _sz, _sz, _vp, _vp, ctypes.POINTER(_vp)], _i),
    "vc_hip_profile_enable": ([_i], _i),
    "vc_hip_profile_labels": ([ctypes.c_char_p], _i),
    "vc_hip_profile_reset": ([], _i),
    "vc_hip_profile_count": ([_szp], _i),
    "vc_hip_profile_entry": ([_sz, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_uint64),
                              ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double),
                              ctypes.POINTER(ctypes.c_double)], _i),
}

EXPORTED = tuple(_SIGNATURES)


class PoolStats(ctypes.Structure):
    _fields_ = [("device_allocations", ctypes.c_uint64), ("reuses", ctypes.c_uint64),
                ("live_bytes", ctypes.c_uint64), ("pooled_bytes", ctypes.c_uint64)]


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built; run python vectorcore_amd/build.py")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (args, res) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = res
        _lib = handle
    return _lib


def check(status: int) -> None:
    if status != OK:
        msg = lib().vc_hip_last_error().decode()
        raise ERRORS.get(status, RuntimeError)(msg)


def available() -> bool:
    return bool(lib().vc_hip_available())


def synchronize() -> None:
    check(lib().vc_hip_synchronize())


def stream_idle() -> bool:
    """Whether the library stream has completed everything enqueued (no wait)."""
    idle = ctypes.c_int(-1)
    check(lib().vc_hip_stream_idle(ctypes.byref(idle)))
    return bool(idle.value)


def pool_stats() -> PoolStats:
    s = PoolStats()
    check(lib().vc_hip_pool_stats_get(ctypes.byref(s)))
    return s


def sizes(values):
    values = [int(v) for v in values]
    return (ctypes.c_size_t * max(1, len(values)))(*values)


class Buffer:
    """A device buffer from the library's pool holding a float32 (or int32) array."""

    def __init__(self, shape, dtype=np.float32):
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        ptr = _vp()
        check(lib().vc_hip_alloc(max(self.nbytes, 4), ctypes.byref(ptr)))
        self.ptr = ptr.value

    @classmethod
    def of(cls, array, dtype=None):
        a = np.ascontiguousarray(array, dtype=dtype or (np.int32 if np.asarray(array).dtype.kind in "iu" else np.float32))
        buf = cls(a.shape, a.dtype)
        if buf.nbytes:
            check(lib().vc_hip_upload(buf.ptr, a.ctypes.data, buf.nbytes))
        return buf

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        check(lib().vc_hip_download(out.ctypes.data, self.ptr, self.nbytes))
        return out

    def release(self):
        if self.ptr:
            check(lib().vc_hip_release(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            if self.ptr and _lib is not None:
                _lib.vc_hip_release(self.ptr)
        except Exception:
            pass


def profile(enable: bool) -> None:
    check(lib().vc_hip_profile_enable(1 if enable else 0))


def profile_labels(labels=None) -> None:
    """Restrict the profiler to these labels (None: all)."""
    check(lib().vc_hip_profile_labels(",".join(labels).encode() if labels else None))


def profile_reset() -> None:
    check(lib().vc_hip_profile_reset())


def profile_read() -> dict:
    """{label: dict(launches, ms, flops, bytes)} summed since the last reset."""
    n = ctypes.c_size_t()
    check(lib().vc_hip_profile_count(ctypes.byref(n)))
    out = {}
    for i in range(n.value):
        label = ctypes.c_char_p()
        launches = ctypes.c_uint64()
        ms, flops, nbytes = ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
        check(lib().vc_hip_profile_entry(i, ctypes.byref(label), ctypes.byref(launches), ctypes.byref(ms),
                                         ctypes.byref(flops), ctypes.byref(nbytes)))
        if launches.value:
            out[label.value.decode()] = dict(launches=launches.value, ms=ms.value, flops=flops.value,
                                             bytes=nbytes.value)
    return out


@contextlib.contextmanager
def gemm_kernel(name: str):
    """Run the enclosed calls with GEMM kernel `name` ("mfma" or "simple"), then restore the previous one."""
    previous = lib().vc_hip_gemm_kernel().decode()
    check(lib().vc_hip_set_gemm_kernel(name.encode()))
    try:
        yield name
    finally:
        check(lib().vc_hip_set_gemm_kernel(previous.encode()))
