"""ORACLE — test infrastructure only.

ctypes wrappers over the two CPU oracles:
  * ``liboracle.so`` — the C restatement of the reference CPU kernels
    (vc_oracle.c), exposed as the functions in this module;
  * ``_ref/libvc_ref.so`` — the reference library built from its own sources
    (build_oracle.py), exposed through :class:`Reference` when it was built.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, and only to check or time the CPU path.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ADD, SUB, MUL, DIV = 0, 1, 2, 3
NEG, RELU, SIGMOID, RELU_GRAD, EXP, LOG = 0, 1, 2, 3, 4, 5
SUM, MAX, ARGMAX = 0, 1, 2

_f32p = ctypes.POINTER(ctypes.c_float)
_szp = ctypes.POINTER(ctypes.c_size_t)
_sz = ctypes.c_size_t
_lib = None


def _load():
    global _lib
    if _lib is None:
        path = HERE / "liboracle.so"
        if not path.exists():
            from oracle.build_oracle import build_oracle
            build_oracle()
        lib = ctypes.CDLL(str(path))
        lib.vco_binary.argtypes = [_f32p, _szp, _sz, _f32p, _szp, _sz, _f32p, _szp, _sz, ctypes.c_int]
        lib.vco_unary.argtypes = [_f32p, _f32p, _sz, ctypes.c_int]
        lib.vco_matmul.argtypes = [_f32p, _f32p, _f32p, _sz, _sz, _sz, ctypes.c_int, ctypes.c_int]
        lib.vco_transpose.argtypes = [_f32p, _f32p, _sz, _sz, _sz]
        lib.vco_sum.argtypes = [_f32p, _sz]
        lib.vco_sum.restype = ctypes.c_float
        lib.vco_reduce_axis.argtypes = [_f32p, _f32p, _sz, _sz, _sz, ctypes.c_int]
        lib.vco_reduce_axis.restype = ctypes.c_int
        lib.vco_scatter_axis.argtypes = [_f32p, _f32p, _f32p, _sz, _sz, _sz]
        lib.vco_sgd.argtypes = [_f32p, _f32p, _sz, ctypes.c_float]
        _lib = lib
    return _lib


def f32(x) -> np.ndarray:
    """float32, C-contiguous, keeping 0-d scalars 0-d."""
    a = np.asarray(x, dtype=np.float32)
    return a if a.flags.c_contiguous else np.ascontiguousarray(a)


def _p(a: np.ndarray):
    return a.ctypes.data_as(_f32p)


def _shape(shape):
    arr = (ctypes.c_size_t * max(1, len(shape)))(*shape)
    return arr, len(shape)


def broadcast_shape(a, b):
    """include/vectorcore/shape.hpp broadcast_shape (src/shape.cpp:34-47)."""
    rank = max(len(a), len(b))
    out = []
    for i in range(rank):
        ai = 1 if i < rank - len(a) else a[i - (rank - len(a))]
        bi = 1 if i < rank - len(b) else b[i - (rank - len(b))]
        if ai != bi and ai != 1 and bi != 1:
            raise ValueError(f"cannot broadcast shapes {list(a)} and {list(b)}")
        out.append(max(ai, bi))
    return tuple(out)


def binary(a, b, op: int, out_shape=None) -> np.ndarray:
    """out = a (op) b over out_shape (default: the broadcast shape)."""
    a, b = f32(a), f32(b)
    out_shape = broadcast_shape(a.shape, b.shape) if out_shape is None else tuple(out_shape)
    out = np.empty(out_shape, dtype=np.float32)
    sa, ra = _shape(a.shape)
    sb, rb = _shape(b.shape)
    so, ro = _shape(out_shape)
    _load().vco_binary(_p(a), sa, ra, _p(b), sb, rb, _p(out), so, ro, op)
    return out


def unary(x, op: int) -> np.ndarray:
    x = f32(x)
    out = np.empty_like(x)
    _load().vco_unary(_p(x), _p(out), x.size, op)
    return out


def matmul2d(a, b, trans_a=False, trans_b=False) -> np.ndarray:
    """out = op(a) @ op(b) for single matrices stored as the flags say."""
    a, b = f32(a), f32(b)
    m = a.shape[1] if trans_a else a.shape[0]
    k = a.shape[0] if trans_a else a.shape[1]
    n = b.shape[0] if trans_b else b.shape[1]
    out = np.empty((m, n), dtype=np.float32)
    _load().vco_matmul(_p(a), _p(b), _p(out), m, k, n, int(trans_a), int(trans_b))
    return out


def matmul(a, b, trans_a=False, trans_b=False) -> np.ndarray:
    """Batched op(A) @ op(B) with broadcast batch dims, looping the batch in
    order over per-batch element offsets (src/ops.cpp:171-240)."""
    a, b = f32(a), f32(b)
    if a.ndim < 2 or b.ndim < 2:
        raise ValueError("matmul requires tensors of rank 2 or more")
    ar, ac = a.shape[-2:]
    br, bc = b.shape[-2:]
    m, k = (ac, ar) if trans_a else (ar, ac)
    n = br if trans_b else bc
    if (bc if trans_b else br) != k:
        raise ValueError(f"matmul shape mismatch: {list(a.shape)} and {list(b.shape)}")
    out_batch = broadcast_shape(a.shape[:-2], b.shape[:-2])
    a_b = np.broadcast_to(a, out_batch + a.shape[-2:]).reshape((-1,) + a.shape[-2:])
    b_b = np.broadcast_to(b, out_batch + b.shape[-2:]).reshape((-1,) + b.shape[-2:])
    batch = int(np.prod(out_batch)) if out_batch else 1
    out = np.empty((batch, m, n), dtype=np.float32)
    for z in range(batch):
        out[z] = matmul2d(a_b[z], b_b[z], trans_a, trans_b)
    return out.reshape(out_batch + (m, n))


def transpose_last2(x) -> np.ndarray:
    x = f32(x)
    rows, cols = x.shape[-2:]
    batch = x.size // max(1, rows * cols) if rows * cols else 0
    out = np.empty(x.shape[:-2] + (cols, rows), dtype=np.float32)
    if x.size:
        _load().vco_transpose(_p(x), _p(out), batch, rows, cols)
    return out


def sum_all(x) -> np.float32:
    x = f32(x)
    return np.float32(_load().vco_sum(_p(x), x.size))


def split_axis(shape, axis):
    """src/ops.cpp:63-80."""
    rank = len(shape)
    if rank == 0:
        raise ValueError("cannot reduce a scalar along an axis")
    if axis < -rank or axis >= rank:
        raise IndexError(f"axis {axis} is out of range for shape {list(shape)}")
    axis = axis + rank if axis < 0 else axis
    outer = int(np.prod(shape[:axis])) if axis else 1
    inner = int(np.prod(shape[axis + 1:])) if axis + 1 < rank else 1
    kept = tuple(shape[:axis]) + (1,) + tuple(shape[axis + 1:])
    removed = tuple(shape[:axis]) + tuple(shape[axis + 1:])
    return axis, outer, shape[axis], inner, kept, removed


def reduce_axis(x, axis: int, op: int, keepdim=False) -> np.ndarray:
    x = f32(x)
    _, outer, length, inner, kept, removed = split_axis(x.shape, axis)
    out = np.empty(kept if keepdim else removed, dtype=np.float32)
    if _load().vco_reduce_axis(_p(x), _p(out), outer, length, inner, op) != 0:
        raise ValueError("max/argmax over an empty axis is undefined")
    return out


def scatter_axis(values, indices, shape, axis) -> np.ndarray:
    values, indices = f32(values), f32(indices)
    _, outer, length, inner, _, _ = split_axis(tuple(shape), axis)
    out = np.empty(shape, dtype=np.float32)
    _load().vco_scatter_axis(_p(values), _p(indices), _p(out), outer, length, inner)
    return out


def sgd_(param: np.ndarray, grad, lr: float) -> None:
    grad = f32(grad)
    assert param.dtype == np.float32 and param.flags.c_contiguous
    _load().vco_sgd(_p(param), _p(grad), param.size, lr)


# --- the reference library itself -----------------------------------------


class Reference:
    """The reference VectorCore built from its own sources, when present."""

    path = HERE / "_ref" / "libvc_ref.so"

    def __init__(self):
        lib = ctypes.CDLL(str(self.path))
        i64p = ctypes.POINTER(ctypes.c_int64)
        lib.ref_last_error.restype = ctypes.c_char_p
        lib.ref_hardware_threads.restype = ctypes.c_uint
        lib.ref_binary.argtypes = [_f32p, _szp, _sz, _f32p, _szp, _sz, _f32p, _szp, _sz, ctypes.c_int]
        lib.ref_unary.argtypes = [_f32p, _f32p, _sz, ctypes.c_int]
        lib.ref_matmul.argtypes = [_f32p, _f32p, _f32p, _sz, _sz, _sz, ctypes.c_int, ctypes.c_int]
        lib.ref_sum.argtypes = [_f32p, _sz, _f32p]
        lib.ref_reduce_axis.argtypes = [_f32p, _f32p, _sz, _sz, _sz, ctypes.c_int]
        lib.ref_matmul_backward.argtypes = [_f32p, _szp, _sz, _f32p, _szp, _sz, _f32p, _f32p, _f32p]
        lib.ref_activation_backward.argtypes = [_f32p, _f32p, _f32p, _sz, _sz, _f32p, _f32p, _f32p]
        lib.ref_cross_entropy.argtypes = [_f32p, i64p, _sz, _sz, _f32p, _f32p, _f32p]
        lib.ref_mlp_create.argtypes = [_sz, _szp, ctypes.POINTER(_f32p), ctypes.POINTER(_f32p), _f32p, _sz, i64p]
        lib.ref_mlp_create.restype = ctypes.c_void_p
        lib.ref_mlp_step.argtypes = [ctypes.c_void_p, ctypes.c_float, _f32p]
        lib.ref_mlp_grads.argtypes = [ctypes.c_void_p, _f32p, ctypes.POINTER(_f32p), ctypes.POINTER(_f32p)]
        lib.ref_mlp_params.argtypes = [ctypes.c_void_p, ctypes.POINTER(_f32p), ctypes.POINTER(_f32p)]
        lib.ref_mlp_destroy.argtypes = [ctypes.c_void_p]
        self.lib = lib
        self._i64p = i64p

    @classmethod
    def available(cls) -> bool:
        return cls.path.exists()

    def _check(self, rc):
        if rc != 0:
            raise RuntimeError(self.lib.ref_last_error().decode())

    def threads(self) -> int:
        return int(self.lib.ref_hardware_threads())

    def binary(self, a, b, op):
        a, b = f32(a), f32(b)
        shape = broadcast_shape(a.shape, b.shape)
        out = np.empty(shape, dtype=np.float32)
        sa, ra = _shape(a.shape)
        sb, rb = _shape(b.shape)
        so, ro = _shape(shape)
        self._check(self.lib.ref_binary(_p(a), sa, ra, _p(b), sb, rb, _p(out), so, ro, op))
        return out

    def unary(self, x, op):
        x = f32(x)
        out = np.empty_like(x)
        self._check(self.lib.ref_unary(_p(x), _p(out), x.size, op))
        return out

    def matmul2d(self, a, b, trans_a=False, trans_b=False):
        a, b = f32(a), f32(b)
        m = a.shape[1] if trans_a else a.shape[0]
        k = a.shape[0] if trans_a else a.shape[1]
        n = b.shape[0] if trans_b else b.shape[1]
        out = np.empty((m, n), dtype=np.float32)
        self._check(self.lib.ref_matmul(_p(a), _p(b), _p(out), m, k, n, int(trans_a), int(trans_b)))
        return out

    def sum_all(self, x):
        x = f32(x)
        out = np.zeros(1, dtype=np.float32)
        self._check(self.lib.ref_sum(_p(x), x.size, _p(out)))
        return out[0]

    def reduce_axis(self, x, axis, op, keepdim=False):
        x = f32(x)
        _, outer, length, inner, kept, removed = split_axis(x.shape, axis)
        out = np.empty(kept if keepdim else removed, dtype=np.float32)
        self._check(self.lib.ref_reduce_axis(_p(x), _p(out), outer, length, inner, op))
        return out

    def matmul_backward(self, a, b, dc):
        a, b, dc = f32(a), f32(b), f32(dc)
        da, db = np.empty_like(a), np.empty_like(b)
        sa, ra = _shape(a.shape)
        sb, rb = _shape(b.shape)
        self._check(self.lib.ref_matmul_backward(_p(a), sa, ra, _p(b), sb, rb, _p(dc), _p(da), _p(db)))
        return da, db

    def activation_backward(self, x, bias, dy):
        x, bias, dy = f32(x), f32(bias), f32(dy)
        rows, cols = x.shape
        y, dx, dbias = np.empty_like(x), np.empty_like(x), np.empty((1, cols), dtype=np.float32)
        self._check(self.lib.ref_activation_backward(_p(x), _p(bias), _p(dy), rows, cols, _p(y), _p(dx),
                                                     _p(dbias)))
        return y, dx, dbias

    def cross_entropy(self, logits, targets, with_argmax=True):
        logits = f32(logits)
        t = np.ascontiguousarray(np.asarray(targets, dtype=np.int64))
        rows, cols = logits.shape
        loss = np.zeros(1, dtype=np.float32)
        grad = np.empty_like(logits)
        am = np.empty(rows, dtype=np.float32) if with_argmax else None
        self._check(self.lib.ref_cross_entropy(_p(logits), t.ctypes.data_as(self._i64p), rows, cols, _p(loss),
                                               _p(grad), _p(am) if am is not None else None))
        return loss[0], grad, am

    def mlp(self, weights, biases, x, targets):
        return ReferenceMlp(self, weights, biases, x, targets)


class ReferenceMlp:
    """x @ W + b layers with ReLU between them, CE loss, SGD (reference API)."""

    def __init__(self, ref: Reference, weights, biases, x, targets):
        self.ref = ref
        self.dims = [weights[0].shape[0]] + [w.shape[1] for w in weights]
        ws = [f32(w) for w in weights]
        bs = [f32(b) for b in biases]
        x = f32(x)
        t = np.ascontiguousarray(np.asarray(targets, dtype=np.int64))
        dims = (ctypes.c_size_t * len(self.dims))(*self.dims)
        wp = (_f32p * len(ws))(*[_p(w) for w in ws])
        bp = (_f32p * len(bs))(*[_p(b) for b in bs])
        self.handle = ref.lib.ref_mlp_create(len(ws), dims, wp, bp, _p(x), x.shape[0], t.ctypes.data_as(ref._i64p))
        if not self.handle:
            raise RuntimeError(ref.lib.ref_last_error().decode())

    def step(self, lr: float) -> float:
        loss = np.zeros(1, dtype=np.float32)
        self.ref._check(self.ref.lib.ref_mlp_step(self.handle, lr, _p(loss)))
        return float(loss[0])

    def grads(self):
        n = len(self.dims) - 1
        dws = [np.empty((self.dims[i], self.dims[i + 1]), dtype=np.float32) for i in range(n)]
        dbs = [np.empty(self.dims[i + 1], dtype=np.float32) for i in range(n)]
        loss = np.zeros(1, dtype=np.float32)
        wp = (_f32p * n)(*[_p(w) for w in dws])
        bp = (_f32p * n)(*[_p(b) for b in dbs])
        self.ref._check(self.ref.lib.ref_mlp_grads(self.handle, _p(loss), wp, bp))
        return float(loss[0]), dws, dbs

    def params(self):
        n = len(self.dims) - 1
        ws = [np.empty((self.dims[i], self.dims[i + 1]), dtype=np.float32) for i in range(n)]
        bs = [np.empty(self.dims[i + 1], dtype=np.float32) for i in range(n)]
        wp = (_f32p * n)(*[_p(w) for w in ws])
        bp = (_f32p * n)(*[_p(b) for b in bs])
        self.ref._check(self.ref.lib.ref_mlp_params(self.handle, wp, bp))
        return ws, bs

    def __del__(self):
        if getattr(self, "handle", None):
            self.ref.lib.ref_mlp_destroy(self.handle)
            self.handle = None
