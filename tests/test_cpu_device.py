"""The runtime's `cpu` device against the oracle, bit for bit.

The cpu device keeps the reference CPU path's per-element arithmetic
(src/cpu/cpu_backend.cpp): full sums in 65536-element chunks of four double
lanes, axis sums in double walked in axis order, the first strict maximum,
broadcasting binary ops with one fp32 operation per element, and max's
gradient scattered to the first maximum. Each case here compares the
device's result with the oracle's restatement of that arithmetic, which the
oracle tests pin against the reference built from its sources. CPU only.
"""

import numpy as np
import pytest

import vectorcore_amd as vc
from oracle import kernels as K


def cpu(x, grad=False):
    return vc.Tensor(np.ascontiguousarray(x, dtype=np.float32), requires_grad=grad, device="cpu")


@pytest.mark.parametrize("n", [0, 1, 3, 4, 65535, 65536, 65537, 3 * 65536 + 5, 1_000_003])
def test_full_sum_bitexact(n):
    x = np.random.default_rng(n).standard_normal(n).astype(np.float32) * 10
    assert np.float32(cpu(x).sum().item()).view(np.uint32) == K.sum_all(x).view(np.uint32)


AXIS_SHAPES = [((3, 4, 5), 1), ((1, 8192, 4096), 1), ((5000, 300), 0), ((7, 1000, 513), 1), ((2, 3, 1100), 2),
               ((64, 1), 0), ((1, 1), 0), ((9, 1030), 0), ((4096, 1000), 1)]


@pytest.mark.parametrize("shape,axis", AXIS_SHAPES)
def test_axis_reductions_bitexact(shape, axis):
    rng = np.random.default_rng(sum(shape) + axis)
    x = rng.standard_normal(shape).astype(np.float32)
    flat = x.reshape(-1)
    flat[::11] = flat[0]  # ties
    flat[5::97] = np.nan  # NaN never wins after the first element
    flat[3::131] = -np.inf
    t = cpu(x)
    for op, method in ((K.SUM, t.sum), (K.MAX, t.max), (K.ARGMAX, t.argmax)):
        got = method(axis).numpy()
        want = K.reduce_axis(x, axis, op)
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32), err_msg=f"op {op}")


def test_nan_first_element_wins_the_maximum():
    x = np.array([[np.nan, 1.0, 2.0], [3.0, np.nan, 3.0]], np.float32)
    np.testing.assert_array_equal(cpu(x).argmax(1).numpy(), K.reduce_axis(x, 1, K.ARGMAX))
    assert np.isnan(cpu(x).max(1).numpy()[0])


BROADCAST = [((1000, 300), (300,)), ((1000, 1), (1, 300)), ((40, 1, 300), (1, 50, 300)), ((40, 50, 1), (50, 7)),
             ((3,), (2, 1)), ((2, 1, 3, 1, 5), (4, 1, 6, 1)), ((1, 7, 1, 9), (8, 1, 6, 1)), ((5,), (1,)), ((), (3, 2))]


@pytest.mark.parametrize("a_shape,b_shape", BROADCAST)
def test_broadcasting_binary_ops_bitexact(a_shape, b_shape):
    rng = np.random.default_rng(len(a_shape) * 31 + len(b_shape))
    a = rng.standard_normal(a_shape).astype(np.float32)
    b = rng.standard_normal(b_shape).astype(np.float32) + 2.5
    ta, tb = cpu(a), cpu(b)
    for op, fn in ((K.ADD, lambda x, y: x + y), (K.SUB, lambda x, y: x - y), (K.MUL, lambda x, y: x * y),
                   (K.DIV, lambda x, y: x / y)):
        np.testing.assert_array_equal(fn(ta, tb).numpy(), K.binary(a, b, op), err_msg=f"op {op}")


def test_broadcast_through_a_transposed_view_bitexact():
    rng = np.random.default_rng(4)
    a = rng.standard_normal((6, 33, 17)).astype(np.float32)
    b = rng.standard_normal((17, 1)).astype(np.float32)
    ta = cpu(a).transpose()  # [6, 17, 33]
    np.testing.assert_array_equal((ta * cpu(b)).numpy(), K.binary(np.swapaxes(a, 1, 2), b, K.MUL))


@pytest.mark.parametrize("shape,axis", [((5, 7), 1), ((6, 1100), 0), ((3, 4, 5), 1), ((1, 600, 3), 1)])
def test_max_gradient_scatter_bitexact(shape, axis):
    rng = np.random.default_rng(sum(shape))
    x = rng.standard_normal(shape).astype(np.float32)
    x.reshape(-1)[::5] = 1.5  # ties go to the first maximum
    t = cpu(x, grad=True)
    upstream = rng.standard_normal(K.reduce_axis(x, axis, K.MAX).shape).astype(np.float32)
    (t.max(axis) * cpu(upstream)).sum().backward()
    idx = K.reduce_axis(x, axis, K.ARGMAX)
    np.testing.assert_array_equal(t.grad.numpy(), K.scatter_axis(upstream, idx, shape, axis))


@pytest.mark.parametrize("m,k,n", [(3, 5, 7), (64, 300, 65), (8, 513, 4100), (130, 257, 3)])
def test_gemm_bitexact(m, k, n):
    rng = np.random.default_rng(m + k + n)
    for ta in (False, True):
        for tb in (False, True):
            a = rng.uniform(-1, 1, size=(k, m) if ta else (m, k)).astype(np.float32)
            b = rng.uniform(-1, 1, size=(n, k) if tb else (k, n)).astype(np.float32)
            left = cpu(a).transpose() if ta else cpu(a)
            right = cpu(b).transpose() if tb else cpu(b)
            np.testing.assert_array_equal((left @ right).numpy(), K.matmul2d(a, b, ta, tb),
                                          err_msg=f"trans_a={ta} trans_b={tb}")


def test_errors_inside_parallel_work_surface_once():
    # A shape error raised inside a parallel region reaches the caller as one
    # exception and leaves the pool usable.
    for _ in range(3):
        with pytest.raises(ValueError):
            cpu(np.ones((2, 3))) @ cpu(np.ones((4, 2)))
    x = np.random.default_rng(0).standard_normal(3_000_000).astype(np.float32)
    assert np.float32(cpu(x).sum().item()) == K.sum_all(x)
