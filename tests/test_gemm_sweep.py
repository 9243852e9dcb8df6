"""Seeded random sweep of the four GEMM entry points against the oracle.

Shapes mix tile edges (1..513 around the 128-wide tiles), odd sizes, long K
over few tiles (split K), misaligned operands (the element-load variants),
batches with affine, broadcast and permuted per-batch offsets, batch
reductions, the folded ReLU mask (zeros and NaN in the mask) and the bias +
ReLU epilogue. Bar: the reference's GEMM tolerance, rtol 1e-4 and atol
1e-4 sqrt(k) (tests/python/test_performance_paths.py:43).
"""

import numpy as np
import pytest

from oracle import kernels as K
from vectorcore_amd import cabi as C

pytestmark = pytest.mark.gpu

EDGE = [1, 2, 3, 4, 5, 7, 31, 32, 33, 63, 64, 65, 127, 128, 129, 255, 256, 257, 383, 511, 513]
CASES = 160


@pytest.fixture(scope="module", autouse=True)
def device():
    assert C.available(), C.lib().vc_hip_last_error().decode()
    yield
    C.synchronize()


def _dim(rng, high):
    r = rng.random()
    if r < 0.45:
        return int(rng.choice(EDGE))
    return int(rng.integers(1, high))


def _view(buf, off, rows, cols, trans):
    """op() operand stored [rows, cols] ([cols, rows] when trans) at element off."""
    if trans:
        return buf[off:off + rows * cols].reshape(cols, rows).T
    return buf[off:off + rows * cols].reshape(rows, cols)


def _oracle(a_h, a_off, b_h, b_off, m, k, n, ta, tb):
    a = np.ascontiguousarray(_view(a_h, a_off, m, k, False) if not ta else a_h[a_off:a_off + m * k].reshape(k, m))
    b = np.ascontiguousarray(_view(b_h, b_off, k, n, False) if not tb else b_h[b_off:b_off + k * n].reshape(n, k))
    return K.matmul2d(a, b, bool(ta), bool(tb))


def _case(rng, index):
    kind = ["matmul", "matmul", "mask", "bias", "reduce"][index % 5]
    m, n, k = _dim(rng, 600), _dim(rng, 600), _dim(rng, 1500)
    if rng.random() < 0.15:  # a long K over a few output tiles: K is split
        m, n, k = int(rng.integers(1, 200)), int(rng.integers(1, 200)), int(rng.integers(2000, 6000))
    ta, tb = int(rng.integers(0, 2)), int(rng.integers(0, 2))
    shift = int(rng.choice([0, 0, 0, 1, 2]))  # elements of misalignment of both operands
    label = f"case {index}: {kind} m={m} k={k} n={n} trans=({ta},{tb}) shift={shift}"
    if kind in ("matmul", "mask"):
        batch = int(rng.integers(1, 4))
        mode = ["affine", "broadcast_b", "table"][int(rng.integers(0, 3))]
        if mode == "affine":
            ao, bo = [z * m * k for z in range(batch)], [z * k * n for z in range(batch)]
        elif mode == "broadcast_b":
            ao, bo = [z * m * k for z in range(batch)], [0] * batch
        else:
            ao = [int(v) * m * k for v in rng.permutation(batch)]
            bo = [int(v) * k * n for v in rng.permutation(batch)]
        label += f" batch={batch} {mode}"
        a_h = rng.uniform(-1, 1, shift + max(ao) + m * k).astype(np.float32)
        b_h = rng.uniform(-1, 1, shift + max(bo) + k * n).astype(np.float32)
        a, b, c = C.Buffer.of(a_h), C.Buffer.of(b_h), C.Buffer((batch, m, n))
        want = np.stack([_oracle(a_h, shift + ao[z], b_h, shift + bo[z], m, k, n, ta, tb) for z in range(batch)])
        if kind == "matmul":
            C.check(C.lib().vc_hip_matmul(a.ptr + 4 * shift, b.ptr + 4 * shift, c.ptr, m, k, n, C.sizes(ao),
                                          C.sizes(bo), batch, ta, tb))
        else:
            mask_h = rng.uniform(-1, 1, batch * m * n).astype(np.float32)
            mask_h[rng.random(mask_h.size) < 0.05] = 0.0
            mask_h[rng.random(mask_h.size) < 0.01] = np.nan
            mask = C.Buffer.of(mask_h)
            C.check(C.lib().vc_hip_matmul_relu_mask(a.ptr + 4 * shift, b.ptr + 4 * shift, c.ptr, m, k, n, C.sizes(ao),
                                                    C.sizes(bo), batch, ta, tb, mask.ptr))
            want = want * (mask_h.reshape(want.shape) > 0).astype(np.float32)
    elif kind == "bias":
        relu = int(rng.integers(0, 2))
        label = f"case {index}: bias m={m} k={k} n={n} relu={relu} shift={shift}"
        a_h = rng.uniform(-1, 1, shift + m * k).astype(np.float32)
        b_h = rng.uniform(-1, 1, shift + k * n).astype(np.float32)
        bias_h = rng.uniform(-1, 1, n).astype(np.float32)
        a, b, c, bias = C.Buffer.of(a_h), C.Buffer.of(b_h), C.Buffer((m, n)), C.Buffer.of(bias_h)
        C.check(C.lib().vc_hip_matmul_bias_relu(a.ptr + 4 * shift, b.ptr + 4 * shift, c.ptr, m, k, n, bias.ptr, relu))
        want = _oracle(a_h, shift, b_h, shift, m, k, n, 0, 0) + bias_h
        if relu:
            want = np.maximum(want, np.float32(0))
    else:
        count = int(rng.integers(1, 5))
        label += f" products={count}"
        a_h = rng.uniform(-1, 1, shift + count * m * k).astype(np.float32)
        b_h = rng.uniform(-1, 1, shift + count * k * n).astype(np.float32)
        a, b, c = C.Buffer.of(a_h), C.Buffer.of(b_h), C.Buffer((m, n))
        C.check(C.lib().vc_hip_matmul_reduce(a.ptr + 4 * shift, b.ptr + 4 * shift, c.ptr, m, k, n, count, m * k, k * n,
                                             ta, tb))
        want = sum(_oracle(a_h, shift + r * m * k, b_h, shift + r * k * n, m, k, n, ta, tb) for r in range(count))
        k *= count
    return label, c.numpy().reshape(want.shape), want, k


def test_gemm_entry_points_random_sweep():
    rng = np.random.default_rng(20261201)
    for index in range(CASES):
        label, got, want, k = _case(rng, index)
        np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-4 * np.sqrt(k), err_msg=label)
