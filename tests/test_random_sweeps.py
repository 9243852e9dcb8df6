"""Seeded random sweeps of C-ABI entry points against the oracle.

GEMM (the four entry points): shapes mix tile edges (1..513 around the
128-wide tiles), odd sizes, long K over few tiles (split K), and two more
sweeps cover the ranges of products that run on 32 x 32 and on 128 x 128
tiles; misaligned operands (the element-load variants), batches with affine,
broadcast and permuted per-batch offsets, batch reductions, the folded ReLU
mask (zeros and NaN in the mask) and the bias + ReLU epilogue. Bar: the reference's GEMM
tolerance, rtol 1e-4 and atol 1e-4 sqrt(k)
(tests/python/test_performance_paths.py:43).

Axis reductions (sum, max, argmax) over random outer x length x inner, the
full sum, and the broadcasting binary ops (operands of rank 1-4 with size-1
axes, A read through a transposed view half the time), with NaN, +-inf, +-0
and ties mixed in. Bars: max, argmax and the binary ops bit-exact; sums
within 1e-6 relative (both sides accumulate in double).
"""

import numpy as np
import pytest

from oracle import kernels as K
from vectorcore_amd import cabi as C

pytestmark = pytest.mark.gpu

EDGE = [1, 2, 3, 4, 5, 7, 31, 32, 33, 63, 64, 65, 127, 128, 129, 255, 256, 257, 383, 511, 513]
CASES = 160
LARGE_CASES = 60  # about 1 G multiply-adds each for the oracle


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


def _shape(rng):
    m, n, k = _dim(rng, 600), _dim(rng, 600), _dim(rng, 1500)
    if rng.random() < 0.15:  # a long K over a few output tiles: K is split
        m, n, k = int(rng.integers(1, 200)), int(rng.integers(1, 200)), int(rng.integers(2000, 6000))
    return m, n, k


SMALL_EDGE = [1, 2, 3, 31, 32, 33, 63, 64, 65, 95, 96, 97, 127, 128, 129, 255, 256, 257]
K_EDGE = [1, 2, 15, 16, 17, 31, 32, 33, 255, 256, 257, 511, 512, 513, 2047, 2048]


def _small_shape(rng):
    """Shapes of at most 16 output tiles of 128 x 128 (times up to 3 batches
    or 4 reduced products) and K up to 2048, the range that runs on 32 x 32
    tiles with K split over a workgroup's waves: edges of the 32-row tiles,
    K around the 16-wide half-wave steps and the 256-wide rounds of 8 waves,
    and 9 to 25 tiles with K from 2049 to 4000 (no split pass)."""
    if rng.random() < 0.15:
        return int(rng.integers(257, 641)), int(rng.integers(257, 641)), int(rng.integers(2049, 4001))

    def dim(edges, high):
        return int(rng.choice(edges)) if rng.random() < 0.45 else int(rng.integers(1, high))

    m, n = dim(SMALL_EDGE, 513), dim(SMALL_EDGE, 513)
    return m, n, dim(K_EDGE, 2049)


LARGE_EDGE = [895, 896, 897, 1023, 1024, 1025, 1151, 1152, 1153, 1279, 1280, 1281, 1407, 1408]


def _large_shape(rng):
    """Shapes of about 64 to 121 output tiles of 128 x 128, the range that
    runs on those tiles: edges of the 128-row tiles (8 x 8 = 64 tiles is the
    last product on 32 x 32 tiles), K 1024 to 2048 over up to 128 tiles (K
    split in 2 to 4 ranges of at least 16 slices), and 25 to 64 tiles with K
    from 2049 to 4000 (split when over 32 tiles)."""
    r = rng.random()
    if r < 0.25:
        return int(rng.integers(1025, 1409)), int(rng.integers(897, 1409)), int(rng.integers(1024, 2049))
    if r < 0.4:
        return int(rng.integers(513, 1025)), int(rng.integers(513, 1025)), int(rng.integers(2049, 4001))

    def dim():
        return int(rng.choice(LARGE_EDGE)) if rng.random() < 0.45 else int(rng.integers(897, 1409))

    m, n = dim(), dim()
    return m, n, _dim(rng, 1200)


def _case(rng, index, shape=_shape):
    kind = ["matmul", "matmul", "mask", "bias", "reduce"][index % 5]
    m, n, k = shape(rng)
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


def test_gemm_entry_points_random_sweep_over_the_32_tile_range():
    rng = np.random.default_rng(20261203)
    for index in range(CASES):
        label, got, want, k = _case(rng, index, _small_shape)
        np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-4 * np.sqrt(k), err_msg=label)


def test_gemm_entry_points_random_sweep_over_the_128_tile_range():
    rng = np.random.default_rng(20261204)
    for index in range(LARGE_CASES):
        label, got, want, k = _case(rng, index, _large_shape)
        np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-4 * np.sqrt(k), err_msg=label)


def _data(rng, n, special):
    x = rng.standard_normal(n).astype(np.float32)
    if special:
        k = max(1, n // 50)
        for val in (np.nan, np.inf, -np.inf, 0.0, -0.0):
            x[rng.integers(0, n, size=rng.integers(0, k + 1))] = val
        if rng.random() < 0.5:  # ties for max / argmax
            x[rng.integers(0, n, size=k)] = np.float32(3.0)
    return x


def _same_bits(got, want):
    return np.array_equal(got.view(np.uint32), want.view(np.uint32)) or np.array_equal(got, want, equal_nan=True)


def test_axis_and_full_reductions_random_sweep():
    rng = np.random.default_rng(20261202)
    for index in range(120):
        op = index % 3
        outer = int(rng.choice([1, 1, 2, 3, int(rng.integers(1, 200))]))
        length = int(rng.choice([1, 2, 3, 63, 64, 65, 255, 256, 1000, int(rng.integers(1, 5000))]))
        inner = int(rng.choice([1, 1, 3, 4, 5, 64, 1000, int(rng.integers(1, 2000))]))
        while outer * length * inner > 2_000_000:
            length, inner = max(1, length // 2), max(1, inner // 2)
        special = rng.random() < 0.4
        xh = _data(rng, outer * length * inner, special)
        x, out = C.Buffer.of(xh), C.Buffer((outer * inner,))
        C.check(C.lib().vc_hip_reduce_axis(x.ptr, out.ptr, outer, length, inner, op))
        got = out.numpy()
        want = K.reduce_axis(xh.reshape(outer, length, inner), 1, op).ravel()
        label = f"case {index}: op {op}, {outer} x {length} x {inner}, special values {special}"
        if op == 0:
            assert np.array_equal(np.isnan(got), np.isnan(want)), label
            inf = np.isinf(want)
            assert np.array_equal(got[inf], want[inf]), label
            fin = np.isfinite(want)
            np.testing.assert_allclose(got[fin], want[fin], rtol=1e-6, atol=1e-6 * np.sqrt(length), err_msg=label)
        else:
            assert _same_bits(got, want), label
    for index in range(20):
        n = int(rng.choice([1, 2, 100, 65535, 65536, 65537, int(rng.integers(1, 4_000_000))]))
        special = rng.random() < 0.2
        xh = _data(rng, n, special)
        x, out = C.Buffer.of(xh), C.Buffer((1,))
        C.check(C.lib().vc_hip_reduce_sum(x.ptr, n, out.ptr))
        got, want = out.numpy()[0], K.sum_all(xh)
        assert (np.isnan(got) and np.isnan(want)) or got == want or abs(got - want) <= 1e-6 * max(1.0, abs(want)), \
            f"full sum of {n} (special values {special}): {got} vs {want}"


def test_broadcasting_binary_ops_random_sweep():
    rng = np.random.default_rng(20261203)
    for index in range(120):
        op = index % 4
        rank = int(rng.integers(1, 5))
        out_shape = [int(rng.choice([1, 2, 3, 7, 64, 130, int(rng.integers(1, 200))])) for _ in range(rank)]
        while np.prod(out_shape) > 1_000_000:
            out_shape[int(np.argmax(out_shape))] //= 2

        def operand():
            r = int(rng.integers(1, rank + 1))
            return [d if rng.random() < 0.7 else 1 for d in out_shape[rank - r:]]

        ash, bsh = operand(), operand()
        ah = _data(rng, int(np.prod(ash)), rng.random() < 0.2).reshape(ash)
        bh = _data(rng, int(np.prod(bsh)), rng.random() < 0.2).reshape(bsh)
        full = [int(d) for d in np.broadcast_shapes(tuple(ash), tuple(bsh))]
        want = K.binary(ah, bh, op, full)
        if len(ash) >= 2 and rng.random() < 0.5:  # A read through a transposed view
            stored = np.ascontiguousarray(np.swapaxes(ah, -1, -2))
            a_strides = [int(s // 4) for s in np.swapaxes(stored, -1, -2).strides]
            a = C.Buffer.of(stored)
        else:
            a_strides = [int(s // 4) for s in ah.strides]
            a = C.Buffer.of(np.ascontiguousarray(ah))
        b = C.Buffer.of(np.ascontiguousarray(bh))
        b_strides = [int(s // 4) for s in np.ascontiguousarray(bh).strides]
        out = C.Buffer((int(np.prod(full)),))
        C.check(C.lib().vc_hip_binary(a.ptr, C.sizes(ash), C.sizes(a_strides), len(ash), b.ptr, C.sizes(bsh),
                                      C.sizes(b_strides), len(bsh), out.ptr, C.sizes(full), len(full), op))
        got = out.numpy().reshape(want.shape)
        assert _same_bits(got, want), f"case {index}: op {op}, a {ash}, b {bsh}, out {full}"
