"""The allocation-free axis reduction, vc_hip_reduce_axis_noalloc, against
vc_hip_reduce_axis through the C ABI: the same bits (the same kernels; only
where the partial results live differs), no pool allocation, two calls in a
row with the second on a smaller input, and a clear error, with nothing
launched, for a shape whose partial results exceed the static array."""

import numpy as np
import pytest

from vectorcore_amd import cabi as C

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def device():
    assert C.available(), C.lib().vc_hip_last_error().decode()
    yield
    C.synchronize()


def reduce(fn, dx, outer, length, inner, op):
    out = C.Buffer((outer * inner,))
    C.check(fn(dx.ptr, out.ptr, outer, length, inner, op))
    return out.numpy()


# (outer, length, inner, op) pairs: a larger call, then a smaller one of the
# same kind right after it on the same static array.
PAIRS = [
    ((1, 8192, 4096, C.SUM), (1, 3000, 1000, C.SUM)),    # bias gradients: one launch of ~2048 blocks (1 MiB), one of ~128
    ((1, 8192, 1000, C.SUM), (1, 3000, 300, C.SUM)),     # narrow one launch, then partials and a combine launch
    ((1, 8192, 4096, C.SUM), (1, 4000, 2048, C.SUM)),    # one-launch column sums twice: the chunk counters reset
    ((3, 700, 999, C.SUM), (2, 300, 37, C.SUM)),         # scalar loads, several outer blocks
    ((1, 5000, 300, C.ARGMAX), (1, 900, 70, C.ARGMAX)),  # a long axis split into segments
    ((1, 5000, 300, C.MAX), (2, 400, 33, C.MAX)),
    ((4096, 1000, 1, C.ARGMAX), (100, 37, 1, C.SUM)),    # rows: no partial results
    ((2, 100, 131000, C.SUM), (1, 70, 500, C.SUM)),      # one segment per column: sums written directly, no partials
]


@pytest.mark.parametrize("first,second", PAIRS)
def test_noalloc_matches_pooled_reduction_twice_in_a_row(first, second):
    rng = np.random.default_rng(sum(first[:3]) + sum(second[:3]))
    inputs = []
    for outer, length, inner, op in (first, second):
        x = rng.standard_normal((outer, length, inner)).astype(np.float32)
        if op != C.SUM:
            x.reshape(-1)[:: 7] = x.reshape(-1)[0]  # ties
        inputs.append(C.Buffer.of(x))
    outs = [C.Buffer((o * i,)) for (o, _, i, _) in (first, second)]
    C.synchronize()
    before = C.pool_stats()
    for (outer, length, inner, op), dx, out in zip((first, second), inputs, outs):
        C.check(C.lib().vc_hip_reduce_axis_noalloc(dx.ptr, out.ptr, outer, length, inner, op))
    C.synchronize()
    after = C.pool_stats()
    assert (after.device_allocations, after.reuses) == (before.device_allocations, before.reuses)
    for (outer, length, inner, op), dx, out in zip((first, second), inputs, outs):
        pooled = reduce(C.lib().vc_hip_reduce_axis, dx, outer, length, inner, op)
        np.testing.assert_array_equal(out.numpy(), pooled, err_msg=f"{(outer, length, inner, op)}")


def test_noalloc_rejects_a_shape_beyond_its_array_and_launches_nothing():
    # 100000 outputs of a max over 64 rows split into 3 segments: 2.4 MB of
    # (value, index) partials, more than the 2 MiB array.
    outer, length, inner = 1, 64, 100_000
    dx = C.Buffer.of(np.ones((outer, length, inner), np.float32))
    out = C.Buffer.of(np.full(outer * inner, 7.0, np.float32))
    status = C.lib().vc_hip_reduce_axis_noalloc(dx.ptr, out.ptr, outer, length, inner, C.MAX)
    assert status == 1, status  # VC_HIP_ERR_INVALID_ARGUMENT
    message = C.lib().vc_hip_last_error().decode()
    assert "allocation-free" in message and "bytes" in message, message
    assert (out.numpy() == 7.0).all()
    np.testing.assert_array_equal(reduce(C.lib().vc_hip_reduce_axis, dx, outer, length, inner, C.MAX),
                                  np.ones(inner, np.float32))
    # the array is still usable after a rejected call
    small = C.Buffer.of(np.arange(64 * 10, dtype=np.float32).reshape(1, 64, 10))
    got = reduce(C.lib().vc_hip_reduce_axis_noalloc, small, 1, 64, 10, C.SUM)
    np.testing.assert_array_equal(got, reduce(C.lib().vc_hip_reduce_axis, small, 1, 64, 10, C.SUM))
