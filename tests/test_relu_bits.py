"""ReLU bitmasks: the fused layer product writes the bits of [c > 0]
(vc_hip_matmul_bias_relu_bits) on the 256-row tiles, and the product that
applies the ReLU's backward rule reads its mask from them
(vc_hip_matmul_relu_bits, vc_hip_matmul_relu_bits_colsum_pending): the
same bits as with the float mask they stand for, on every kernel setting
(the other kernels expand the bits into a float mask first)."""

import ctypes

import numpy as np
import pytest

import vectorcore_amd as vc
from vectorcore_amd import cabi as C

pytestmark = pytest.mark.gpu

# "mfma" is the automatic setting; the others force one kernel where the operands allow it.
KERNELS = ["mfma", "mfma128", "simple", "mfma256", "mfma256x128"]
INVALID_ARGUMENT = 1  # VC_HIP_ERR_INVALID_ARGUMENT


@pytest.fixture(scope="module", autouse=True)
def device():
    assert C.available(), C.lib().vc_hip_last_error().decode()
    yield
    C.synchronize()


def pack_relu_bits(x):
    """Bit i % 32 of word [i // 32, j] is [x[i, j] > 0] (rows past the matrix 0)."""
    m, n = x.shape
    pos = np.zeros(((m + 31) // 32 * 32, n), dtype=np.uint64)
    pos[:m] = x > 0
    shifts = np.arange(32, dtype=np.uint64)[None, :, None]
    return (pos.reshape(-1, 32, n) << shifts).sum(axis=1).astype(np.uint32)


def valid_bits(m, n):
    """The bits of rows inside the matrix (the last group's rows past m are unspecified)."""
    keep = np.full(((m + 31) // 32, n), 0xFFFFFFFF, dtype=np.uint32)
    if m % 32:
        keep[-1] = np.uint32((1 << (m % 32)) - 1)
    return keep


def bias_relu_bits(a, b, bias):
    m, k = a.shape
    n = b.shape[1]
    da, db, dbias = C.Buffer.of(a), C.Buffer.of(b), C.Buffer.of(bias)
    c, plain = C.Buffer((m, n)), C.Buffer((m, n))
    words = C.Buffer.of(np.full(((m + 31) // 32, n), 0xA5A5A5A5, dtype=np.uint32), dtype=np.uint32)
    written = ctypes.c_int(-1)
    C.check(C.lib().vc_hip_matmul_bias_relu_bits(da.ptr, db.ptr, c.ptr, m, k, n, dbias.ptr, words.ptr,
                                                 ctypes.byref(written)))
    C.check(C.lib().vc_hip_matmul_bias_relu(da.ptr, db.ptr, plain.ptr, m, k, n, dbias.ptr, 1))
    return c.numpy(), plain.numpy(), words.numpy(), written.value


# 256-row tiles with partial last tiles in both directions, one column tile,
# a K of four; the train step's first layer (NN through a transposed copy of
# B, then the 256 x 256 tiles) and a row count that is not a multiple of 32;
# K not a multiple of 4 (no 16-byte loads: another kernel, no bits).
PRODUCER_SHAPES = [(300, 96, 520), (1030, 64, 700), (260, 4, 8), (8192, 1024, 4096), (4100, 1028, 4096),
                   (300, 97, 520)]


@pytest.mark.parametrize("kernel", KERNELS)
@pytest.mark.parametrize("m,k,n", PRODUCER_SHAPES)
def test_layer_product_writes_the_bits_of_its_positive_outputs(kernel, m, k, n):
    rng = np.random.default_rng(m + 7 * k + n)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    bias[:3] = [np.inf, -np.inf, 0.0]
    with C.gemm_kernel(kernel):
        c, plain, words, written = bias_relu_bits(a, b, bias)
    np.testing.assert_array_equal(c, plain)  # the same bits as the layer product without them
    fits = k % 4 == 0 and n % 4 == 0
    if kernel in ("mfma256", "mfma256x128"):
        assert written == int(fits)
    elif kernel in ("mfma128", "simple"):
        assert written == 0
    elif (m, k, n) == (8192, 1024, 4096):
        assert written == 1  # the train step's layer takes the 256 x 256 tiles
    if written:
        keep = valid_bits(m, n)
        np.testing.assert_array_equal(words & keep, pack_relu_bits(c) & keep)
    else:
        assert (words == 0xA5A5A5A5).all()  # not written


def masked_pair(m, k, n, ta, tb, seed):
    rng = np.random.default_rng(seed)
    a = rng.uniform(-1, 1, size=(k, m) if ta else (m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, size=(n, k) if tb else (k, n)).astype(np.float32)
    mask = rng.standard_normal((m, n)).astype(np.float32)
    mask[rng.random((m, n)) < 0.1] = 0.0
    mask.flat[:6] = [0.0, -0.0, np.nan, np.inf, -np.inf, 1e-38]
    return a, b, mask


# The train step's second masked product (8192 x 4096, K = 1000: the
# 256 x 256 tiles with the bits); partial tiles; a split-K shape and a small
# one (other kernels: the bits are expanded first).
CONSUMER_SHAPES = [(8192, 1000, 4096), (300, 96, 520), (1030, 64, 700), (4100, 1028, 4096), (2048, 4096, 64),
                   (100, 70, 33)]


@pytest.mark.parametrize("kernel", KERNELS)
@pytest.mark.parametrize("m,k,n", CONSUMER_SHAPES)
def test_bits_mask_the_product_as_the_float_mask_does(kernel, m, k, n):
    z0 = C.sizes([0])
    for ta, tb in ((0, 1), (0, 0), (1, 0)):
        if (m, k, n) == (8192, 1000, 4096) and (ta, tb) != (0, 1):
            continue  # the full-size shape once, as the step runs it
        a, b, mask = masked_pair(m, k, n, ta, tb, m + k + n + 2 * ta + tb)
        da, db, dm = C.Buffer.of(a), C.Buffer.of(b), C.Buffer.of(mask)
        dw = C.Buffer.of(pack_relu_bits(mask), dtype=np.uint32)
        with C.gemm_kernel(kernel):
            want, got = C.Buffer((m, n)), C.Buffer((m, n))
            C.check(C.lib().vc_hip_matmul_relu_mask(da.ptr, db.ptr, want.ptr, m, k, n, z0, z0, 1, ta, tb, dm.ptr))
            C.check(C.lib().vc_hip_matmul_relu_bits(da.ptr, db.ptr, got.ptr, m, k, n, ta, tb, dw.ptr))
            np.testing.assert_array_equal(got.numpy(), want.numpy(), err_msg=f"{kernel} ta={ta} tb={tb}")
            sums = []
            for entry, operand in ((C.lib().vc_hip_matmul_relu_mask_colsum_pending, dm),
                                   (C.lib().vc_hip_matmul_relu_bits_colsum_pending, dw)):
                c, s, h = C.Buffer((m, n)), C.Buffer((n,)), ctypes.c_void_p()
                C.check(entry(da.ptr, db.ptr, c.ptr, m, k, n, ta, tb, operand.ptr, s.ptr, ctypes.byref(h)))
                if h.value:
                    C.check(C.lib().vc_hip_colsum_finish(h, s.ptr))
                    C.check(C.lib().vc_hip_colsum_release(h))
                sums.append((c.numpy(), s.numpy()))
            np.testing.assert_array_equal(sums[1][0], sums[0][0])
            np.testing.assert_array_equal(sums[1][1], sums[0][1])
            np.testing.assert_array_equal(sums[1][0], want.numpy())


def test_layer_bits_feed_the_relu_backward_product():
    """The bits a layer product writes, read by dH = dY W^T, give the product
    masked by the layer's output (the train step's first layer and its
    gradient)."""
    m, k, n, k2 = 8192, 1024, 4096, 1000
    rng = np.random.default_rng(12)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = (rng.uniform(-1, 1, size=(k, n)) / np.sqrt(k)).astype(np.float32)
    bias = (rng.uniform(-1, 1, size=n) / np.sqrt(k)).astype(np.float32)
    h, _, words, written = bias_relu_bits(x, w, bias)
    assert written == 1
    dy = rng.standard_normal((m, k2)).astype(np.float32)
    w2 = rng.standard_normal((n, k2)).astype(np.float32)
    ddy, dw2, dh = C.Buffer.of(dy), C.Buffer.of(w2), C.Buffer.of(h)
    dwords = C.Buffer.of(words, dtype=np.uint32)
    got, want = C.Buffer((m, n)), C.Buffer((m, n))
    C.check(C.lib().vc_hip_matmul_relu_bits(ddy.ptr, dw2.ptr, got.ptr, m, k2, n, 0, 1, dwords.ptr))
    C.check(C.lib().vc_hip_matmul_relu_mask(ddy.ptr, dw2.ptr, want.ptr, m, k2, n, C.sizes([0]), C.sizes([0]), 1,
                                            0, 1, dh.ptr))
    np.testing.assert_array_equal(got.numpy(), want.numpy())


def test_bits_entry_points_reject_null_arguments():
    a = C.Buffer.of(np.ones((4, 4), np.float32))
    flag = ctypes.c_int()
    assert C.lib().vc_hip_matmul_bias_relu_bits(a.ptr, a.ptr, a.ptr, 4, 4, 4, None, None,
                                                ctypes.byref(flag)) == INVALID_ARGUMENT
    assert C.lib().vc_hip_matmul_relu_bits(a.ptr, a.ptr, a.ptr, 4, 4, 4, 0, 1, None) == INVALID_ARGUMENT
    s, h = C.Buffer((4,)), ctypes.c_void_p()
    assert C.lib().vc_hip_matmul_relu_bits_colsum_pending(a.ptr, a.ptr, a.ptr, 4, 4, 4, 0, 1, None, s.ptr,
                                                          ctypes.byref(h)) == INVALID_ARGUMENT


def test_train_step_reads_the_relu_masks_as_bits():
    """In an MLP's backward with deferred layers, the two masked products read
    the layers' bits (each product's traffic count includes m n / 8 bytes of
    mask, not 4 m n) and give the gradients of the eager layers bit for bit."""
    rng = np.random.default_rng(3)
    # 4096 rows and 4096-wide hidden layers: every product is a full round of
    # 256 x 256 tiles, so none splits K (a split product's mask is applied
    # after the split sum, from expanded bits).
    m, sizes = 4096, [256, 4096, 4096, 100]
    xs = rng.standard_normal((m, sizes[0])).astype(np.float32)
    targets = rng.integers(0, sizes[-1], m)
    ws = [(rng.uniform(-1, 1, size=(i, o)) / np.sqrt(i)).astype(np.float32) for i, o in zip(sizes, sizes[1:])]
    bs = [(rng.uniform(-1, 1, size=o) / np.sqrt(i)).astype(np.float32) for i, o in zip(sizes, sizes[1:])]

    def step(defer):
        previous = vc.hip_defer_products(defer)
        try:
            with C.gemm_kernel("mfma256"):
                params = [vc.Tensor(p, requires_grad=True, device="hip") for pair in zip(ws, bs) for p in pair]
                h = vc.Tensor(xs, device="hip")
                for i in range(3):
                    h = h @ params[2 * i] + params[2 * i + 1]
                    if i < 2:
                        h = h.relu()
                loss = vc.cross_entropy(h, [int(t) for t in targets])
                C.profile(True)
                C.profile_reset()
                loss.backward()
                vc.synchronize()
                prof = C.profile_read()
                C.profile(False)
                return [np.array(p.grad.numpy(), copy=True) for p in params], prof
        finally:
            vc.hip_defer_products(previous)

    eager, _ = step(False)
    deferred, prof = step(True)
    for g_eager, g_deferred in zip(eager, deferred):
        np.testing.assert_array_equal(g_deferred, g_eager)
    nt = prof["gemm_nt"]
    assert nt["launches"] == 2
    # dH2 (4096 x 4096, K = 100) and dH1 (4096 x 4096, K = 4096): operands, C
    # and 1/8 byte of mask per element
    want = sum(4.0 * (m * kk + kk * n + m * n) + m * n / 8.0 for kk, n in ((100, 4096), (4096, 4096)))
    assert nt["bytes"] == want


def test_bits_random_sweep():
    """Seeded random shapes (tile edges, odd sizes, aligned and not), transposes
    and kernel settings: the product masked by bits is the float-mask
    product's bits, and the layer product's bits are [c > 0] where written."""
    rng = np.random.default_rng(2024)
    edges = [1, 3, 4, 31, 32, 33, 64, 127, 128, 129, 255, 256, 257, 300, 513]
    z0 = C.sizes([0])
    for case in range(40):
        m, n = (int(rng.choice(edges)) if rng.random() < 0.5 else int(rng.integers(1, 700)) for _ in range(2))
        k = int(rng.choice([1, 4, 16, 32, 33, 64, 100, 256, 300]))
        ta, tb = int(rng.random() < 0.3), int(rng.random() < 0.6)
        kernel = KERNELS[case % len(KERNELS)]
        a, b, mask = masked_pair(m, k, n, ta, tb, 1000 + case)
        da, db, dm = C.Buffer.of(a), C.Buffer.of(b), C.Buffer.of(mask)
        dw = C.Buffer.of(pack_relu_bits(mask), dtype=np.uint32)
        with C.gemm_kernel(kernel):
            want, got = C.Buffer((m, n)), C.Buffer((m, n))
            C.check(C.lib().vc_hip_matmul_relu_mask(da.ptr, db.ptr, want.ptr, m, k, n, z0, z0, 1, ta, tb, dm.ptr))
            C.check(C.lib().vc_hip_matmul_relu_bits(da.ptr, db.ptr, got.ptr, m, k, n, ta, tb, dw.ptr))
            np.testing.assert_array_equal(got.numpy(), want.numpy(), err_msg=f"case {case}: {m}x{k}x{n} "
                                          f"ta={ta} tb={tb} {kernel}")
            x = rng.standard_normal((m, k)).astype(np.float32)
            w = rng.standard_normal((k, n)).astype(np.float32)
            bias = rng.standard_normal(n).astype(np.float32)
            c, plain, words, written = bias_relu_bits(x, w, bias)
        np.testing.assert_array_equal(c, plain, err_msg=f"case {case}")
        if written:
            keep = valid_bits(m, n)
            np.testing.assert_array_equal(words & keep, pack_relu_bits(c) & keep, err_msg=f"case {case}")
