"""GPU parity of every C-ABI entry point (include/vc_hip.h) against the oracle.

Bars: bit-exact for indices (argmax), for pure-fp32 elementwise chains and
for data movement; the reference's own tolerance pairs elsewhere (GEMM:
rtol 1e-4, atol 1e-4 sqrt(k), tests/python/test_performance_paths.py:43);
reductions within 1e-4 relative; transcendental elementwise results within
1e-5 relative.
"""

import ctypes

import numpy as np
import pytest

from oracle import kernels as K
from tests.golden.make_golden import GEMM_SHAPES, gemm_inputs
from vectorcore_amd import cabi as C
from vectorcore_amd import workloads as W

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def device():
    assert C.available(), C.lib().vc_hip_last_error().decode()
    yield
    C.synchronize()


@pytest.fixture(params=["mfma", "simple", "mfma256", "mfma256x128"])
def gemm_kernel(request):
    """Runs a GEMM test on the MFMA kernels, again on the portable FMA kernel
    (the reference re-runs its matmul tests with its portable kernel forced,
    tests/python/test_performance_paths.py:89-103), and again with every
    product whose operands allow it on the 256 x 256 and on the 256 x 128
    tiles, so that their edges (partial tiles, K past the last slice, split K)
    are checked on small shapes too."""
    with C.gemm_kernel(request.param):
        assert C.lib().vc_hip_gemm_kernel().decode() == request.param
        yield request.param


def run_gemm(a, b, m, k, n, ta, tb, batch=1, a_offsets=None, b_offsets=None):
    da, db = C.Buffer.of(a), C.Buffer.of(b)
    dc = C.Buffer((batch, m, n))
    ao = a_offsets if a_offsets is not None else [z * m * k for z in range(batch)]
    bo = b_offsets if b_offsets is not None else [z * k * n for z in range(batch)]
    C.check(C.lib().vc_hip_matmul(da.ptr, db.ptr, dc.ptr, m, k, n, C.sizes(ao), C.sizes(bo), batch, int(ta), int(tb)))
    return dc.numpy()


@pytest.mark.parametrize("m,k,n", GEMM_SHAPES)
def test_gemm_matches_reference_fixture(golden, gemm_kernel, m, k, n):
    for ta in (0, 1):
        for tb in (0, 1):
            a, b = gemm_inputs(m, k, n, ta, tb)
            got = run_gemm(a, b, m, k, n, ta, tb)[0]
            np.testing.assert_allclose(got, golden[f"gemm_{m}_{k}_{n}_{ta}{tb}_c"], rtol=1e-4, atol=1e-4 * np.sqrt(k),
                                       err_msg=f"trans_a={ta} trans_b={tb}")


# The first nine shapes are above the FMA kernel's threshold (2^20
# multiply-adds with K <= 1024), so with "mfma" they run on a matrix-core
# kernel: the 32 x 32 tiles of small products up to (512, 1024, 1000), the
# 128 x 128 tiles from 65 of them (1030, 129, 1100) and (1100, 256, 1030), and
# (1, 4096, 3) with K split across 128 x 128 workgroups. Covered: a whole
# tile, a partial K slice (60, 129), partial m and n tiles (130, 70, 257, 383,
# 1030, 1100), and vector and scalar loads in all four transposes. The last
# three run on the FMA kernel with either setting, except that "mfma" gives
# (64, 300, 3) with A transposed (a weight gradient, K the batch) to the
# 32 x 32 tiles: K in one slice (7), and K over two and four of its 256-deep
# slices (300, 1000), the last partial.
@pytest.mark.parametrize("m,k,n", [(256, 64, 128), (192, 256, 64), (256, 60, 128), (130, 64, 128), (256, 64, 70),
                                   (257, 129, 383), (512, 1024, 1000), (1030, 129, 1100), (1100, 256, 1030),
                                   (1, 4096, 3), (2000, 7, 129), (1000, 7, 1), (64, 300, 3), (2, 1000, 64)])
def test_gemm_edges_against_oracle(gemm_kernel, m, k, n):
    rng = np.random.default_rng(m * 7 + k * 3 + n)
    for ta in (0, 1):
        for tb in (0, 1):
            a = rng.uniform(-1, 1, size=(k, m) if ta else (m, k)).astype(np.float32)
            b = rng.uniform(-1, 1, size=(n, k) if tb else (k, n)).astype(np.float32)
            np.testing.assert_allclose(run_gemm(a, b, m, k, n, ta, tb)[0], K.matmul2d(a, b, bool(ta), bool(tb)),
                                       rtol=1e-4, atol=1e-4 * np.sqrt(k), err_msg=f"trans_a={ta} trans_b={tb}")


# Products on both sides of the rule that gives small products the 32 x 32
# tiles (gemm_small_kernel: up to 64 tiles of 128 x 128 with K <= 2048, or 9 to
# 32 tiles with any K) and the rest the 128 x 128 tiles (K split across
# workgroups when they are few: 1100 x 2100 x 500 in two ranges of at least 32
# slices; 2000 x 1100 x 700 (96 tiles) and two 700 x 1500 x 1200 (120 tiles) in
# two ranges of at least 16): checked against float64 with the reference's
# tolerance and repeated bit for bit.
@pytest.mark.parametrize("m,k,n,batch", [(1024, 1024, 1024, 1), (1100, 2100, 300, 1), (300, 4100, 1100, 1),
                                         (65, 2047, 4033, 1), (100, 515, 90, 5), (1100, 2100, 500, 1),
                                         (2049, 1024, 1025, 1), (96, 4100, 96, 2), (40, 8192, 40, 1),
                                         (2000, 1100, 700, 1), (700, 1500, 1200, 2)])
def test_gemm_on_both_sides_of_the_small_tile_rule(m, k, n, batch):
    rng = np.random.default_rng(m + 3 * k + 7 * n + batch)
    for ta, tb in ((0, 0), (1, 0), (0, 1), (1, 1)):
        a = rng.uniform(-1, 1, size=(batch,) + ((k, m) if ta else (m, k))).astype(np.float32)
        b = rng.uniform(-1, 1, size=(batch,) + ((n, k) if tb else (k, n))).astype(np.float32)
        got = run_gemm(a, b, m, k, n, ta, tb, batch=batch)
        want = np.matmul((a.transpose(0, 2, 1) if ta else a).astype(np.float64),
                         (b.transpose(0, 2, 1) if tb else b).astype(np.float64))
        np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-4 * np.sqrt(k),
                                   err_msg=f"{m}x{k}x{n} b{batch} ta={ta} tb={tb}")
        np.testing.assert_array_equal(run_gemm(a, b, m, k, n, ta, tb, batch=batch), got)


@pytest.mark.parametrize("m,k,n", [(33, 70, 41), (200, 300, 150)])
def test_gemm_batched_offsets_affine_and_table(gemm_kernel, m, k, n):
    # (33, 70, 41) runs on the FMA kernel, (200, 300, 150) with "mfma" on the
    # 32 x 32 tiles.
    rng = np.random.default_rng(3)
    a = rng.standard_normal((4, m, k)).astype(np.float32)
    b = rng.standard_normal((2, k, n)).astype(np.float32)
    # batch z reads a[z] and b[z % 2]: not affine, goes through the offset table
    got = run_gemm(a, b, m, k, n, 0, 0, batch=4, a_offsets=[z * m * k for z in range(4)],
                   b_offsets=[(z % 2) * k * n for z in range(4)])
    for z in range(4):
        np.testing.assert_allclose(got[z], K.matmul2d(a[z], b[z % 2]), rtol=1e-4, atol=1e-4 * np.sqrt(k))
    # broadcast B: affine with stride 0
    got = run_gemm(a, b, m, k, n, 0, 0, batch=4, b_offsets=[0, 0, 0, 0])
    for z in range(4):
        np.testing.assert_allclose(got[z], K.matmul2d(a[z], b[0]), rtol=1e-4, atol=1e-4 * np.sqrt(k))


def test_gemm_split_k_long_reductions(gemm_kernel):
    """Few output tiles and a long K: the K range is split across workgroups
    and the partial products are summed in split order, so results repeat
    bit for bit."""
    rng = np.random.default_rng(11)
    for (m, k, n, batch) in ((257, 4133, 383, 1), (64, 2100, 96, 3), (130, 8192, 1, 1)):
        for ta, tb in ((0, 0), (1, 0), (0, 1), (1, 1)):
            a = rng.uniform(-1, 1, size=(batch,) + ((k, m) if ta else (m, k))).astype(np.float32)
            b = rng.uniform(-1, 1, size=(batch,) + ((n, k) if tb else (k, n))).astype(np.float32)
            got = run_gemm(a, b, m, k, n, ta, tb, batch=batch)
            for z in range(batch):
                np.testing.assert_allclose(got[z], K.matmul2d(a[z], b[z], bool(ta), bool(tb)), rtol=1e-4,
                                           atol=1e-4 * np.sqrt(k), err_msg=f"{m}x{k}x{n} b{batch} ta={ta} tb={tb}")
            np.testing.assert_array_equal(run_gemm(a, b, m, k, n, ta, tb, batch=batch), got)


def test_gemm_relu_mask_is_gemm_then_relu_backward_bitexact(gemm_kernel):
    """vc_hip_matmul_relu_mask = vc_hip_matmul, then vc_hip_relu_backward with
    the same mask source: same bits, including a split-K shape and a batch."""
    rng = np.random.default_rng(21)
    for (m, k, n, batch) in ((257, 129, 383, 1), (130, 8192, 64, 1), (64, 96, 72, 3)):
        for ta, tb in ((0, 0), (0, 1), (1, 0), (1, 1)):
            a = rng.uniform(-1, 1, size=(batch,) + ((k, m) if ta else (m, k))).astype(np.float32)
            b = rng.uniform(-1, 1, size=(batch,) + ((n, k) if tb else (k, n))).astype(np.float32)
            x = rng.standard_normal((batch, m, n)).astype(np.float32)
            x.flat[:5] = [0.0, -0.0, np.nan, np.inf, -np.inf]
            da, db, dx = C.Buffer.of(a), C.Buffer.of(b), C.Buffer.of(x)
            fused, plain, masked = C.Buffer((batch, m, n)), C.Buffer((batch, m, n)), C.Buffer((batch, m, n))
            ao, bo = C.sizes([z * m * k for z in range(batch)]), C.sizes([z * k * n for z in range(batch)])
            C.check(C.lib().vc_hip_matmul_relu_mask(da.ptr, db.ptr, fused.ptr, m, k, n, ao, bo, batch, ta, tb, dx.ptr))
            C.check(C.lib().vc_hip_matmul(da.ptr, db.ptr, plain.ptr, m, k, n, ao, bo, batch, ta, tb))
            C.check(C.lib().vc_hip_relu_backward(plain.ptr, dx.ptr, masked.ptr, batch * m * n))
            np.testing.assert_array_equal(fused.numpy(), masked.numpy(), err_msg=f"{m}x{k}x{n} ta={ta} tb={tb}")
            assert (fused.numpy() == 0).any() and (fused.numpy() != 0).any()


# Shapes that run unsplit on both tile sizes: K below 4 slices of 32 (no split
# for few tiles), or at least 256 tiles of 256 x 256 (a full round of
# workgroups on either kernel); partial tiles along m and n, and K not a
# multiple of the 32-deep slice.
BIG_VS_128 = [(300, 96, 520), (1030, 64, 700), (260, 4, 8), (4096, 256, 4096), (4000, 200, 4100), (4100, 1028, 4096)]


@pytest.mark.parametrize("m,k,n", BIG_VS_128)
def test_big_tiles_give_the_bits_of_the_128_tiles(m, k, n):
    """The 256 x 256 and 256 x 128 tiles compute each 64 x 64 block of C as a
    128 x 128 tile's wave does (same MFMA blocks, lane layouts and k order), so
    products, the fused ReLU mask, the bias + ReLU epilogue and the column-sum
    partial rows are the same bits on all three, in all four transposes."""
    rng = np.random.default_rng(m + 3 * k + 5 * n)
    x = rng.standard_normal((m, n)).astype(np.float32)
    x.flat[:5] = [0.0, -0.0, np.nan, np.inf, -np.inf]
    bias = rng.standard_normal(n).astype(np.float32)
    dx, dbias = C.Buffer.of(x), C.Buffer.of(bias)
    z0 = C.sizes([0])
    for ta, tb in ((0, 0), (0, 1), (1, 0), (1, 1)):
        a = rng.uniform(-1, 1, size=(k, m) if ta else (m, k)).astype(np.float32)
        b = rng.uniform(-1, 1, size=(n, k) if tb else (k, n)).astype(np.float32)
        da, db = C.Buffer.of(a), C.Buffer.of(b)
        outs = {}
        for kernel in ("mfma128", "mfma256", "mfma256x128"):
            with C.gemm_kernel(kernel):
                plain, masked, sums = C.Buffer((m, n)), C.Buffer((m, n)), C.Buffer((n,))
                C.check(C.lib().vc_hip_matmul(da.ptr, db.ptr, plain.ptr, m, k, n, z0, z0, 1, ta, tb))
                C.check(C.lib().vc_hip_matmul_relu_mask_colsum(da.ptr, db.ptr, masked.ptr, m, k, n, ta, tb, dx.ptr,
                                                               sums.ptr))
                outs[kernel] = [plain.numpy(), masked.numpy(), sums.numpy()]
                if not ta and not tb:
                    fwd = C.Buffer((m, n))
                    C.check(C.lib().vc_hip_matmul_bias_relu(da.ptr, db.ptr, fwd.ptr, m, k, n, dbias.ptr, 1))
                    outs[kernel].append(fwd.numpy())
        for big in ("mfma256", "mfma256x128"):
            for name, x128, xbig in zip(("product", "masked", "column sums", "bias + relu"), outs["mfma128"],
                                        outs[big]):
                np.testing.assert_array_equal(xbig, x128, err_msg=f"{big}: {name} {m}x{k}x{n} ta={ta} tb={tb}")
        rows = rng.choice(m, min(m, 48), replace=False)
        opa = (a.T if ta else a)[rows]
        np.testing.assert_allclose(outs["mfma256"][0][rows], K.matmul2d(np.ascontiguousarray(opa), b, False, bool(tb)),
                                   rtol=1e-4, atol=1e-4 * np.sqrt(k))


@pytest.mark.parametrize("m,k,n", [(300, 257, 130), (128, 64, 200), (100, 70, 33), (4096, 512, 1000),
                                   (1000, 256, 1100), (1030, 128, 1030), (2048, 4096, 64), (8192, 1000, 4096)])
def test_masked_product_with_column_sums(gemm_kernel, m, k, n):
    """vc_hip_matmul_relu_mask_colsum: the product is vc_hip_matmul_relu_mask's
    bits, and the column sums equal the reduction of that product (the
    oracle's sequential double sum) to the last bit or within 1e-6. Covers
    128 x 128 tiles (whole rows; a partial last tile of 104 rows; one of 6
    rows), 32 x 32 tiles (a few 128 x 128 tiles' worth: 300 x 130, 128 x
    200), the FMA kernel (100 x 33), a split-K shape (2048 x 4096 x 64: the
    sums come from a separate reduction) and the portable kernel (the
    same)."""
    rng = np.random.default_rng(m + k + n)
    a = rng.uniform(-1, 1, size=(m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, size=(n, k)).astype(np.float32)
    x = rng.standard_normal((m, n)).astype(np.float32)
    x.flat[:4] = [0.0, -0.0, np.nan, np.inf]
    da, db, dx = C.Buffer.of(a), C.Buffer.of(b), C.Buffer.of(x)
    fused, plain, sums = C.Buffer((m, n)), C.Buffer((m, n)), C.Buffer((n,))
    C.check(C.lib().vc_hip_matmul_relu_mask_colsum(da.ptr, db.ptr, fused.ptr, m, k, n, 0, 1, dx.ptr, sums.ptr))
    C.check(C.lib().vc_hip_matmul_relu_mask(da.ptr, db.ptr, plain.ptr, m, k, n, C.sizes([0]), C.sizes([0]), 1, 0, 1,
                                            dx.ptr))
    product = plain.numpy()
    np.testing.assert_array_equal(fused.numpy(), product)
    want = K.reduce_axis(product, 0, K.SUM)
    got = sums.numpy()
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-6 * np.abs(product).sum(0).max())
    assert (got == want).mean() > 0.99


# 32 x 32 tiles (6 full tiles of rows, then 8 rows); 128 x 128 tiles (7 full
# tiles of rows, then 104 rows)
@pytest.mark.parametrize("m,n", [(200, 96), (1000, 1100)])
def test_column_sums_leave_out_rows_past_the_matrix(m, n):
    # An infinity in B makes the padded rows of the last tile NaN (0 * inf);
    # those rows are not part of C and must not reach the sums.
    rng = np.random.default_rng(5)
    k = 64
    a = rng.uniform(0.5, 1, size=(m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, size=(n, k)).astype(np.float32)
    b[7, 3] = np.inf
    x = np.ones((m, n), np.float32)
    da, db, dx = C.Buffer.of(a), C.Buffer.of(b), C.Buffer.of(x)
    out, sums = C.Buffer((m, n)), C.Buffer((n,))
    C.check(C.lib().vc_hip_matmul_relu_mask_colsum(da.ptr, db.ptr, out.ptr, m, k, n, 0, 1, dx.ptr, sums.ptr))
    got, product = sums.numpy(), out.numpy()
    assert np.isposinf(got[7]) and np.isposinf(product[:, 7]).all()
    np.testing.assert_allclose(np.delete(got, 7), np.delete(K.reduce_axis(product, 0, K.SUM), 7), rtol=1e-6)


def test_large_nn_product_runs_as_nt_on_a_transposed_copy_with_the_same_bits():
    """From 4096 rows an NN product transposes B and runs the NT kernel; the
    LDS tiles, and so the bits, are those of NN on B as stored. Shapes below
    and above the threshold, with edges that are not multiples of the tile."""
    rng = np.random.default_rng(31)
    for (m, k, n) in ((4100, 516, 132), (4095, 516, 132), (8192, 1024, 1000)):
        a = rng.uniform(-1, 1, size=(m, k)).astype(np.float32)
        b = rng.uniform(-1, 1, size=(k, n)).astype(np.float32)
        nn = run_gemm(a, b, m, k, n, 0, 0)[0]
        nt = run_gemm(a, np.ascontiguousarray(b.T), m, k, n, 0, 1)[0]
        np.testing.assert_array_equal(nn, nt, err_msg=f"{m}x{k}x{n}")
        rows = rng.choice(m, 64, replace=False)
        np.testing.assert_allclose(nn[rows], K.matmul2d(a[rows], b), rtol=1e-4, atol=1e-4 * np.sqrt(k))


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (300, 513, 257), (129, 64, 4100), (64, 4096, 64), (256, 2048, 384),
                                   (4100, 516, 132)])
def test_matmul_bias_relu_is_product_then_add_then_relu_bitexact(gemm_kernel, m, k, n):
    # The fused epilogue against the unfused product followed by the row add
    # and ReLU in fp32 (x > 0 ? x : 0). (64, 4096, 64) splits K, so the
    # epilogue runs in the split combine; (4100, 516, 132) takes the
    # transposed-B route of large products.
    rng = np.random.default_rng(m + k + n)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    product = run_gemm(a, b, m, k, n, False, False)[0]
    np.testing.assert_allclose(product, K.matmul2d(a, b), rtol=1e-4, atol=1e-4 * np.sqrt(k))
    da, db, dbias = C.Buffer.of(a), C.Buffer.of(b), C.Buffer.of(bias)
    for with_bias, relu in [(True, True), (True, False), (False, True)]:
        dc = C.Buffer((m, n))
        C.check(C.lib().vc_hip_matmul_bias_relu(da.ptr, db.ptr, dc.ptr, m, k, n, dbias.ptr if with_bias else None,
                                                int(relu)))
        expected = product + bias if with_bias else product.copy()
        if relu:
            expected = np.where(expected > 0, expected, np.float32(0))
        np.testing.assert_array_equal(dc.numpy(), expected)


def test_gemm_batch_reduce_matches_summed_products(gemm_kernel):
    """dB of a batch-broadcast B: sum_z A[z]^T dC[z] in one launch."""
    bm = W.bmm(batch=3, m=96, k=80, n=72, seed=1)
    a, dc = bm["a"], bm["dc"]
    da, ddc = C.Buffer.of(a), C.Buffer.of(dc)
    out = C.Buffer((80, 72))
    C.check(C.lib().vc_hip_matmul_reduce(da.ptr, ddc.ptr, out.ptr, 80, 96, 72, 3, 96 * 80, 96 * 72, 1, 0))
    expected = K.reduce_axis(K.matmul(a, dc, True, False), 0, K.SUM)
    np.testing.assert_allclose(out.numpy(), expected, rtol=1e-4, atol=1e-4 * np.sqrt(3 * 96))


# Config 2's broadcast dB (8 products of 1024^3: one product per split on
# 256 x 128 tiles), partial tiles with 3 products, K past the last slice, all
# four transposes, and a product count that exceeds one round (the 128 x 128
# tiles then, whatever the setting).
@pytest.mark.parametrize("m,k,n,count", [(1024, 1024, 1024, 8), (300, 100, 520, 3), (1030, 64, 700, 2),
                                         (2048, 256, 2048, 8)])
def test_batch_reduce_on_the_256_row_tiles_gives_the_bits_of_the_128_tiles(m, k, n, count):
    """A batch reduction split one product per split computes each product's
    64 x 64 blocks as the 128 x 128 tiles do and adds the partials in split
    order: the same bits on both tile sizes."""
    rng = np.random.default_rng(m + k + n + count)
    for ta, tb in ((1, 0), (0, 1), (0, 0), (1, 1)):
        a = rng.standard_normal((count, k, m) if ta else (count, m, k)).astype(np.float32)
        b = rng.standard_normal((count, n, k) if tb else (count, k, n)).astype(np.float32)
        da, db = C.Buffer.of(a), C.Buffer.of(b)
        outs = {}
        for kernel in ("mfma128", "mfma", "mfma256x128", "mfma256"):
            with C.gemm_kernel(kernel):
                out = C.Buffer((m, n))
                C.check(C.lib().vc_hip_matmul_reduce(da.ptr, db.ptr, out.ptr, m, k, n, count, m * k, k * n, ta, tb))
                outs[kernel] = out.numpy()
        # The automatic setting takes the 256 x 128 tiles for config 2's case;
        # the smaller products take the 32 x 32 tiles (other bits).
        same = ("mfma", "mfma256x128", "mfma256") if (m, k, n, count) == (1024, 1024, 1024, 8) else \
            ("mfma256x128", "mfma256")
        for kernel in same:
            np.testing.assert_array_equal(outs[kernel], outs["mfma128"], err_msg=f"{kernel} ta={ta} tb={tb}")
        rows = rng.choice(m, min(m, 24), replace=False)
        opa = np.swapaxes(a, 1, 2) if ta else a
        opb = np.swapaxes(b, 1, 2) if tb else b
        want = np.einsum("zik,zkj->ij", opa[:, rows].astype(np.float64), opb.astype(np.float64))
        np.testing.assert_allclose(outs["mfma"][rows], want, rtol=1e-4, atol=1e-4 * np.sqrt(count * k))


def binary_dev(a, b, op):
    a, b = K.f32(a), K.f32(b)
    shape = K.broadcast_shape(a.shape, b.shape)
    da, db, dy = C.Buffer.of(a), C.Buffer.of(b), C.Buffer(shape)
    sa = [int(np.prod(a.shape[i + 1:])) for i in range(a.ndim)]
    sb = [int(np.prod(b.shape[i + 1:])) for i in range(b.ndim)]
    C.check(C.lib().vc_hip_binary(da.ptr, C.sizes(a.shape), C.sizes(sa), a.ndim, db.ptr, C.sizes(b.shape),
                                  C.sizes(sb), b.ndim, dy.ptr, C.sizes(shape), len(shape), op))
    return dy.numpy()


BROADCAST_CASES = [((1000, 300), (1000, 300)), ((1000, 300), ()), ((), (1000, 300)), ((1000, 300), (300,)),
                   ((1000, 300), (1000, 1)), ((1000, 1), (1, 300)), ((40, 1, 300), (1, 50, 300)),
                   ((40, 50, 1), (50, 7)), ((3,), (2, 1)), ((4096, 4096), (1, 4096)), ((7, 9), (7, 9))]


@pytest.mark.parametrize("a_shape,b_shape", BROADCAST_CASES)
def test_binary_bitexact(a_shape, b_shape):
    rng = np.random.default_rng(len(a_shape) * 13 + len(b_shape))
    a = rng.uniform(0.5, 2, size=a_shape).astype(np.float32)
    b = rng.uniform(0.5, 2, size=b_shape).astype(np.float32)
    for op in (C.ADD, C.SUB, C.MUL, C.DIV):
        np.testing.assert_array_equal(binary_dev(a, b, op), K.binary(a, b, op), err_msg=f"op {op}")


def test_binary_scalar_operand_bitexact():
    x = np.random.default_rng(4).standard_normal(10_001).astype(np.float32)
    dx, dy = C.Buffer.of(x), C.Buffer(x.shape)
    for op in (C.ADD, C.SUB, C.MUL, C.DIV):
        for first in (0, 1):
            C.check(C.lib().vc_hip_binary_scalar(dx.ptr, x.size, ctypes.c_float(0.1), first, dy.ptr, op))
            s = np.float32(0.1)
            expected = K.binary(s, x, op) if first else K.binary(x, s, op)
            np.testing.assert_array_equal(dy.numpy(), expected)


def unary_dev(x, op):
    dx, dy = C.Buffer.of(x), C.Buffer(x.shape)
    C.check(C.lib().vc_hip_unary(dx.ptr, dy.ptr, x.size, op))
    return dy.numpy()


def test_unary_against_oracle():
    x = np.random.default_rng(3).uniform(-5, 5, size=(700, 301)).astype(np.float32)
    x[0, :4] = [0.0, -0.0, np.nan, np.inf]
    for op in (C.NEG, C.RELU, C.RELU_GRAD):
        np.testing.assert_array_equal(unary_dev(x, op), K.unary(x, op))
    for op in (C.SIGMOID, C.EXP):
        np.testing.assert_allclose(unary_dev(x, op), K.unary(x, op), rtol=1e-5, atol=0)
    pos = np.abs(x[1:]) + np.float32(1e-3)
    np.testing.assert_allclose(unary_dev(pos, C.LOG), K.unary(pos, C.LOG), rtol=1e-5, atol=1e-7)


def test_fused_activation_gradients_bitexact():
    rng = np.random.default_rng(5)
    g = rng.standard_normal(100_003).astype(np.float32)
    x = rng.standard_normal(100_003).astype(np.float32)
    x[:3] = [0.0, -0.0, np.nan]
    y = K.unary(x, K.SIGMOID)
    pos = np.abs(x) + np.float32(0.5)
    dg, dx, dy, dpos, out = C.Buffer.of(g), C.Buffer.of(x), C.Buffer.of(y), C.Buffer.of(pos), C.Buffer(g.shape)
    L = C.lib()
    C.check(L.vc_hip_relu_backward(dg.ptr, dx.ptr, out.ptr, g.size))
    np.testing.assert_array_equal(out.numpy(), K.binary(g, K.unary(x, K.RELU_GRAD), K.MUL))
    C.check(L.vc_hip_sigmoid_backward(dg.ptr, dy.ptr, out.ptr, g.size))
    np.testing.assert_array_equal(out.numpy(), K.binary(K.binary(g, y, K.MUL), K.binary(np.float32(1), y, K.SUB), K.MUL))
    C.check(L.vc_hip_exp_backward(dg.ptr, dy.ptr, out.ptr, g.size))
    np.testing.assert_array_equal(out.numpy(), K.binary(g, y, K.MUL))
    C.check(L.vc_hip_log_backward(dg.ptr, dpos.ptr, out.ptr, g.size))
    np.testing.assert_array_equal(out.numpy(), K.binary(g, pos, K.DIV))


def test_div_backward_bitexact_with_broadcast():
    rng = np.random.default_rng(6)
    a = rng.standard_normal((37, 45)).astype(np.float32)
    b = rng.uniform(1, 2, size=(45,)).astype(np.float32)
    g = rng.standard_normal((37, 45)).astype(np.float32)
    da, db, dg = C.Buffer.of(a), C.Buffer.of(b), C.Buffer.of(g)
    ga, gb = C.Buffer(g.shape), C.Buffer(g.shape)
    C.check(C.lib().vc_hip_div_backward(dg.ptr, da.ptr, C.sizes(a.shape), C.sizes([45, 1]), 2, db.ptr, C.sizes([45]),
                                        C.sizes([1]), 1, C.sizes(g.shape), 2, ga.ptr, gb.ptr))
    np.testing.assert_array_equal(ga.numpy(), K.binary(g, b, K.DIV))
    expected_gb = K.binary(K.unary(K.binary(g, a, K.MUL), K.NEG), K.binary(b, b, K.MUL), K.DIV)
    np.testing.assert_array_equal(gb.numpy(), expected_gb)


def test_axpy_matches_sgd_bitexact():
    rng = np.random.default_rng(7)
    p = rng.standard_normal(25_001).astype(np.float32)
    g = rng.standard_normal(25_001).astype(np.float32)
    dp, dg = C.Buffer.of(p), C.Buffer.of(g)
    C.check(C.lib().vc_hip_axpy(dp.ptr, dg.ptr, p.size, ctypes.c_float(-0.01)))
    expected = p.copy()
    K.sgd_(expected, g, 0.01)
    np.testing.assert_array_equal(dp.numpy(), expected)


def test_axpy_batch_matches_per_tensor_sgd_bitexact():
    # 21 tensors: more than one launch's list, empty and sub-vector sizes,
    # ragged tails, and two views at a 4-byte offset (the unaligned path).
    rng = np.random.default_rng(11)
    sizes_ = [25_001, 0, 1, 3, 4, 5, 4097, 128, 77, 1 << 16, 9, 2, 6, 31, 64, 1000, 17, 8, 12345, 3, 513]
    params = [rng.standard_normal(s).astype(np.float32) for s in sizes_]
    grads = [rng.standard_normal(s).astype(np.float32) for s in sizes_]
    # Every third entry writes a separate output buffer and leaves its target alone.
    bufs = []
    outputs, targets, sources = [], [], []
    for i, (p, g) in enumerate(zip(params, grads)):
        shift = 1 if i in (4, 17) else 0  # a float into a larger buffer: not 16-byte aligned
        dp = C.Buffer.of(np.concatenate([np.zeros(shift, np.float32), p]))
        dg = C.Buffer.of(np.concatenate([np.zeros(shift, np.float32), g]))
        do = C.Buffer((shift + p.size,)) if i % 3 == 2 else dp
        bufs.append((dp, do, dg, shift))  # every buffer stays alive until the checks
        outputs.append(do.ptr + 4 * shift)
        targets.append(dp.ptr + 4 * shift)
        sources.append(dg.ptr + 4 * shift)
    n = len(sizes_)
    ptrs = ctypes.c_void_p * n
    C.check(C.lib().vc_hip_axpy_batch(ptrs(*outputs), ptrs(*targets), ptrs(*sources), C.sizes(sizes_), n,
                                      ctypes.c_float(-0.05)))
    for (dp, do, _, shift), p, g in zip(bufs, params, grads):
        expected = p.copy()
        K.sgd_(expected, g, 0.05)
        np.testing.assert_array_equal(do.numpy()[shift:], expected)
        if do is not dp:
            np.testing.assert_array_equal(dp.numpy()[shift:], p)
    C.check(C.lib().vc_hip_axpy_batch(None, None, None, None, 0, ctypes.c_float(1.0)))


def reduce_axis_dev(x, axis, op):
    _, outer, length, inner, _, removed = K.split_axis(x.shape, axis)
    dx, dy = C.Buffer.of(x), C.Buffer(removed)
    C.check(C.lib().vc_hip_reduce_axis(dx.ptr, dy.ptr, outer, length, inner, op))
    return dy.numpy()


@pytest.mark.parametrize("shape", [(64, 500, 33), (5, 300, 7), (4096, 4096), (8192, 1000), (3, 4, 5), (1, 3_000_001),
                                   (8, 1024 * 1024), (3001, 2051), (70, 8192), (2049, 2048), (1000, 700), (3001, 301),
                                   (3000, 300), (2000, 512), (2000, 448), (1500, 2044), (2000, 2047), (700, 250),
                                   (1024, 4096), (600, 4100)])
def test_reduce_axis_against_oracle(shape):
    # Column sums of one matrix with at least 8 column chunks (64 columns
    # each with 16-byte loads, 16 with scalar loads) take the one-launch
    # kernel (the last block of each column chunk adds the partials): about
    # 2048 blocks from 32 chunks up, as (4096, 4096) and (2049, 2048) with
    # 16-byte loads, (3001, 2051) with scalar loads and short last segments,
    # (1024, 4096) with 4 segments and (600, 4100) with 2 (segments of at
    # least 256 rows), (70, 8192) with one; about 128 below, as (8192, 1000),
    # (1000, 700) with a short last chunk and 3 short segments and (3001, 301)
    # with scalar loads. (3000, 300)
    # has 5 chunks: partials, then a combine launch. At the boundaries:
    # (2000, 512) has 8 chunks (one launch), (2000, 448) 7 (two launches),
    # (1500, 2044) 32 with a short last one (about 2048 blocks). Rows that
    # are not whole 128-byte lines with a chunk count divisible by 8 give
    # each XCD a contiguous run of chunks: (8192, 1000), (1500, 2044), and
    # with scalar loads (2000, 2047) and (700, 250).
    rng = np.random.default_rng(len(shape) + shape[-1])
    x = rng.standard_normal(shape).astype(np.float32)
    for axis in range(len(shape)):
        got = reduce_axis_dev(x, axis, C.SUM)
        want = K.reduce_axis(x, axis, K.SUM)
        np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-6)
        if x.shape[axis] <= 100_000:
            np.testing.assert_array_equal(reduce_axis_dev(x, axis, C.MAX), K.reduce_axis(x, axis, K.MAX))
            np.testing.assert_array_equal(reduce_axis_dev(x, axis, C.ARGMAX), K.reduce_axis(x, axis, K.ARGMAX))


def test_reduce_axis_nan_and_ties_match_reference_fixture(golden):
    x = golden["reduce_x"]
    for axis in (0, 1, 2):
        np.testing.assert_array_equal(reduce_axis_dev(x, axis, C.MAX), golden[f"reduce_max_{axis}"])
        np.testing.assert_array_equal(reduce_axis_dev(x, axis, C.ARGMAX), golden[f"reduce_argmax_{axis}"])
        np.testing.assert_allclose(reduce_axis_dev(x, axis, C.SUM), golden[f"reduce_sum_{axis}"], rtol=1e-6)
    ties = np.array([[1, 3, 3], [2, 2, 0], [np.nan, 5, 1], [0, np.nan, -1]], dtype=np.float32)
    np.testing.assert_array_equal(reduce_axis_dev(ties, 1, C.ARGMAX), [1, 0, 0, 0])


def test_reductions_are_deterministic():
    x = np.random.default_rng(8).standard_normal((4096, 4096)).astype(np.float32)
    dx, dy = C.Buffer.of(x), C.Buffer((4096,))
    runs = []
    for _ in range(3):
        C.check(C.lib().vc_hip_reduce_axis(dx.ptr, dy.ptr, 1, 4096, 4096, C.SUM))
        runs.append(dy.numpy())
    assert all(np.array_equal(runs[0], r) for r in runs[1:])
    s = C.Buffer((1,))
    sums = set()
    for _ in range(3):
        C.check(C.lib().vc_hip_reduce_sum(dx.ptr, x.size, s.ptr))
        sums.add(float(s.numpy()[0]))
    assert len(sums) == 1
    assert np.isclose(sums.pop(), K.sum_all(x), rtol=1e-6, atol=1e-3)


def test_reduce_sum_edges():
    for n in (0, 1, 3, 1025, 300_001):
        x = np.random.default_rng(n).standard_normal(n).astype(np.float32)
        dx, s = C.Buffer.of(x) if n else C.Buffer((1,)), C.Buffer((1,))
        C.check(C.lib().vc_hip_reduce_sum(dx.ptr, n, s.ptr))
        np.testing.assert_allclose(s.numpy()[0], K.sum_all(x), rtol=1e-6, atol=1e-6)


def test_reduce_sum_one_launch_large_unaligned_and_repeated():
    # 2^25 + 1 floats: 2048 chunks (the most one launch takes) and a partial
    # last chunk; read from an address one float past alignment (scalar
    # loads) and aligned, twice each (the completion counters reset).
    n = (1 << 25) + 1
    x = np.random.default_rng(11).standard_normal(n + 1).astype(np.float32)
    dx, s = C.Buffer.of(x), C.Buffer((1,))
    for shift in (1, 0, 1, 0):
        C.check(C.lib().vc_hip_reduce_sum(dx.ptr + 4 * shift, n, s.ptr))
        np.testing.assert_allclose(s.numpy()[0], K.sum_all(x[shift:shift + n]), rtol=1e-6, atol=1e-4)


def test_scatter_and_transpose_exact():
    rng = np.random.default_rng(9)
    x = rng.standard_normal((6, 40, 9)).astype(np.float32)
    idx = K.reduce_axis(x, 1, K.ARGMAX)
    vals = rng.standard_normal((6, 9)).astype(np.float32)
    dv, di, do = C.Buffer.of(vals), C.Buffer.of(idx), C.Buffer(x.shape)
    C.check(C.lib().vc_hip_scatter_axis(dv.ptr, di.ptr, do.ptr, 6, 40, 9))
    np.testing.assert_array_equal(do.numpy(), K.scatter_axis(vals, idx, x.shape, 1))
    for shape in [(2, 3, 4), (1, 1000, 300), (5, 33, 65)]:
        t = rng.standard_normal(shape).astype(np.float32)
        dt, dout = C.Buffer.of(t), C.Buffer(shape[:-2] + (shape[-1], shape[-2]))
        C.check(C.lib().vc_hip_transpose_last2(dt.ptr, dout.ptr, shape[0], shape[1], shape[2]))
        np.testing.assert_array_equal(dout.numpy(), K.transpose_last2(t))


def xent_dev(logits, targets, with_stats=False):
    rows, classes = logits.shape
    dl, dt = C.Buffer.of(logits), C.Buffer.of(np.asarray(targets).astype(np.int32), dtype=np.int32)
    stats, loss = C.Buffer((rows, 2)), C.Buffer((1,))
    C.check(C.lib().vc_hip_xent_forward(dl.ptr, dt.ptr, rows, classes, stats.ptr, loss.ptr))
    one = C.Buffer.of(np.ones(1, dtype=np.float32))
    grad = C.Buffer(logits.shape)
    C.check(C.lib().vc_hip_xent_backward(dl.ptr, dt.ptr, stats.ptr, one.ptr, rows, classes, grad.ptr))
    if with_stats:
        return loss.numpy()[0], grad.numpy(), stats.numpy()
    return loss.numpy()[0], grad.numpy()


def test_cross_entropy_matches_reference_fixture(golden):
    loss, grad = xent_dev(golden["xent_logits"], golden["xent_targets"])
    np.testing.assert_allclose(loss, golden["xent_loss"], rtol=1e-6)
    np.testing.assert_allclose(grad, golden["xent_grad"], rtol=1e-5, atol=1e-9)


# Two rows per wavefront hold 1, 2, 4 or 8 float4s per lane (up to 128, 256,
# 512, 1024 classes): 3, 37, 2 and 130 (scalar loads), 200 and 512 (vector
# loads, 200 a partial last float4 slot), 257 and 1000; odd row counts leave
# the last wavefront half a pair. One row per wavefront holds 8 or 16 float4s
# per lane (up to 2048, 4096 classes); with the grid at the workgroups resident
# at once (three or two per CU), 4000 x 1500 and 2100 x 4095 (scalar loads)
# give waves more than one row.
@pytest.mark.parametrize("rows,classes", [(512, 1000), (300, 3), (64, 37), (4, 2), (257, 200), (65, 130),
                                          (33, 512), (31, 257), (4000, 1500), (2100, 4095)])
def test_cross_entropy_against_oracle(rows, classes):
    from oracle import autograd as A
    xe = W.xent(rows=rows, classes=classes, seed=rows + classes)
    loss, grad = xent_dev(xe["logits"], xe["targets"])
    t = A.T(xe["logits"], True)
    ref_loss = A.cross_entropy(t, xe["targets"])
    ref_loss.backward()
    np.testing.assert_allclose(loss, ref_loss.data, rtol=1e-6)
    np.testing.assert_allclose(grad, t.grad.data, rtol=1e-5, atol=1e-9)


def test_cross_entropy_backward_with_the_seed_by_value_is_bitexact():
    xe = W.xent(rows=300, classes=1000, seed=9)
    logits, targets = xe["logits"], xe["targets"].astype(np.int32)
    rows, classes = logits.shape
    dl, dt = C.Buffer.of(logits), C.Buffer.of(targets, dtype=np.int32)
    stats, loss = C.Buffer((rows, 2)), C.Buffer((1,))
    C.check(C.lib().vc_hip_xent_forward(dl.ptr, dt.ptr, rows, classes, stats.ptr, loss.ptr))
    for seed in (1.0, 0.37, -2.5):
        by_ptr, by_value = C.Buffer(logits.shape), C.Buffer(logits.shape)
        dseed = C.Buffer.of(np.array([seed], np.float32))
        C.check(C.lib().vc_hip_xent_backward(dl.ptr, dt.ptr, stats.ptr, dseed.ptr, rows, classes, by_ptr.ptr))
        C.check(C.lib().vc_hip_xent_backward_value(dl.ptr, dt.ptr, stats.ptr, ctypes.c_float(seed), rows, classes,
                                                   by_value.ptr))
        np.testing.assert_array_equal(by_value.numpy(), by_ptr.numpy())
    assert C.lib().vc_hip_xent_backward(dl.ptr, dt.ptr, stats.ptr, None, rows, classes, by_ptr.ptr) != 0


def test_cross_entropy_forward_back_to_back_calls():
    # The register-held forward finishes the loss in whichever row block
    # ends last and returns its block counter to zero: calls in a row, with
    # grids of different sizes, each give the oracle's loss.
    from oracle import autograd as A
    for i, (rows, classes) in enumerate([(5000, 1000), (7, 1000), (300, 40), (5000, 1000), (64, 4096), (1, 8)] * 2):
        xe = W.xent(rows=rows, classes=classes, seed=100 + i)
        loss, _ = xent_dev(xe["logits"], xe["targets"])
        want = A.cross_entropy(A.T(xe["logits"]), xe["targets"]).data
        np.testing.assert_allclose(loss, want, rtol=1e-6, err_msg=f"call {i}: {rows}x{classes}")


@pytest.mark.parametrize("classes", [1000, 2000])
def test_cross_entropy_vector_and_scalar_loads_agree(classes):
    # Aligned rows of 1000 classes (two per wavefront) or 2000 (one per
    # wavefront) are loaded into registers with 16-byte loads, the same rows
    # one float off 16-byte alignment with scalar loads into the same places;
    # the backward runs its vector and its scalar kernel. Every path takes its
    # exponentials from one function and adds them in one order, so
    # statistics, loss and gradients agree bit for bit.
    xe = W.xent(rows=2001, classes=classes, seed=17)
    logits, targets = xe["logits"], xe["targets"].astype(np.int32)
    rows, classes = logits.shape
    padded = np.concatenate([np.zeros(1, np.float32), logits.reshape(-1)])
    dl, dpad, dt = C.Buffer.of(logits), C.Buffer.of(padded), C.Buffer.of(targets, dtype=np.int32)
    shifted = dpad.ptr + 4  # 4 bytes past a pool buffer's 256-byte alignment
    out = {}
    for name, ptr in (("registers", dl.ptr), ("streaming", shifted)):
        stats, loss = C.Buffer((rows, 2)), C.Buffer((1,))
        C.check(C.lib().vc_hip_xent_forward(ptr, dt.ptr, rows, classes, stats.ptr, loss.ptr))
        out[name] = (stats, loss.numpy()[0])
    s_reg, s_str = out["registers"][0].numpy(), out["streaming"][0].numpy()
    np.testing.assert_array_equal(s_str, s_reg)
    assert out["streaming"][1] == out["registers"][1]
    grads = []
    for ptr in (dl.ptr, shifted):
        g = C.Buffer((rows, classes))
        C.check(C.lib().vc_hip_xent_backward_value(ptr, dt.ptr, out["registers"][0].ptr, ctypes.c_float(1.0), rows,
                                                   classes, g.ptr))
        grads.append(g.numpy())
    np.testing.assert_array_equal(grads[1], grads[0])


@pytest.mark.parametrize("rows,classes", [(8192, 1000), (17, 1000), (300, 37), (300, 3), (100, 3000), (64, 2048),
                                          (5, 4), (300, 500), (33, 301)])
def test_cross_entropy_backward_with_column_sums(rows, classes):
    """vc_hip_xent_backward_colsum: the gradient is the plain backward's bits
    and the column sums equal the oracle's reduction of that gradient. The
    rows take 1, 2, 4 or 8 float4s per lane (3, 500, 1000, 2048 classes); 37
    and 301 classes (not multiples of 4) load the rows with scalar loads, 3000
    (beyond the register-held rows) takes the plain kernel and a separate
    reduction; 17 and 33 rows leave the last row block short."""
    xe = W.xent(rows=rows, classes=classes, seed=rows + classes)
    logits, targets = xe["logits"], xe["targets"].astype(np.int32)
    dl, dt = C.Buffer.of(logits), C.Buffer.of(targets, dtype=np.int32)
    stats, loss = C.Buffer((rows, 2)), C.Buffer((1,))
    C.check(C.lib().vc_hip_xent_forward(dl.ptr, dt.ptr, rows, classes, stats.ptr, loss.ptr))
    seed = C.Buffer.of(np.array([0.75], np.float32))
    for device_seed in (False, True):
        plain, fused, sums = C.Buffer((rows, classes)), C.Buffer((rows, classes)), C.Buffer((classes,))
        C.check(C.lib().vc_hip_xent_backward_value(dl.ptr, dt.ptr, stats.ptr, ctypes.c_float(0.75), rows, classes,
                                                   plain.ptr))
        C.check(C.lib().vc_hip_xent_backward_colsum(dl.ptr, dt.ptr, stats.ptr, seed.ptr if device_seed else None,
                                                    ctypes.c_float(0.0 if device_seed else 0.75), rows, classes,
                                                    fused.ptr, sums.ptr))
        grad = plain.numpy()
        np.testing.assert_array_equal(fused.numpy(), grad)
        want = K.reduce_axis(grad, 0, K.SUM)
        got = sums.numpy()
        np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-6 * np.abs(grad).sum(0).max())
        assert (got == want).mean() > 0.99


def _special_rows(classes, rng):
    """Rows that exercise the max and non-finite rules, with their targets."""
    base = lambda: -np.abs(rng.standard_normal(classes)).astype(np.float32) - 0.5
    rows, targets = [], []

    def add(row, t):
        rows.append(row)
        targets.append(t)

    r = base(); r[3], r[classes - 2] = -0.0, 0.0; add(r, 1)      # zero maximum, -0.0 first
    r = base(); r[2], r[classes - 1] = 0.0, -0.0; add(r, 0)      # zero maximum, +0.0 first
    add(np.full(classes, -np.inf, np.float32), 1)                # all -inf: m = -inf
    r = base(); r[0] = np.nan; add(r, 1)                         # NaN element 0 is the max
    r = base(); r[classes // 2] = np.nan; add(r, 0)              # NaN elsewhere: skipped by max, NaN term
    r = base(); r[1] = np.inf; add(r, 0)                         # +inf maximum
    r = base(); r[classes - 1] = -np.inf; add(r, 0)              # -inf off the target: NaN term
    r = base(); r[2] = -np.inf; add(r, 2)                        # -inf at the target: term -inf
    r = base(); r[classes - 3] = 30.0; add(r, classes - 3)       # ordinary, target is the maximum
    return np.stack(rows), targets


@pytest.mark.parametrize("classes", [1000, 40, 37, 200, 510, 2000, 4100])
def test_cross_entropy_special_values_match_the_oracle(classes):
    # 1000, 40 and 200 take the register-held kernel with two rows per
    # wavefront (8, 1 and 2 float4s per lane), 37 and 510 (not multiples of 4)
    # the same kernel with scalar loads and a partial last float4 (1 and 4
    # per lane), 2000 the kernel with one row per wavefront, 4100 (too long
    # for registers) the streaming one. Each row alone, so
    # one NaN row does not hide the others; the row maximum must carry the
    # reference's sign of zero.
    from oracle import autograd as A
    rows, targets = _special_rows(classes, np.random.default_rng(classes))
    for i, (row, t) in enumerate(zip(rows, targets)):
        logits = row[None, :]
        loss, grad, stats = xent_dev(logits, [t], with_stats=True)
        ref = A.T(logits, True)
        ref_loss = A.cross_entropy(ref, [t])
        ref_loss.backward()
        np.testing.assert_allclose(loss, ref_loss.data, rtol=1e-6, equal_nan=True, err_msg=f"row {i}")
        np.testing.assert_allclose(grad, ref.grad.data, rtol=1e-5, atol=1e-9, equal_nan=True, err_msg=f"row {i}")
        m = K.reduce_axis(logits, 1, K.MAX)[0]
        if np.isnan(m):
            assert np.isnan(stats[0, 0]), f"row {i}"
        else:
            assert stats[0, 0].view(np.uint32) == np.float32(m).view(np.uint32), f"row {i}: {stats[0, 0]} vs {m}"
    # the finite rows together, many times over: the per-block loss partials
    keep = [0, 1, 8]
    many = np.concatenate([rows[keep]] * 700)
    many_t = [targets[k] for k in keep] * 700
    loss, grad = xent_dev(many, many_t)
    ref = A.T(many, True)
    ref_loss = A.cross_entropy(ref, many_t)
    ref_loss.backward()
    np.testing.assert_allclose(loss, ref_loss.data, rtol=1e-6)
    np.testing.assert_allclose(grad, ref.grad.data, rtol=1e-5, atol=1e-9)


def test_scalar_mirror_publishes_the_value_at_its_point_in_the_stream():
    x = C.Buffer.of(np.array([3.25], np.float32))
    m = ctypes.c_void_p()
    C.check(C.lib().vc_hip_mirror_scalar(x.ptr, ctypes.byref(m)))
    C.check(C.lib().vc_hip_fill(x.ptr, 1, ctypes.c_float(-7.0)))  # enqueued after the mirror's copy
    big = C.Buffer((1 << 22,))
    C.check(C.lib().vc_hip_fill(big.ptr, 1 << 22, ctypes.c_float(1.0)))
    v = ctypes.c_float()
    C.check(C.lib().vc_hip_mirror_read(m, ctypes.byref(v)))
    assert v.value == 3.25
    C.check(C.lib().vc_hip_mirror_read(m, ctypes.byref(v)))  # a second read sees the same value
    assert v.value == 3.25
    C.check(C.lib().vc_hip_mirror_release(m))
    assert x.numpy()[0] == -7.0
    assert C.lib().vc_hip_mirror_scalar(None, ctypes.byref(m)) != 0


@pytest.mark.parametrize("rows,classes", [(257, 1000), (64, 2000), (33, 5000), (5, 3)])
@pytest.mark.parametrize("profiling", [False, True])
def test_published_forward_matches_the_forward_and_its_mirror(rows, classes, profiling):
    # vc_hip_xent_forward_published: the loss and statistics bits of
    # vc_hip_xent_forward, and a mirror holding the loss. Register-held rows
    # (1000, 2000, 3 classes) write the host slot from the forward's kernel
    # unless the profiler holds its dispatch events; streamed rows (5000) and
    # profiled calls publish with a copy after the forward.
    rng = np.random.default_rng(rows + classes)
    x = (rng.standard_normal((rows, classes)) * 2).astype(np.float32)
    t = rng.integers(0, classes, rows).astype(np.int32)
    dx, dt = C.Buffer.of(x), C.Buffer.of(t, dtype=np.int32)
    st1, st2 = C.Buffer((rows, 2)), C.Buffer((rows, 2))
    l1, l2 = C.Buffer((1,)), C.Buffer((1,))
    C.check(C.lib().vc_hip_xent_forward(dx.ptr, dt.ptr, rows, classes, st1.ptr, l1.ptr))
    m = ctypes.c_void_p()
    C.profile(profiling)
    try:
        C.check(C.lib().vc_hip_xent_forward_published(dx.ptr, dt.ptr, rows, classes, st2.ptr, l2.ptr, ctypes.byref(m)))
    finally:
        C.profile(False)
    C.check(C.lib().vc_hip_fill(l2.ptr, 1, ctypes.c_float(-7.0)))  # after the published value
    v = ctypes.c_float()
    C.check(C.lib().vc_hip_mirror_read(m, ctypes.byref(v)))
    C.check(C.lib().vc_hip_mirror_release(m))
    assert np.float32(v.value).tobytes() == l1.numpy()[0].tobytes()
    np.testing.assert_array_equal(st2.numpy(), st1.numpy())
    assert l2.numpy()[0] == -7.0
    assert C.lib().vc_hip_xent_forward_published(dx.ptr, dt.ptr, rows, classes, st2.ptr, l2.ptr, None) != 0


def test_pool_reuses_released_buffers():
    before = C.pool_stats()
    bufs = [C.Buffer((1 << 20,)) for _ in range(4)]
    for b in bufs:
        b.release()
    mid = C.pool_stats()
    bufs = [C.Buffer((1 << 20,)) for _ in range(4)]
    after = C.pool_stats()
    assert after.device_allocations == mid.device_allocations
    assert after.reuses >= mid.reuses + 4
    assert mid.device_allocations <= before.device_allocations + 4
    for b in bufs:
        b.release()


def test_errors_are_reported_not_thrown():
    with pytest.raises(ValueError):
        C.check(C.lib().vc_hip_unary(None, None, 4, 99))
    with pytest.raises(ValueError):
        C.check(C.lib().vc_hip_reduce_axis(None, None, 1, 0, 1, C.MAX))
    assert b"empty axis" in C.lib().vc_hip_last_error()


def test_profiler_times_selected_labels():
    """The event profiler records labelled calls (dispatch timestamps) and can
    be restricted to chosen labels; bench.py relies on both."""
    x = C.Buffer.of(np.ones(1 << 20, np.float32))
    y, s = C.Buffer((1 << 20,)), C.Buffer((1,))
    try:
        C.profile_labels(["reduce_sum"])
        C.profile(True)
        C.profile_reset()
        C.check(C.lib().vc_hip_reduce_sum(x.ptr, 1 << 20, s.ptr))
        C.check(C.lib().vc_hip_unary(x.ptr, y.ptr, 1 << 20, C.NEG))
        got = C.profile_read()
        assert set(got) == {"reduce_sum"}
        assert got["reduce_sum"]["launches"] == 1 and got["reduce_sum"]["ms"] > 0
        assert got["reduce_sum"]["bytes"] == 4.0 * (1 << 20)
        C.profile_labels(None)
        C.profile_reset()
        C.check(C.lib().vc_hip_reduce_sum(x.ptr, 1 << 20, s.ptr))
        C.check(C.lib().vc_hip_unary(x.ptr, y.ptr, 1 << 20, C.NEG))
        got = C.profile_read()
        assert {"reduce_sum", "unary_neg"} <= set(got)
        assert all(v["ms"] > 0 for v in got.values())
    finally:
        C.profile(False)
        C.profile_labels(None)
    assert float(s.numpy()[0]) == float(1 << 20)
