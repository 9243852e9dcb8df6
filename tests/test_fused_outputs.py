"""Results that one kernel leaves for a later op, on the GPU:

- the cross-entropy forward's row argmax (vc_hip_xent_forward_argmax), which
  argmax(1) of the unchanged logits takes instead of reading them again;
- pending column sums (vc_hip_*_colsum_pending): the partial rows a product
  or the cross-entropy backward keeps, finished by vc_hip_colsum_finish or
  inside the SGD update (vc_hip_axpy_batch_colsum) with the same bits;
- the reference's item() contract as an opt-in (hip_strict_item).

Bars: argmax bit-exact against the oracle (the reference's first strict
maximum, NaN-first rule); the finished column sums equal to the bits of the
existing column-sum entry points, and within 1e-6 relative of the oracle's
double reduction.
"""

import ctypes

import numpy as np
import pytest

import vectorcore_amd as vc
from oracle import kernels as K
from vectorcore_amd import cabi as C
from vectorcore_amd import workloads as W

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def device():
    assert C.available(), C.lib().vc_hip_last_error().decode()
    yield
    C.synchronize()


def _rows_with_ties_and_specials(rows, classes, rng):
    x = (rng.standard_normal((rows, classes)) * 2).astype(np.float32)
    r = min(rows, 12)
    if classes >= 4:
        x[0, [1, classes - 1]] = x[0].max() + 1.0                       # a tie: the first wins
        x[1 % rows, :] = -np.inf                                       # all -inf: index 0
        x[2 % rows, 0] = np.nan                                        # NaN element 0 wins
        x[3 % rows, classes // 2] = np.nan                             # interior NaN is skipped
        x[4 % rows, :] = -np.abs(x[4 % rows]) - 1.0
        x[4 % rows, [2, classes - 1]] = [-0.0, 0.0]                    # zero maximum, -0 first
        x[5 % rows, :] = -np.abs(x[5 % rows]) - 1.0
        x[5 % rows, [1, 3]] = [0.0, -0.0]                              # zero maximum, +0 first
        x[6 % rows, classes - 1] = np.inf                              # +inf at the end
        x[7 % rows, :] = 1.5                                           # all equal: index 0
        x[8 % rows, 1:] = np.nan                                       # NaN after a finite first element
    return x[:max(rows, r)]


# Paths of the forward: two rows per wavefront with 1, 2, 4, 8 float4s per
# lane (3, 37 and 130 classes take scalar loads; 200 a partial last float4),
# one row per wavefront with 8 or 16 (2000, 2001, 4096), streamed rows (4101,
# 5000); odd row counts leave half a wavefront pair.
FORWARD_SHAPES = [(300, 3), (64, 37), (257, 200), (65, 130), (33, 512), (512, 1000), (31, 1001), (64, 2000),
                  (17, 2001), (9, 4096), (11, 4101), (10, 5000)]


@pytest.mark.parametrize("rows,classes", FORWARD_SHAPES)
def test_forward_argmax_is_the_reference_argmax(rows, classes):
    rng = np.random.default_rng(rows * 7 + classes)
    x = _rows_with_ties_and_specials(rows, classes, rng)
    rows = x.shape[0]
    t = rng.integers(0, classes, rows).astype(np.int32)
    dx, dt = C.Buffer.of(x), C.Buffer.of(t, dtype=np.int32)
    st1, l1 = C.Buffer((rows, 2)), C.Buffer((1,))
    C.check(C.lib().vc_hip_xent_forward(dx.ptr, dt.ptr, rows, classes, st1.ptr, l1.ptr))
    for published in (False, True):
        st2, l2, am = C.Buffer((rows, 2)), C.Buffer((1,)), C.Buffer((rows,))
        m = ctypes.c_void_p()
        C.check(C.lib().vc_hip_xent_forward_argmax(dx.ptr, dt.ptr, rows, classes, st2.ptr, l2.ptr, am.ptr,
                                                    ctypes.byref(m) if published else None))
        if published:
            v = ctypes.c_float()
            C.check(C.lib().vc_hip_mirror_read(m, ctypes.byref(v)))
            C.check(C.lib().vc_hip_mirror_release(m))
            assert np.float32(v.value).tobytes() == l1.numpy()[0].tobytes()
        # the argmax changes neither the statistics nor the loss
        np.testing.assert_array_equal(st2.numpy().view(np.uint32), st1.numpy().view(np.uint32))
        assert l2.numpy().tobytes() == l1.numpy().tobytes()
        want = K.reduce_axis(x, 1, K.ARGMAX)
        np.testing.assert_array_equal(am.numpy(), want)
        kernel = C.Buffer((rows,))
        C.check(C.lib().vc_hip_reduce_axis(dx.ptr, kernel.ptr, rows, classes, 1, C.ARGMAX))
        np.testing.assert_array_equal(am.numpy(), kernel.numpy())
    assert C.lib().vc_hip_xent_forward_argmax(dx.ptr, dt.ptr, rows, classes, st1.ptr, l1.ptr, None, None) == 1


def test_forward_argmax_of_the_full_size_loss():
    xe = W.xent()
    x, t = xe["logits"], xe["targets"].astype(np.int32)
    rows, classes = x.shape
    dx, dt = C.Buffer.of(x), C.Buffer.of(t, dtype=np.int32)
    st, loss, am = C.Buffer((rows, 2)), C.Buffer((1,)), C.Buffer((rows,))
    C.check(C.lib().vc_hip_xent_forward_argmax(dx.ptr, dt.ptr, rows, classes, st.ptr, loss.ptr, am.ptr, None))
    np.testing.assert_array_equal(am.numpy(), np.argmax(x, axis=1).astype(np.float32))


def _profile(fn, labels=None):
    vc.synchronize()
    vc.hip_profile_reset()
    vc.hip_profile(True, labels=labels)
    try:
        out = fn()
    finally:
        vc.hip_profile(False)
    return out, vc.hip_profile_read()


def test_argmax_after_the_loss_takes_the_forward_indices():
    rng = np.random.default_rng(5)
    x = _rows_with_ties_and_specials(700, 1000, rng)
    x = np.nan_to_num(x, nan=0.25, posinf=50.0, neginf=-50.0)  # finite logits: ties and zero maxima stay
    targets = [int(v) for v in rng.integers(0, 1000, x.shape[0])]
    logits = vc.Tensor(x, requires_grad=True, device="hip")
    loss = vc.cross_entropy(logits, targets)
    loss.backward()
    want = K.reduce_axis(x, 1, K.ARGMAX)
    got, prof = _profile(lambda: logits.detach().argmax(1).numpy())
    np.testing.assert_array_equal(got, want)
    assert "reduce_axis_argmax" not in prof, prof  # no second read of the logits
    # the kept indices are taken once: a second argmax runs the kernel, same values
    got, prof = _profile(lambda: logits.argmax(1, keepdim=True).numpy())
    np.testing.assert_array_equal(got.reshape(-1), want)
    assert prof.get("reduce_axis_argmax", {}).get("launches") == 1, prof


def test_an_in_place_write_between_loss_and_argmax_falls_back_to_the_kernel():
    rng = np.random.default_rng(6)
    x = (rng.standard_normal((300, 1000)) * 2).astype(np.float32)
    targets = [int(v) for v in rng.integers(0, 1000, 300)]
    logits = vc.Tensor(x, requires_grad=True, device="hip")
    loss = vc.cross_entropy(logits, targets)
    loss.backward()
    g = logits.grad.numpy()
    vc.sgd_step([logits], 1e4)  # moves every row's maximum
    updated = x - np.float32(1e4) * g
    got, prof = _profile(lambda: logits.argmax(1).numpy())
    assert prof.get("reduce_axis_argmax", {}).get("launches") == 1, prof
    np.testing.assert_array_equal(got, K.reduce_axis(logits.numpy(), 1, K.ARGMAX))
    assert (got != K.reduce_axis(x, 1, K.ARGMAX)).any()
    np.testing.assert_allclose(logits.numpy(), updated, rtol=1e-6, atol=1e-6)


def test_argmax_of_other_views_of_the_logits_runs_the_kernel():
    x = (np.random.default_rng(7).standard_normal((64, 100)) * 2).astype(np.float32)
    logits = vc.Tensor(x, device="hip")
    vc.cross_entropy(logits, list(range(64)))
    got, prof = _profile(lambda: logits.reshape([128, 50]).argmax(1).numpy())  # another row length
    np.testing.assert_array_equal(got, K.reduce_axis(x.reshape(128, 50), 1, K.ARGMAX))
    assert prof.get("reduce_axis_argmax", {}).get("launches") == 1, prof
    np.testing.assert_array_equal(logits.argmax(1).numpy(), K.reduce_axis(x, 1, K.ARGMAX))


# ---- pending column sums --------------------------------------------------------

def _masked_product(m, k, n, seed):
    rng = np.random.default_rng(seed)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((n, k)).astype(np.float32)  # NT: dY W^T with W stored [n, k]
    mask = rng.standard_normal((m, n)).astype(np.float32)
    return a, b, mask


# 128 x 128 MFMA tiles (72 and 81 of them: a partial last tile of 104 rows,
# a last tile of 6 rows, fewer than one wave's 64), 32 x 32 MFMA tiles (a few
# 128 x 128 tiles' worth: whole, a partial last tile of 8 rows, of 2 rows),
# the FMA kernel (tiny products, and forced; 300 rows leave a partial 16-row
# tile), and a product split along K (no partial rows: the sums are written
# at once).
PENDING_SHAPES = [(1000, 128, 1100, "mfma"), (1030, 64, 1100, "mfma"), (1024, 256, 512, "mfma"),
                  (1000, 128, 300, "mfma"), (130, 64, 257, "mfma"), (300, 3, 64, "mfma"), (37, 16, 70, "mfma"),
                  (700, 96, 200, "simple"), (64, 8192, 256, "mfma")]


@pytest.mark.parametrize("m,k,n,kernel", PENDING_SHAPES)
def test_pending_product_sums_finish_to_the_column_sum_entry_points_bits(m, k, n, kernel):
    a, b, mask = _masked_product(m, k, n, m + k + n)
    da, db, dm = C.Buffer.of(a), C.Buffer.of(b), C.Buffer.of(mask)
    with C.gemm_kernel(kernel):
        c1, s1 = C.Buffer((m, n)), C.Buffer((n,))
        C.check(C.lib().vc_hip_matmul_relu_mask_colsum(da.ptr, db.ptr, c1.ptr, m, k, n, 0, 1, dm.ptr, s1.ptr))
        c2, s2 = C.Buffer((m, n)), C.Buffer.of(np.full(n, 7.0, np.float32))
        h = ctypes.c_void_p()
        C.check(C.lib().vc_hip_matmul_relu_mask_colsum_pending(da.ptr, db.ptr, c2.ptr, m, k, n, 0, 1, dm.ptr, s2.ptr,
                                                               ctypes.byref(h)))
    np.testing.assert_array_equal(c2.numpy(), c1.numpy())
    if k == 8192:  # split along K: no handle, the sums are written
        assert not h.value
        np.testing.assert_array_equal(s2.numpy(), s1.numpy())
    else:
        assert h.value
        assert (s2.numpy() == 7.0).all()  # not written while pending
        cols = ctypes.c_size_t()
        C.check(C.lib().vc_hip_colsum_size(h, ctypes.byref(cols)))
        assert cols.value == n
        for _ in range(2):  # a handle can be finished more than once
            f = C.Buffer((n,))
            C.check(C.lib().vc_hip_colsum_finish(h, f.ptr))
            np.testing.assert_array_equal(f.numpy(), s1.numpy())
        C.check(C.lib().vc_hip_colsum_release(h))
    c = c1.numpy()
    want = K.reduce_axis(c, 0, K.SUM)
    np.testing.assert_allclose(s1.numpy(), want, rtol=1e-6, atol=1e-6 * np.abs(c).sum(0).max())


@pytest.mark.parametrize("m,n", [(200, 128), (1030, 1100)])  # 32 x 32 tiles; 128 x 128 tiles, 6 rows in the last
def test_pending_sums_leave_out_rows_past_the_matrix_even_when_b_is_infinite(m, n):
    # In a last, partial MFMA tile the rows past M hold 0 * B; with an
    # infinite entry of B that is NaN, which must not reach the sums. Here
    # every real row of column 5 is +inf (a positive A entry times the +inf
    # of B, unmasked), so its sum is +inf, and NaN would mean padding rows
    # were added.
    k = 64
    a, b, mask = _masked_product(m, k, n, 3)
    a[:, 7] = np.abs(a[:, 7]) + 0.5
    b[5, 7] = np.inf
    mask[:, 5] = 1.0
    da, db, dm = C.Buffer.of(a), C.Buffer.of(b), C.Buffer.of(mask)
    c, s, h = C.Buffer((m, n)), C.Buffer((n,)), ctypes.c_void_p()
    C.check(C.lib().vc_hip_matmul_relu_mask_colsum_pending(da.ptr, db.ptr, c.ptr, m, k, n, 0, 1, dm.ptr, s.ptr,
                                                           ctypes.byref(h)))
    C.check(C.lib().vc_hip_colsum_finish(h, s.ptr))
    C.check(C.lib().vc_hip_colsum_release(h))
    got, cc = s.numpy(), c.numpy()
    assert np.isposinf(cc[:, 5]).all()
    assert got[5] == np.inf
    assert np.isfinite(np.delete(got, 5)).all()
    np.testing.assert_allclose(got, K.reduce_axis(cc, 0, K.SUM), rtol=1e-6, atol=1e-5)


def test_sgd_with_pending_sums_gives_the_bits_of_finish_then_axpy():
    # A list of plain tensors and pending sums from a product (128 partial
    # rows of 4096 columns, as the train step's db1 and db2) and from the
    # cross-entropy backward (512 partial rows of 1000, as db3), updated in
    # one launch; the same list with the sums finished first and plain
    # vc_hip_axpy_batch gives the same bits. The handles stay usable.
    rng = np.random.default_rng(11)
    handles, sums_ref = [], []
    a, b, mask = _masked_product(8192, 64, 4096, 12)
    da, db, dm = C.Buffer.of(a), C.Buffer.of(b), C.Buffer.of(mask)
    c, s = C.Buffer((8192, 4096)), C.Buffer((4096,))
    h = ctypes.c_void_p()
    C.check(C.lib().vc_hip_matmul_relu_mask_colsum_pending(da.ptr, db.ptr, c.ptr, 8192, 64, 4096, 0, 1, dm.ptr, s.ptr,
                                                           ctypes.byref(h)))
    handles.append(h)
    xe = W.xent(rows=8192, classes=1000, seed=13)
    dl, dt = C.Buffer.of(xe["logits"]), C.Buffer.of(xe["targets"].astype(np.int32), dtype=np.int32)
    st, loss = C.Buffer((8192, 2)), C.Buffer((1,))
    C.check(C.lib().vc_hip_xent_forward(dl.ptr, dt.ptr, 8192, 1000, st.ptr, loss.ptr))
    g, s3, h3 = C.Buffer((8192, 1000)), C.Buffer((1000,)), ctypes.c_void_p()
    C.check(C.lib().vc_hip_xent_backward_colsum_pending(dl.ptr, dt.ptr, st.ptr, None, ctypes.c_float(1.0), 8192, 1000,
                                                        g.ptr, s3.ptr, ctypes.byref(h3)))
    assert h3.value
    handles.append(h3)
    for hh, n in zip(handles, (4096, 1000)):
        f = C.Buffer((n,))
        C.check(C.lib().vc_hip_colsum_finish(hh, f.ptr))
        sums_ref.append(f)
    # entries: plain, pending (4096), plain odd-sized, pending (1000)
    counts = [5000, 4096, 1001, 1000]
    params = [rng.standard_normal(n).astype(np.float32) for n in counts]
    plain_src = [C.Buffer.of(rng.standard_normal(n).astype(np.float32)) for n in (5000, 1001)]
    sources_ref = [plain_src[0], sums_ref[0], plain_src[1], sums_ref[1]]
    alpha = -0.01
    t_ref = [C.Buffer.of(p) for p in params]
    t_new = [C.Buffer.of(p) for p in params]
    P = ctypes.c_void_p * 4
    C.check(C.lib().vc_hip_axpy_batch(P(*[t.ptr for t in t_ref]), P(*[t.ptr for t in t_ref]),
                                      P(*[s.ptr for s in sources_ref]), C.sizes(counts), 4, ctypes.c_float(alpha)))
    pend = P(None, handles[0].value, None, handles[1].value)
    srcs = P(plain_src[0].ptr, None, plain_src[1].ptr, None)
    C.check(C.lib().vc_hip_axpy_batch_colsum(P(*[t.ptr for t in t_new]), P(*[t.ptr for t in t_new]), srcs, pend,
                                             C.sizes(counts), 4, ctypes.c_float(alpha)))
    for r, n in zip(t_ref, t_new):
        np.testing.assert_array_equal(n.numpy(), r.numpy())
    f = C.Buffer((1000,))
    C.check(C.lib().vc_hip_colsum_finish(handles[1], f.ptr))  # still valid after the update
    np.testing.assert_array_equal(f.numpy(), sums_ref[1].numpy())
    # a count that is not the handle's column count is rejected
    bad = C.lib().vc_hip_axpy_batch_colsum(P(t_new[1].ptr), P(t_new[1].ptr), P(None), P(handles[0].value),
                                           C.sizes([4095]),
                                           1, ctypes.c_float(alpha))
    assert bad == 1
    for hh in handles:
        C.check(C.lib().vc_hip_colsum_release(hh))


def _spiral_step(params, sp):
    xs = vc.Tensor(sp["x"], device="hip")
    loss = vc.cross_entropy((xs @ params[0] + params[1]).relu() @ params[2] + params[3], sp["targets"])
    loss.backward()
    return loss


def test_spiral_step_finishes_bias_sums_inside_the_update():
    # The spiral step's bias gradients stay pending (db1 from the FMA kernel's
    # epilogue, db2 from the cross-entropy backward) until sgd_step, which
    # adds them in its own launch: eight launches per step, none of them a
    # column-sum pass. Reading the gradients first (which finishes them) and
    # then stepping gives the same parameters bit for bit.
    sp = W.spiral()

    def fresh():
        ps = []
        for w, b in zip(sp["weights"], sp["biases"]):
            ps += [vc.Tensor(w, requires_grad=True, device="hip"), vc.Tensor(b, requires_grad=True, device="hip")]
        return ps

    a, b = fresh(), fresh()
    _spiral_step(a, sp)
    vc.synchronize()
    vc.hip_profile_reset()
    vc.hip_profile(True)
    try:
        _spiral_step(b, sp)
        vc.sgd_step(b, sp["lr"])
        vc.synchronize()
    finally:
        vc.hip_profile(False)
    prof = vc.hip_profile_read()
    launches = sum(v["launches"] for v in prof.values())
    if vc.hip_defer_products():  # eager forward products add their bias-add and ReLU launches
        assert launches <= 8, prof
    assert "column_sum_combine" not in prof and "reduce_axis_sum" not in prof, prof
    read = [p.grad.numpy() for p in a]  # finishes the pending sums
    vc.sgd_step(a, sp["lr"])
    for p, q in zip(a, b):
        np.testing.assert_array_equal(p.numpy(), q.numpy())
    # against the oracle's float64-free restatement of the reference
    from oracle import autograd as A
    ref = A.Mlp(sp["weights"], sp["biases"])
    A.cross_entropy(ref.logits(A.T(sp["x"])), sp["targets"]).backward()
    for g, r in zip(read, ref.params()):
        np.testing.assert_allclose(g, r.grad.data, rtol=1e-4, atol=1e-6)


def test_train_step_bias_sums_are_deterministic_and_match_the_unfused_path():
    # A three-layer step: the bias sums stay pending into sgd_step. Two runs
    # give the same parameters bit for bit, and so does a run that reads the
    # gradients first; retained activations turn the producers' sums off
    # (separate reductions), which agree to 1e-6.
    m = W.mlp(batch=1024, dims=(256, 512, 384, 100), seed=21)

    def run(read_grads_first, retain=False):
        ps = []
        for w, b in zip(m["weights"], m["biases"]):
            ps += [vc.Tensor(w, requires_grad=True, device="hip"), vc.Tensor(b, requires_grad=True, device="hip")]
        h = vc.Tensor(m["x"], device="hip")
        for i in range(3):
            h = h @ ps[2 * i] + ps[2 * i + 1]
            if retain:
                h.retain_grad()
            if i < 2:
                h = h.relu()
        vc.cross_entropy(h, m["targets"]).backward()
        grads = [p.grad.numpy() for p in ps] if read_grads_first else None
        vc.sgd_step(ps, m["lr"])
        return [p.numpy() for p in ps], grads

    first, _ = run(False)
    second, _ = run(False)
    for p, q in zip(first, second):
        np.testing.assert_array_equal(p, q)
    read, grads = run(True)
    for p, q in zip(first, read):
        np.testing.assert_array_equal(p, q)
    _, plain = run(True, retain=True)
    for k in (1, 3, 5):
        np.testing.assert_allclose(grads[k], plain[k], rtol=1e-6, atol=1e-6 * np.abs(plain[k]).max())
    for k in (0, 2, 4):
        np.testing.assert_array_equal(grads[k], plain[k])


# ---- the reference's item() contract as an opt-in --------------------------------

def test_strict_item_returns_with_the_stream_idle():
    m = W.mlp(batch=4096, dims=(1024, 2048, 1000), seed=4)
    ps = []
    for w, b in zip(m["weights"], m["biases"]):
        ps += [vc.Tensor(w, requires_grad=True, device="hip"), vc.Tensor(b, requires_grad=True, device="hip")]
    x = vc.Tensor(m["x"], device="hip")
    previous = vc.hip_strict_item(True)
    try:
        assert vc.hip_strict_item() is True
        for _ in range(2):
            loss = vc.cross_entropy((x @ ps[0] + ps[1]).relu() @ ps[2] + ps[3], m["targets"])
            loss.backward()
            vc.sgd_step(ps, m["lr"])  # enqueued after the loss
            value = loss.item()
            assert C.stream_idle(), "item() returned before the queued work finished"
            assert np.isfinite(value)
            vc.zero_grad(ps)
    finally:
        vc.hip_strict_item(previous)
    assert vc.hip_strict_item() is previous
