"""Semantics of the tensor/autograd runtime on every device.

Restates the behaviour the reference's own suites check
(tests/cpp/test_vectorcore.cpp, tests/python/test_vectorcore.py,
test_autograd_correctness.py, test_classifier_ops.py,
test_performance_paths.py): known-answer vectors, finite-difference
gradients, version-counter rejection, leaf-only .grad, broadcasting,
asynchronous device ordering. Each test runs on "cpu" and on "hip"; the hip
cases need the GPU and carry the gpu marker.
"""

import zlib

import numpy as np
import pytest

import vectorcore_amd as vc

DEVICES = [pytest.param("cpu", id="cpu"), pytest.param("hip", id="hip", marks=pytest.mark.gpu)]
hip_only = pytest.mark.gpu


@pytest.fixture(params=DEVICES)
def device(request):
    if request.param == "hip":
        assert vc.hip_available(), "the hip device must be available on a GPU run"
    return request.param


GEMM_DEVICES = DEVICES + [pytest.param("hip-simple", id="hip-simple", marks=pytest.mark.gpu)]


@pytest.fixture(params=GEMM_DEVICES)
def gemm_device(request):
    """A device for matmul, gradcheck and MLP tests: cpu, hip with the MFMA
    GEMM, and hip with the portable FMA GEMM selected (the reference re-runs
    these tests with its portable kernel forced,
    tests/python/test_performance_paths.py:89-103)."""
    if request.param == "cpu":
        yield "cpu"
        return
    assert vc.hip_available(), "the hip device must be available on a GPU run"
    kernel = "simple" if request.param == "hip-simple" else "mfma"
    previous = vc.hip_set_gemm_kernel(kernel)
    try:
        assert vc.hip_gemm_kernel() == kernel
        yield "hip"
    finally:
        vc.hip_set_gemm_kernel(previous)


def npy(t):
    return t.to("cpu").numpy()


def close(t, expected, rtol=1e-5, atol=1e-5):
    np.testing.assert_allclose(npy(t), np.asarray(expected, dtype=np.float32).reshape(t.shape), rtol=rtol, atol=atol)


def T(values, device, requires_grad=False):
    return vc.Tensor(np.asarray(values, dtype=np.float32), requires_grad=requires_grad, device=device)


# --- tensors and views ---------------------------------------------------------


def test_metadata_indexing_and_views():
    v = vc.Tensor([[1, 2, 3], [4, 5, 6]], requires_grad=True)
    assert v.shape == [2, 3] and v.strides == [3, 1] and v.ndim == 2 and v.numel == 6
    assert v.at([1, 2]) == 6 and "requires_grad=true" in repr(v)
    w = vc.Tensor([1, 2, 3, 4])
    flat = w.reshape([2, 2]).flatten()
    assert flat.shape == [4]
    with pytest.raises(IndexError):
        v.at([3, 0])
    with pytest.raises(ValueError):
        w.reshape([3, 2])


def test_version_counter_shared_by_views_and_bumped_by_sgd(device):
    w = T([1.0, 2.0], device, True)
    start = w._version
    view = w.reshape([2, 1])
    _ = (w * 1.0).sum()
    assert w._version == start
    (w * 1.0).sum().backward()
    vc.sgd_step([w], 0.1)
    assert w._version == start + 1 and view._version == w._version


def test_device_transfer_round_trip(device):
    x = np.random.default_rng(0).standard_normal((5, 7)).astype(np.float32)
    t = vc.Tensor(x).to(device)
    assert t.device == device
    np.testing.assert_array_equal(npy(t), x)
    np.testing.assert_array_equal(npy(t.to("cpu").to(device)), x)


# --- forward known answers -------------------------------------------------------


def test_elementwise_and_scalars(device):
    a, b = T([[1, 2], [3, 4]], device), T([[4, 3], [2, 1]], device)
    close(a + b, [5, 5, 5, 5])
    close(a - b, [-3, -1, 1, 3])
    close(a * b, [4, 6, 6, 4])
    close(a / b, [0.25, 2 / 3, 1.5, 4])
    close(-a, [-1, -2, -3, -4])
    close(2.0 + a * 2.0, [4, 6, 8, 10])
    close(3.0 / a - (1.0 - a), [3 - 0, 1.5 + 1, 1 + 2, 0.75 + 3])


def test_broadcasting(device):
    m = T([[1, 2, 3], [4, 5, 6]], device)
    close(m + T([10, 20, 30], device), [11, 22, 33, 14, 25, 36])
    close(m + T([[10, 20, 30]], device), [11, 22, 33, 14, 25, 36])
    close(m + vc.Tensor(2.0, device=device), [3, 4, 5, 6, 7, 8])
    high = T(np.ones((2, 3, 4)), device)
    close(high * T([[1, 2, 3, 4]], device), np.tile([1, 2, 3, 4], 6))
    with pytest.raises(ValueError):
        m + T(np.ones((2, 2)), device)


def test_matmul_transpose_and_batches(gemm_device):
    a, b = T([[1, 2, 3], [4, 5, 6]], gemm_device), T([[7, 8], [9, 10], [11, 12]], gemm_device)
    close(a @ b, [58, 64, 139, 154])
    close(a.transpose(), [1, 4, 2, 5, 3, 6])
    close(T(np.arange(1, 9).reshape(2, 2, 2), gemm_device).transpose(), [1, 3, 2, 4, 5, 7, 6, 8])
    with pytest.raises(ValueError):
        a @ T(np.ones((4, 2)), gemm_device)
    with pytest.raises(ValueError):
        T(np.ones((2, 2, 3)), gemm_device) @ T(np.ones((3, 3, 1)), gemm_device)


def test_reductions_activations_and_softmax(device):
    v = T([-2, -1, 0, 1, 2], device)
    assert v.sum().item() == 0 and v.mean().item() == 0
    close(v.relu(), [0, 0, 0, 1, 2])
    assert abs(npy(v.sigmoid())[2] - 0.5) < 1e-6
    x = T([[1, 5, 3], [4, 2, 6]], device)
    close(x.sum(0), [5, 7, 9])
    close(x.sum(-1, keepdim=True), [9, 12])
    assert x.sum(1, keepdim=True).shape == [2, 1]
    close(x.mean(1), [3, 4])
    close(x.max(1), [5, 6])
    close(x.max(0), [4, 5, 6])
    close(x.argmax(1), [1, 2])
    assert x.max().item() == 6
    close(T([0, 1], device).exp(), [1, np.e])
    close(T([1, np.exp(2)], device).log(), [0, 2])
    close(x.softmax(1).sum(1), [1, 1], atol=1e-6)
    close(T([[1, 3, 3], [2, 2, 0]], device).argmax(1), [1, 0])
    assert vc.Tensor(np.zeros(0, np.float32), device=device).sum().item() == 0
    for bad in (lambda: x.sum(2), lambda: x.max(-3), lambda: vc.Tensor(1.0, device=device).sum(0),
                lambda: vc.Tensor(np.zeros(0, np.float32), device=device).mean()):
        with pytest.raises((ValueError, IndexError, RuntimeError)):
            bad()


@pytest.mark.parametrize("axis", [0, 1, 2, -1, -3])
@pytest.mark.parametrize("keepdim", [False, True])
def test_axis_reductions_match_numpy(device, axis, keepdim):
    x = np.random.default_rng(2).normal(size=(3, 4, 5)).astype(np.float32)
    t = vc.Tensor(x, device=device)
    close(t.sum(axis, keepdim), x.sum(axis=axis, keepdims=keepdim), rtol=1e-4, atol=1e-5)
    close(t.mean(axis, keepdim), x.mean(axis=axis, keepdims=keepdim), rtol=1e-4, atol=1e-5)
    close(t.max(axis, keepdim), x.max(axis=axis, keepdims=keepdim))
    close(t.argmax(axis, keepdim), x.argmax(axis=axis).reshape(x.max(axis=axis, keepdims=keepdim).shape))


def test_reductions_without_axis(device):
    x = np.random.default_rng(3).normal(size=(3, 4)).astype(np.float32)
    t = vc.Tensor(x, device=device)
    assert np.isclose(t.max().item(), x.max()) and t.argmax().item() == x.argmax()
    assert t.sum(keepdim=True).shape == [1, 1] and t.max(keepdim=True).shape == [1, 1]


def test_softmax_stable_for_huge_logits(device):
    t = T([[1000.0, 1001.0, 1002.0], [-1000.0, 0.0, 1000.0]], device, True)
    p = npy(t.softmax(-1))
    assert np.all(np.isfinite(p))
    np.testing.assert_allclose(p[0], np.exp([0, 1, 2]) / np.exp([0, 1, 2]).sum(), rtol=1e-5)
    vc.cross_entropy(t, [2, 0]).backward()
    assert np.all(np.isfinite(npy(t.grad)))


# --- autograd semantics ------------------------------------------------------------


def test_autograd_known_answers(gemm_device):
    x = T([1, 2, 3], gemm_device, True)
    ((x * x) + x).sum().backward()
    close(x.grad, [3, 5, 7])
    x.zero_grad()
    assert x.grad is None
    x, b = T([[1, 2, 3], [4, 5, 6]], gemm_device, True), T([0.1, 0.2, 0.3], gemm_device, True)
    (x + b).sum().backward()
    close(x.grad, np.ones(6))
    close(b.grad, [2, 2, 2])
    a, w = T([[1, 2, 3], [4, 5, 6]], gemm_device, True), T([[1, 2], [3, 4], [5, 6]], gemm_device, True)
    a.matmul(w).sum().backward()
    close(a.grad, [3, 7, 11, 3, 7, 11])
    close(w.grad, [5, 5, 7, 7, 9, 9])
    gx, gb = T([[-1, 2, 3], [-4, 5, 6]], gemm_device, True), T([0.5, 1.0, -2.0], gemm_device, True)
    (gx + gb).relu().sum().backward()
    close(gx.grad, [0, 1, 1, 0, 1, 1])
    close(gb.grad, [0, 2, 2])


def test_gradient_accumulation_and_retain_grad(device):
    x = T([1, 2], device, True)
    (x * 3.0).sum().backward()
    (x * 4.0).sum().backward()
    close(x.grad, [7, 7])
    a = T([1, 2], device, True)
    hidden, kept = a * 2.0, a * 3.0
    kept.retain_grad()
    assert kept.retains_grad
    ((hidden * hidden).sum() + kept.sum()).backward()
    assert a.is_leaf and not hidden.is_leaf and hidden.grad is None
    close(kept.grad, [1, 1])
    close(a.grad, [11, 19])
    with pytest.raises(RuntimeError):
        T([1.0], device).retain_grad()


def test_batched_and_broadcast_matmul_grads(gemm_device):
    a, w = T([[[1, 2]], [[3, 4]]], gemm_device, True), T([[1, 0], [0, 2]], gemm_device, True)
    y = a.matmul(w)
    assert y.shape == [2, 1, 2]
    close(y, [1, 4, 3, 8])
    y.sum().backward()
    close(w.grad, [4, 4, 6, 6])
    close(a.grad, [1, 2, 1, 2])


def test_cross_entropy_value_gradient_and_errors(device):
    logits = T(np.zeros((2, 2)), device, True)
    loss = vc.cross_entropy(logits, [0, 1])
    assert abs(loss.item() - np.log(2)) < 1e-6
    loss.backward()
    close(logits.grad, [-0.25, 0.25, 0.25, -0.25])
    with pytest.raises(ValueError):
        vc.cross_entropy(logits, [0])
    with pytest.raises(IndexError):
        vc.cross_entropy(logits, [0, 2])
    with pytest.raises(ValueError):
        vc.cross_entropy(T([1.0, 2.0], device), [0])
    assert np.isclose(vc.cross_entropy(T(np.zeros((3, 2)), device), np.array([0, 1, 1])).item(), np.log(2))


def test_cross_entropy_with_changing_targets(device):
    """The device keeps the last targets; a new vector replaces them."""
    rng = np.random.default_rng(9)
    logits = (rng.normal(size=(40, 7)) * 2).astype(np.float32)
    a, b = rng.integers(0, 7, 40), rng.integers(0, 7, 40)
    t = vc.Tensor(logits, device=device)
    got = [vc.cross_entropy(t, tg).item() for tg in (a, b, a, a)]
    cpu = vc.Tensor(logits)
    want = [vc.cross_entropy(cpu, tg).item() for tg in (a, b, a, a)]
    np.testing.assert_allclose(got, want, rtol=1e-6)
    assert got[0] == got[2] == got[3] and got[0] != got[1]


def test_cross_entropy_matches_torch(device):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(6)
    logits = (rng.normal(size=(6, 4)) * 2).astype(np.float32)
    targets = [0, 3, 1, 1, 2, 0]
    t = vc.Tensor(logits, requires_grad=True, device=device)
    loss = vc.cross_entropy(t, targets)
    loss.backward()
    tt = torch.tensor(logits, requires_grad=True)
    ref = torch.nn.functional.cross_entropy(tt, torch.tensor(targets))
    ref.backward()
    assert np.isclose(loss.item(), ref.item(), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(npy(t.grad), tt.grad.numpy(), rtol=1e-4, atol=1e-6)


def test_max_gradient_goes_to_first_of_ties(device):
    t = T([[1.0, 3.0, 3.0]], device, True)
    t.max(1).sum().backward()
    close(t.grad, [[0, 1, 0]])


def test_relu_kink_gives_finite_gradient(device):
    x = T([0.0, -0.0, 1.0], device, True)
    x.relu().sum().backward()
    assert np.all(np.isfinite(npy(x.grad)))


def test_in_place_updates_between_forward_and_backward_are_rejected(device):
    w, x = T([2.0], device, True), T([3.0], device, True)
    loss = (w * x).sum()
    (w * 1.0).sum().backward()
    vc.sgd_step([w], 1.0)
    with pytest.raises(RuntimeError, match="modified in place"):
        loss.backward()
    w2 = T([[0.5, -1.0], [2.0, 1.5]], device, True)
    loss = (T([[1.0, 2.0]], device, True) @ w2).sum()
    flat = w2.flatten().detach()
    flat.requires_grad = True
    (flat * 1.0).sum().backward()
    vc.sgd_step([flat], 1.0)  # shares storage with w2
    with pytest.raises(RuntimeError, match="modified in place"):
        loss.backward()
    x = T([0.5, -0.5], device, True)
    y = x.sigmoid()
    loss = y.sum()
    ys = y.detach()
    ys.requires_grad = True
    (ys * 1.0).sum().backward()
    vc.sgd_step([ys], 1.0)  # rewrites sigmoid's saved output
    with pytest.raises(RuntimeError, match="modified in place"):
        loss.backward()


def test_mutation_after_backward_is_allowed_and_training_converges(device):
    w = T([2.0], device, True)
    (w * w).sum().backward()
    vc.sgd_step([w], 0.1)
    assert np.isclose(w.item(), 2.0 - 0.1 * 4.0)
    w = T([[0.0]], device, True)
    x, y = T([[1.0], [2.0], [3.0]], device), T([[2.0], [4.0], [6.0]], device)
    for _ in range(200):
        vc.mse_loss(x @ w, y).backward()
        vc.sgd_step([w], 0.05)
        vc.zero_grad([w])
    assert abs(w.item() - 2.0) < 1e-3


# --- ReLU rule folded into the product that feeds it -----------------------------------
# On hip the engine lets a matrix product apply the mask of the ReLU whose
# output it alone consumes (and which keeps no gradient), in the same kernel.


def _relu_net(device, retain=False, reuse=False, seed=7):
    rng = np.random.default_rng(seed)
    x = T(rng.standard_normal((64, 48)), device)
    w1 = T(rng.standard_normal((48, 96)) * 0.2, device, True)
    b1 = T(rng.standard_normal(96) * 0.1, device, True)
    w2 = T(rng.standard_normal((96, 40)) * 0.2, device, True)
    h = (x @ w1 + b1).relu()
    if retain:
        h.retain_grad()
    y = h @ w2
    if reuse:  # h feeds two products
        y = y + h @ (w2 * 0.5)
    (y * y).sum().backward()
    return h, [w1, b1, w2]


def test_relu_fold_gives_the_unfolded_bits(gemm_device):
    _, folded = _relu_net(gemm_device)
    h, plain = _relu_net(gemm_device, retain=True)  # a kept gradient turns the fold off
    for p, q in zip(folded, plain):
        np.testing.assert_array_equal(npy(p.grad), npy(q.grad))
    _, cpu = _relu_net("cpu")
    for p, q in zip(folded, cpu):
        np.testing.assert_allclose(npy(p.grad), npy(q.grad), rtol=1e-4, atol=1e-4)
    # the kept gradient is the one before the mask: dense where h == 0 too
    assert (npy(h.grad) != 0).sum() > (npy(h) > 0).sum()


@hip_only
def test_bias_gradients_come_from_the_producing_kernels():
    # In cross_entropy(relu(x @ W1 + b1) @ W2 + b2) the product giving
    # dz1 = (dy W2^T) * [z1 > 0] also leaves dz1's column sums, and the
    # cross-entropy backward leaves those of dlogits; b1's and b2's add rules
    # take them instead of reducing dz1 and dlogits again. The values equal
    # the unfused path's (retained gradients turn both off) and the cpu
    # device's.
    rng = np.random.default_rng(41)
    xs = rng.standard_normal((1000, 200)).astype(np.float32)
    w1s = (rng.standard_normal((200, 300)) * 0.1).astype(np.float32)
    b1s = (rng.standard_normal(300) * 0.1).astype(np.float32)
    w2s = (rng.standard_normal((300, 52)) * 0.1).astype(np.float32)
    b2s = (rng.standard_normal(52) * 0.1).astype(np.float32)

    def grads(device, retain=False, profile=False):
        x = T(xs, device)
        w1, b1, w2, b2 = (T(v, device, True) for v in (w1s, b1s, w2s, b2s))
        h = (x @ w1 + b1).relu()
        logits = h @ w2 + b2
        if retain:
            h.retain_grad()
            logits.retain_grad()
        if profile:
            vc.synchronize()
            vc.hip_profile_reset()
            vc.hip_profile(True, labels=["column_sum_combine", "reduce_axis_sum"])
        vc.cross_entropy(logits, [i % 52 for i in range(1000)]).backward()
        out = [npy(p.grad) for p in (w1, b1, w2, b2)]
        if profile:
            vc.hip_profile(False)
            return out, vc.hip_profile_read()
        return out

    fused, prof = grads("hip", profile=True)
    assert prof.get("column_sum_combine", {}).get("launches", 0) == 2, prof
    assert "reduce_axis_sum" not in prof, prof  # no separate reduction of dz1 or dlogits
    plain = grads("hip", retain=True)
    for k in (1, 3):
        np.testing.assert_allclose(fused[k], plain[k], rtol=1e-6, atol=1e-9)
        assert (fused[k] == plain[k]).mean() > 0.99
    for k in (0, 2):
        np.testing.assert_array_equal(fused[k], plain[k])
    for f, c in zip(fused, grads("cpu")):
        np.testing.assert_allclose(f, c, rtol=1e-4, atol=1e-6)


def test_relu_fold_with_a_shared_activation(device):
    _, got = _relu_net(device, reuse=True)
    _, cpu = _relu_net("cpu", reuse=True)
    for p, q in zip(got, cpu):
        np.testing.assert_allclose(npy(p.grad), npy(q.grad), rtol=1e-4, atol=1e-4)


def test_relu_fold_keeps_the_version_check(device):
    w = T(np.linspace(-1, 1, 12).reshape(3, 4), device, True)
    w2 = T(np.ones((4, 2)), device, True)
    loss = (w.relu() @ w2).sum()
    ws = w.detach()
    ws.requires_grad = True
    (ws * 1.0).sum().backward()
    vc.sgd_step([ws], 1.0)  # rewrites the ReLU's saved input
    with pytest.raises(RuntimeError, match="modified in place"):
        loss.backward()


# --- deferred forward products (hip) --------------------------------------------------
# A 2-D product on hip is computed when its storage is first read, so that a
# row-bias add and a ReLU applied to it run in the product's epilogue. Every
# observable value must be the bits of eager execution.


def _eager_then_deferred(fn):
    previous = vc.hip_defer_products(False)
    try:
        eager = fn()
    finally:
        vc.hip_defer_products(previous)
    vc.hip_defer_products(True)
    try:
        return eager, fn()
    finally:
        vc.hip_defer_products(previous)


def _assert_same_bits(eager, deferred):
    assert len(eager) == len(deferred)
    for i, (e, d) in enumerate(zip(eager, deferred)):
        np.testing.assert_array_equal(np.asarray(d), np.asarray(e), err_msg=f"value {i}")


@hip_only
def test_deferred_layers_give_the_eager_bits():
    rng = np.random.default_rng(5)
    xs = rng.standard_normal((300, 70)).astype(np.float32)
    ws = [(rng.standard_normal((70, 130)) * 0.2).astype(np.float32),
          (rng.standard_normal((130, 33)) * 0.2).astype(np.float32)]
    bs = [(rng.standard_normal(130) * 0.1).astype(np.float32), (rng.standard_normal((1, 33)) * 0.1).astype(np.float32)]
    targets = [i % 33 for i in range(300)]

    def run():
        x = vc.Tensor(xs, device="hip")
        w1, w2 = (vc.Tensor(w, requires_grad=True, device="hip") for w in ws)
        b1, b2 = (vc.Tensor(b, requires_grad=True, device="hip") for b in bs)
        pre = x @ w1 + b1
        h = pre.relu()
        logits = b2 + h @ w2  # the bias as the left operand
        loss = vc.cross_entropy(logits, targets)
        loss.backward()
        out = [loss.item()] + [npy(p.grad) for p in (w1, b1, w2, b2)]
        vc.sgd_step([w1, b1, w2, b2], 0.1)
        # read after the update: the values of the forward pass
        out += [npy(pre), npy(h), npy(logits)] + [npy(p) for p in (w1, b1, w2, b2)]
        return out

    _assert_same_bits(*_eager_then_deferred(run))


@hip_only
def test_deferred_product_read_after_its_operands_change():
    rng = np.random.default_rng(6)
    xs = rng.standard_normal((40, 24)).astype(np.float32)
    w0 = rng.standard_normal((24, 36)).astype(np.float32)
    b0 = rng.standard_normal(36).astype(np.float32)

    def run():
        x = vc.Tensor(xs, device="hip")
        w = vc.Tensor(w0, requires_grad=True, device="hip")
        b = vc.Tensor(b0, requires_grad=True, device="hip")
        p1 = x @ w
        q1 = (p1 + b).relu()
        ((w * 1.0).sum() + (b * 1.0).sum()).backward()
        vc.sgd_step([w, b], 0.5)  # w -= 0.5, b -= 0.5
        p2 = x @ w
        q2 = p2 + b
        vc.sgd_step([w, b], 0.5)  # a second update while p2 and q2 are still pending
        p3 = (x @ w).relu()
        return [npy(q1), npy(p1), npy(q2), npy(p2), npy(p3), npy(w), npy(b)]

    eager, deferred = _eager_then_deferred(run)
    _assert_same_bits(eager, deferred)
    tol = dict(rtol=1e-4, atol=1e-4 * np.sqrt(24))
    np.testing.assert_allclose(deferred[1], xs.astype(np.float64) @ w0, **tol)
    np.testing.assert_allclose(deferred[0], np.maximum(xs.astype(np.float64) @ w0 + b0, 0), **tol)
    np.testing.assert_allclose(deferred[2], xs.astype(np.float64) @ (w0 - 0.5) + (b0 - 0.5), **tol)
    np.testing.assert_allclose(deferred[4], np.maximum(xs.astype(np.float64) @ (w0 - 1.0), 0), **tol)


@hip_only
def test_deferred_product_shared_reshaped_and_as_a_bias():
    rng = np.random.default_rng(8)
    xs, ws = rng.standard_normal((17, 9)).astype(np.float32), rng.standard_normal((9, 21)).astype(np.float32)
    us, vs = rng.standard_normal((1, 5)).astype(np.float32), rng.standard_normal((5, 21)).astype(np.float32)

    def run():
        x, w = vc.Tensor(xs, device="hip"), vc.Tensor(ws, requires_grad=True, device="hip")
        u, v = vc.Tensor(us, device="hip"), vc.Tensor(vs, requires_grad=True, device="hip")
        h = x @ w
        bias = u @ v  # [1, 21], itself a deferred product
        fused = (h + bias).relu()
        doubled = h * 2.0  # h is also read directly
        flat = (x @ w).reshape([17 * 21]).relu()  # elementwise, so the ReLU of a reshaped product still fuses
        (fused.sum() + doubled.sum() + flat.sum()).backward()
        return [npy(fused), npy(doubled), npy(flat), npy(w.grad), npy(v.grad)]

    _assert_same_bits(*_eager_then_deferred(run))


@hip_only
def test_partial_in_place_update_of_a_deferred_operand():
    # The device interface's axpy_inplace may update a range of a storage. A
    # product still deferred on that storage keeps the old values, and the
    # storage keeps the elements outside the range.
    rng = np.random.default_rng(12)
    xs, ws = rng.standard_normal((5, 6)).astype(np.float32), rng.standard_normal((6, 7)).astype(np.float32)
    gs = rng.standard_normal(42).astype(np.float32)

    def run():
        x, w, g = vc.Tensor(xs, device="hip"), vc.Tensor(ws, device="hip"), vc.Tensor(gs, device="hip")
        p = x @ w
        vc._vectorcore._axpy_inplace(w, 10, g, 3, 20, -0.5)  # w.flat[10:30] -= 0.5 * g[3:23]
        return [npy(p), npy(w)]

    eager, deferred = _eager_then_deferred(run)
    _assert_same_bits(eager, deferred)
    updated = ws.reshape(-1)[10:30] - np.float32(0.5) * gs[3:23]
    np.testing.assert_array_equal(deferred[1].reshape(-1)[:10], ws.reshape(-1)[:10])
    np.testing.assert_array_equal(deferred[1].reshape(-1)[30:], ws.reshape(-1)[30:])
    np.testing.assert_allclose(deferred[1].reshape(-1)[10:30], updated, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(deferred[0], xs.astype(np.float64) @ ws, rtol=1e-4, atol=1e-4 * np.sqrt(6))


@hip_only
def test_sgd_with_a_gradient_aliasing_its_parameter_and_a_pending_product():
    # w.backward(w) stores w itself as w.grad (the same storage). A product
    # recorded on w is still pending when sgd_step runs, so the update moves
    # w to a fresh buffer; it must read the gradient from w's current
    # contents, giving w - lr * w as the reference's host loop does.
    rng = np.random.default_rng(21)
    xs, w0 = rng.standard_normal((33, 20)).astype(np.float32), rng.standard_normal((20, 18)).astype(np.float32)

    def run():
        x = vc.Tensor(xs, device="hip")
        w = vc.Tensor(w0, requires_grad=True, device="hip")
        p = x @ w
        w.backward(w)
        vc.sgd_step([w], 0.25)
        return [npy(p), npy(w)]

    eager, deferred = _eager_then_deferred(run)
    _assert_same_bits(eager, deferred)
    np.testing.assert_array_equal(deferred[1], w0 - np.float32(0.25) * w0)
    np.testing.assert_allclose(deferred[0], xs.astype(np.float64) @ w0, rtol=1e-4, atol=1e-4 * np.sqrt(20))


@hip_only
def test_long_chain_of_deferred_products():
    # 3000 products, each of the one before, none read until the end: the
    # chain is computed in bounded pieces and gives the eager bits.
    rng = np.random.default_rng(10)
    xs = rng.standard_normal((8, 8)).astype(np.float32)
    ws = (np.eye(8) + 0.01 * rng.standard_normal((8, 8))).astype(np.float32)
    bs = (0.01 * rng.standard_normal(8)).astype(np.float32)

    def run():
        x, w, b = (vc.Tensor(v, device="hip") for v in (xs, ws, bs))
        for _ in range(3000):
            x = (x @ w + b).relu()
        return [npy(x)]

    eager, deferred = _eager_then_deferred(run)
    _assert_same_bits(eager, deferred)
    assert np.isfinite(deferred[0]).all()


@hip_only
def test_relu_rule_falls_back_to_its_input_when_the_output_changes():
    rng = np.random.default_rng(9)
    xs, ws = rng.standard_normal((6, 5)).astype(np.float32), rng.standard_normal((5, 4)).astype(np.float32)

    def run(device):
        x = vc.Tensor(xs, requires_grad=True, device=device)
        w = vc.Tensor(ws, device=device)
        y = (x @ w).relu()
        loss = y.sum()
        ys = y.detach()
        ys.requires_grad = True
        (ys * -3.0).sum().backward()
        vc.sgd_step([ys], 1.0)  # rewrites the ReLU's output: every entry becomes >= 3
        loss.backward()  # the mask must still be [x @ w > 0]
        return [npy(x.grad), npy(y)]

    got = run("hip")
    np.testing.assert_allclose(got[0], run("cpu")[0], rtol=1e-5, atol=1e-5)
    assert (got[1] >= 3.0).all()
    mask = (xs.astype(np.float64) @ ws > 0).astype(np.float64)
    np.testing.assert_allclose(got[0], mask @ ws.T, rtol=1e-5, atol=1e-5)


# --- finite-difference gradcheck (test_autograd_correctness.py:47-143) ----------------


def _uniform(r, shape, lo=-1.0, hi=1.0):
    return r.uniform(lo, hi, size=shape).astype(np.float32)


def _away(r, shape):
    return (r.uniform(0.2, 1.0, size=shape) * r.choice([-1.0, 1.0], size=shape)).astype(np.float32)


def _separated(r, shape):
    n = int(np.prod(shape))
    return (r.permutation(n) * 0.1 - n * 0.05).reshape(shape).astype(np.float32)


def _signed_perm(r, n):
    m = np.zeros((n, n))
    m[np.arange(n), r.permutation(n)] = r.choice([-1.0, 1.0], size=n)
    return (m + r.uniform(-0.01, 0.01, size=(n, n))).astype(np.float32)


GRADCHECK = [
    ("add_row", lambda a, b: a + b, [lambda r: _uniform(r, (2, 3)), lambda r: _uniform(r, (3,))]),
    ("add_outer", lambda a, b: a + b, [lambda r: _uniform(r, (2, 1)), lambda r: _uniform(r, (1, 3))]),
    ("sub_col", lambda a, b: a - b, [lambda r: _uniform(r, (2, 3)), lambda r: _uniform(r, (2, 1))]),
    ("mul_rank3", lambda a, b: a * b, [lambda r: _uniform(r, (2, 3, 4)), lambda r: _uniform(r, (4,))]),
    ("div_bcast", lambda a, b: a / b, [lambda r: _uniform(r, (2, 3)), lambda r: _uniform(r, (3,), 1, 2)]),
    ("div_scalar", lambda a, b: a / b, [lambda r: _uniform(r, (2, 3)), lambda r: _uniform(r, (), 1, 2)]),
    ("neg", lambda a: -a, [lambda r: _uniform(r, (2, 3))]),
    ("affine", lambda a: a * 2.5 + 1.0, [lambda r: _uniform(r, (4,))]),
    ("reverse", lambda a: 3.0 / a - (1.0 - a), [lambda r: _uniform(r, (4,), 1, 2)]),
    ("matmul", lambda a, b: a @ b, [lambda r: _uniform(r, (3, 4)), lambda r: _uniform(r, (4, 2))]),
    ("matmul_vec", lambda a, b: a @ b, [lambda r: _uniform(r, (1, 5)), lambda r: _uniform(r, (5, 1))]),
    ("transpose", lambda a: a.T, [lambda r: _uniform(r, (3, 2))]),
    ("sum", lambda a: a.sum(), [lambda r: _uniform(r, (2, 3))]),
    ("mean", lambda a: a.mean(), [lambda r: _uniform(r, (2, 3))]),
    ("relu", lambda a: a.relu(), [lambda r: _away(r, (3, 4))]),
    ("sigmoid", lambda a: a.sigmoid(), [lambda r: _uniform(r, (3, 4), -3, 3)]),
    ("reshape", lambda a: a.reshape([3, 2]) * 2.0, [lambda r: _uniform(r, (2, 3))]),
    ("reused", lambda a: a * a + a, [lambda r: _uniform(r, (5,))]),
    ("linear_sigmoid", lambda x, w, b: (x @ w + b).sigmoid(),
     [lambda r: _uniform(r, (4, 3)), lambda r: _uniform(r, (3, 2)), lambda r: _uniform(r, (2,))]),
    ("two_layer_mse", lambda x, w1, w2, y: (((x @ w1).relu() @ w2 - y) * ((x @ w1).relu() @ w2 - y)).mean(),
     [lambda r: _away(r, (4, 3)), lambda r: _signed_perm(r, 3), lambda r: _uniform(r, (3, 1)),
      lambda r: _uniform(r, (4, 1))]),
    ("exp", lambda a: a.exp(), [lambda r: _uniform(r, (2, 3))]),
    ("log", lambda a: a.log(), [lambda r: _uniform(r, (2, 3), 1, 2)]),
    ("sum_axis0", lambda a: a.sum(0), [lambda r: _uniform(r, (3, 4))]),
    ("sum_keep_times", lambda a: a.sum(-1, keepdim=True) * a, [lambda r: _uniform(r, (2, 3, 4))]),
    ("mean_axis1", lambda a: a.mean(1), [lambda r: _uniform(r, (2, 3, 4))]),
    ("max_axis1", lambda a: a.max(1), [lambda r: _separated(r, (3, 4))]),
    ("max_axis0_keep", lambda a: a.max(0, keepdim=True) * a, [lambda r: _separated(r, (3, 4))]),
    ("max_all", lambda a: a.max(), [lambda r: _separated(r, (2, 3))]),
    ("softmax_rows", lambda a: a.softmax(-1), [lambda r: _uniform(r, (3, 4), -2, 2)]),
    ("softmax_axis0", lambda a: a.softmax(0), [lambda r: _uniform(r, (3, 4), -2, 2)]),
    ("log_softmax", lambda a: a.log_softmax(1), [lambda r: _uniform(r, (3, 4), -2, 2)]),
    ("cross_entropy", lambda a: vc.cross_entropy(a, [2, 0, 3]), [lambda r: _uniform(r, (3, 4), -2, 2)]),
    ("bmm", lambda a, b: a @ b, [lambda r: _uniform(r, (2, 3, 4)), lambda r: _uniform(r, (2, 4, 2))]),
    ("bmm_bcast_rhs", lambda a, b: a @ b, [lambda r: _uniform(r, (2, 3, 4)), lambda r: _uniform(r, (4, 2))]),
    ("bmm_bcast_lhs", lambda a, b: a @ b, [lambda r: _uniform(r, (3, 4)), lambda r: _uniform(r, (2, 4, 2))]),
    ("bmm_bcast_both", lambda a, b: a @ b, [lambda r: _uniform(r, (2, 1, 3, 4)), lambda r: _uniform(r, (3, 4, 2))]),
    ("transpose_rank3", lambda a: a.transpose(), [lambda r: _uniform(r, (2, 3, 4))]),
    ("mlp_classifier", lambda x, w1, w2: vc.cross_entropy((x @ w1).relu() @ w2, [0, 2, 1, 2]),
     [lambda r: _away(r, (4, 3)), lambda r: _signed_perm(r, 3), lambda r: _uniform(r, (3, 3))]),
]


@pytest.mark.parametrize("name,fn,factories", GRADCHECK, ids=[c[0] for c in GRADCHECK])
def test_gradcheck(gemm_device, name, fn, factories, eps=5e-3):
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    inputs = [f(rng) for f in factories]
    leaves = [vc.Tensor(x, requires_grad=True, device=gemm_device) for x in inputs]
    out = fn(*leaves)
    weights = np.random.default_rng(99).uniform(0.5, 1.5, size=out.shape).astype(np.float32)
    (out * vc.Tensor(weights, device=gemm_device)).sum().backward()

    def objective(values):
        r = fn(*[vc.Tensor(v, device=gemm_device) for v in values])
        return float((r * vc.Tensor(weights, device=gemm_device)).sum().item())

    for i, (leaf, base) in enumerate(zip(leaves, inputs)):
        assert leaf.grad is not None, f"input {i} received no gradient"
        numeric = np.zeros(base.size)
        for p in range(base.size):
            plus = [v.copy() for v in inputs]
            minus = [v.copy() for v in inputs]
            plus[i].reshape(-1)[p] += eps
            minus[i].reshape(-1)[p] -= eps
            numeric[p] = (objective(plus) - objective(minus)) / (2 * eps)
        np.testing.assert_allclose(npy(leaf.grad).reshape(-1), numeric, rtol=1e-2, atol=1e-2,
                                   err_msg=f"input {i} of {name} on {gemm_device}")


# --- kernels at edge shapes (test_performance_paths.py) ----------------------------------

GEMM_SHAPES = [(3, 5, 7), (4, 33, 33), (8, 256, 12), (16, 512, 24), (9, 257, 13), (63, 100, 97), (64, 64, 96),
               (65, 300, 95), (127, 513, 129), (200, 37, 1), (1, 300, 300), (300, 1, 300), (8, 3, 4100),
               (777, 64, 5), (128, 64, 128), (192, 256, 64), (128, 60, 128), (130, 64, 128), (128, 64, 70)]


@pytest.mark.parametrize("m,k,n", GEMM_SHAPES)
def test_matmul_edge_shapes(gemm_device, m, k, n):
    rng = np.random.default_rng(m * 10007 + k * 101 + n)
    a = rng.uniform(-1, 1, size=(m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, size=(k, n)).astype(np.float32)
    got = npy(vc.Tensor(a, device=gemm_device) @ vc.Tensor(b, device=gemm_device))
    np.testing.assert_allclose(got, a.astype(np.float64) @ b.astype(np.float64), rtol=1e-4, atol=1e-4 * np.sqrt(k))


@pytest.mark.parametrize("m,k,n", [(128, 64, 192), (64, 128, 64), (100, 72, 90), (128, 60, 128)])
def test_matmul_gradients_transposed_in_place(gemm_device, m, k, n):
    rng = np.random.default_rng(m + k + n)
    a = rng.uniform(-1, 1, size=(m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, size=(k, n)).astype(np.float32)
    g = rng.uniform(-1, 1, size=(m, n)).astype(np.float32)
    ta, tb = vc.Tensor(a, requires_grad=True, device=gemm_device), vc.Tensor(b, requires_grad=True, device=gemm_device)
    (ta @ tb).backward(vc.Tensor(g, device=gemm_device))
    np.testing.assert_allclose(npy(ta.grad), g.astype(np.float64) @ b.T, rtol=1e-4, atol=1e-4 * np.sqrt(n))
    np.testing.assert_allclose(npy(tb.grad), a.T.astype(np.float64) @ g, rtol=1e-4, atol=1e-4 * np.sqrt(m))


BROADCAST_CASES = [((1000, 300), (1000, 300)), ((1000, 300), ()), ((), (1000, 300)), ((1000, 300), (300,)),
                   ((1000, 300), (1000, 1)), ((1000, 1), (1, 300)), ((40, 1, 300), (1, 50, 300)),
                   ((40, 50, 1), (50, 7)), ((3,), (2, 1))]


@pytest.mark.parametrize("a_shape,b_shape", BROADCAST_CASES)
def test_elementwise_paths(device, a_shape, b_shape):
    rng = np.random.default_rng(len(a_shape) * 13 + len(b_shape))
    a = rng.uniform(0.5, 2, size=a_shape).astype(np.float32)
    b = rng.uniform(0.5, 2, size=b_shape).astype(np.float32)
    ta, tb = vc.Tensor(a, device=device), vc.Tensor(b, device=device)
    for op, ref in ((lambda x, y: x + y, np.add), (lambda x, y: x - y, np.subtract), (lambda x, y: x * y, np.multiply),
                    (lambda x, y: x / y, np.divide)):
        np.testing.assert_allclose(npy(op(ta, tb)), ref(a, b), rtol=1e-6, atol=1e-6)


def test_large_unary_ops(device):
    x = np.random.default_rng(3).uniform(-5, 5, size=(700, 300)).astype(np.float32)
    t = vc.Tensor(x, device=device)
    np.testing.assert_allclose(npy(t.relu()), np.maximum(x, 0))
    np.testing.assert_allclose(npy(t.sigmoid()), 1 / (1 + np.exp(-x)), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(npy(t.exp()), np.exp(x), rtol=1e-5)
    np.testing.assert_allclose(npy(-t), -x)


def test_sum_is_deterministic_and_accurate(device):
    x = np.random.default_rng(4).normal(size=3_000_001).astype(np.float32)
    t = vc.Tensor(x, device=device)
    values = {t.sum().item() for _ in range(5)}
    assert len(values) == 1
    assert np.isclose(values.pop(), x.astype(np.float64).sum(), rtol=1e-6, atol=1e-3)


def test_large_axis_reductions(device):
    x = np.random.default_rng(5).normal(size=(64, 500, 33)).astype(np.float32)
    t = vc.Tensor(x, device=device)
    for axis in (0, 1, 2):
        np.testing.assert_allclose(npy(t.sum(axis)), x.sum(axis=axis), rtol=1e-4, atol=1e-4)
        np.testing.assert_allclose(npy(t.max(axis)), x.max(axis=axis))
        np.testing.assert_array_equal(npy(t.argmax(axis)), x.argmax(axis=axis))


def test_broadcast_gradient_reduction_shapes(device):
    rng = np.random.default_rng(6)
    for big, small in [((8, 5, 7), (7,)), ((8, 5, 7), (5, 1)), ((8, 5, 7), (8, 1, 7)), ((8, 5, 7), (1, 1, 1)),
                       ((8, 5, 7), ())]:
        a = vc.Tensor(rng.normal(size=big).astype(np.float32), device=device)
        b = vc.Tensor(rng.normal(size=small).astype(np.float32), requires_grad=True, device=device)
        w = rng.normal(size=big).astype(np.float32)
        ((a + b) * vc.Tensor(w, device=device)).sum().backward()
        axes = tuple(range(len(big) - len(small))) + tuple(len(big) - len(small) + i for i, d in enumerate(small) if d == 1)
        expected = w.sum(axis=axes).reshape(small) if small else w.sum()
        np.testing.assert_allclose(npy(b.grad), expected, rtol=1e-4, atol=1e-4)


def test_mlp_learns_nonlinear_spiral(gemm_device):
    rng = np.random.default_rng(0)
    feats, labels = [], []
    for k in range(3):
        r = np.linspace(0.05, 1.0, 60)
        t = np.linspace(4.0 * k, 4.0 * (k + 1), 60) + rng.normal(scale=0.2, size=60)
        feats.append(np.column_stack([r * np.sin(t), r * np.cos(t)]))
        labels += [k] * 60
    x = vc.Tensor(np.concatenate(feats).astype(np.float32), device=gemm_device)
    first, second = vc.Linear(2, 64, 1), vc.Linear(64, 3, 2)
    params = [p.to(gemm_device).detach() for p in (first.weight, first.bias, second.weight, second.bias)]
    for p in params:
        p.requires_grad = True
    first.weight, first.bias, second.weight, second.bias = params
    for _ in range(600):
        loss = vc.cross_entropy(second(first(x).relu()), labels)
        loss.backward()
        vc.sgd_step(params, 1.0)
        vc.zero_grad(params)
    pred = npy(second(first(x).relu()).argmax(1)).astype(int)
    assert (pred == np.array(labels)).mean() > 0.95


# --- asynchronous device execution (test_performance_paths.py:182-227) ----------------


@hip_only
def test_hip_long_dependency_chain_without_sync():
    x = vc.Tensor(np.zeros(1000, dtype=np.float32), device="hip")
    for _ in range(2000):
        x = x + 1.0
    np.testing.assert_allclose(npy(x), 2000.0)


@hip_only
def test_hip_in_place_update_is_ordered():
    w = vc.Tensor(np.ones(256, dtype=np.float32), requires_grad=True, device="hip")
    before = w * 2.0
    (w * 1.0).sum().backward()
    vc.sgd_step([w], 0.5)
    after = w * 2.0
    np.testing.assert_allclose(npy(before), 2.0)
    np.testing.assert_allclose(npy(after), 1.0)


@hip_only
def test_hip_buffer_reuse_does_not_corrupt_results():
    rng = np.random.default_rng(7)
    expected, results = [], []
    for _ in range(200):
        data = rng.normal(size=int(rng.integers(1, 5000))).astype(np.float32)
        t = vc.Tensor(data, device="hip")
        tmp = (t * 3.0).relu()
        results.append((tmp - t).sum())
        expected.append(float((np.maximum(data * 3.0, 0) - data).astype(np.float64).sum()))
        del t, tmp
    for got, want in zip(results, expected):
        assert np.isclose(got.item(), want, rtol=1e-4, atol=1e-3)


@hip_only
def test_hip_synchronize_and_sgd_matches_cpu():
    vc.synchronize()
    rng = np.random.default_rng(7)
    w_np, x_np = rng.normal(size=(3, 2)).astype(np.float32), rng.normal(size=(4, 3)).astype(np.float32)
    out = {}
    for dev in ("cpu", "hip"):
        w, x = vc.Tensor(w_np, requires_grad=True, device=dev), vc.Tensor(x_np, device=dev)
        for _ in range(5):
            vc.cross_entropy(x @ w, [0, 1, 1, 0]).backward()
            vc.sgd_step([w], 0.5)
            vc.zero_grad([w])
        out[dev] = npy(w)
    vc.synchronize()
    np.testing.assert_allclose(out["hip"], out["cpu"], rtol=1e-4, atol=1e-5)


@hip_only
def test_hip_sgd_over_many_parameters_matches_one_at_a_time():
    # sgd_step batches hip parameters into list launches; a parameter listed
    # twice must still be stepped twice, in order, like the one-at-a-time loop.
    rng = np.random.default_rng(3)
    shapes = [(int(rng.integers(1, 300)),) for _ in range(19)] + [(64, 33), (5,)]
    data = [rng.normal(size=s).astype(np.float32) for s in shapes]
    coef = [rng.normal(size=s).astype(np.float32) for s in shapes]

    def stepped(batched):
        ps = [vc.Tensor(d, requires_grad=True, device="hip") for d in data]
        loss = None
        for p, c in zip(ps, coef):
            term = (p * vc.Tensor(c, device="hip")).sum()
            loss = term if loss is None else loss + term
        loss.backward()
        order = ps + [ps[3], ps[20]]
        if batched:
            vc.sgd_step(order, 0.25)
        else:
            for p in order:
                vc.sgd_step([p], 0.25)
        return [npy(p) for p in ps]

    for got, want in zip(stepped(True), stepped(False)):
        np.testing.assert_array_equal(got, want)
    np.testing.assert_allclose(stepped(True)[3], data[3] - 0.5 * coef[3], rtol=1e-6, atol=1e-6)


@hip_only
def test_hip_loss_item_is_published_without_a_full_synchronisation():
    # loss.item() reads the value the loss kernel published; later work (the
    # backward pass, the update) does not change it, and an in-place update of
    # the loss storage itself withdraws the published value.
    rng = np.random.default_rng(13)
    logits = vc.Tensor(rng.standard_normal((64, 10)).astype(np.float32), requires_grad=True, device="hip")
    targets = list(rng.integers(0, 10, 64))
    loss = vc.cross_entropy(logits, targets)
    loss.backward()
    vc.sgd_step([logits], 0.5)
    got = loss.item()
    ref = vc.cross_entropy(vc.Tensor(npy(logits) + 0.5 * npy(logits.grad), device="cpu"), targets).item()
    assert np.isclose(got, ref, rtol=1e-6)
    total = (logits * 1.0).sum()
    assert np.isclose(total.item(), float(npy(logits).astype(np.float64).sum()), rtol=1e-5, atol=1e-4)
    seed = loss.detach()
    seed.requires_grad = True
    (seed * 2.0).sum().backward()
    vc.sgd_step([seed], 1.0)  # rewrites the loss storage: seed -= 2
    assert np.isclose(loss.item(), got - 2.0, rtol=1e-6)


@hip_only
def test_hip_gemm_kernel_reported():
    assert vc.hip_gemm_kernel() in ("mfma", "simple")
    assert "gfx950" in vc.hip_device_name()
    previous = vc.hip_set_gemm_kernel("simple")
    try:
        assert vc.hip_gemm_kernel() == "simple"
        with pytest.raises(ValueError, match="unknown GEMM kernel"):
            vc.hip_set_gemm_kernel("tiled")
        assert vc.hip_gemm_kernel() == "simple"
    finally:
        vc.hip_set_gemm_kernel(previous)
    assert vc.hip_gemm_kernel() == previous


def test_hip_unavailable_is_loud_on_cpu_hosts():
    if vc.hip_available():
        pytest.skip("a GPU is present")
    with pytest.raises(RuntimeError, match="HIP"):
        vc.Tensor([1.0], device="hip")
    with pytest.raises(RuntimeError):
        vc.Tensor([1.0], device="metal")
    with pytest.raises(RuntimeError, match="HIP"):
        vc.hip_set_gemm_kernel("simple")
    assert vc.hip_gemm_kernel() == "unavailable"


@pytest.mark.parametrize("call", [
    lambda: vc.Tensor([[1.0, 2.0]]).sum(2),
    lambda: vc.Tensor([[1.0, 2.0]]).max(-3),
    lambda: vc.Tensor(3.0).sum(0),
    lambda: vc.Tensor(np.zeros((2, 0), dtype=np.float32)).max(1),
    lambda: vc.Tensor(np.zeros((2, 0), dtype=np.float32)).mean(1),
    lambda: vc.Tensor(np.ones((2, 3, 4), dtype=np.float32)) @ vc.Tensor(np.ones((3, 5, 2), dtype=np.float32)),
    lambda: vc.Tensor(np.ones((2, 3), dtype=np.float32)) @ vc.Tensor(np.ones((4, 2), dtype=np.float32)),
    lambda: vc.Tensor([1.0, 2.0]) @ vc.Tensor([1.0, 2.0]),
    lambda: vc.cross_entropy(vc.Tensor([1.0, 2.0]), [0]),
    lambda: vc.cross_entropy(vc.Tensor([[1.0, 2.0]]), [0, 1]),
    lambda: vc.cross_entropy(vc.Tensor([[1.0, 2.0]]), [2]),
])
def test_invalid_inputs_raise(call):
    with pytest.raises((ValueError, IndexError, RuntimeError)):
        call()


def test_sum_of_empty_axis_is_zero(device):
    close(vc.Tensor(np.zeros((2, 0), dtype=np.float32), device=device).sum(1), [0.0, 0.0])


def test_reference_module_name_is_the_same_module():
    # The reference's tests and examples start with `import vectorcore as vc`
    # (python/bindings.cpp:63).
    import vectorcore
    assert vectorcore.Tensor is vc.Tensor and vectorcore.cross_entropy is vc.cross_entropy
    assert vectorcore.Linear is vc.Linear and vectorcore.sgd_step is vc.sgd_step
    x = vectorcore.Tensor([1.0, 2.0, 3.0], requires_grad=True)
    ((x * x) + x).sum().backward()
    np.testing.assert_array_equal(x.grad.numpy(), [3, 5, 7])
