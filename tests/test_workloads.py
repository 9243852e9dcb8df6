"""GPU parity of the five backward-pass workloads through the runtime
(autograd graph, hip device) against the oracle and the reference fixtures.

Tolerances (written per check): bit-exact for argmax; 1e-5 relative for
elementwise gradients (with an absolute floor for values near zero); 1e-4
relative for GEMM and reduction results (with the reference's own
atol = 1e-4 sqrt(k) for GEMMs, tests/python/test_performance_paths.py:43).
"""

import numpy as np
import pytest

import vectorcore_amd as vc
from oracle import autograd as A
from oracle import kernels as K
from vectorcore_amd import workloads as W

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def hip_device():
    assert vc.hip_available(), "the hip device must be available on a GPU run"


@pytest.fixture(params=["mfma", "simple"])
def gemm_kernel(request):
    """The MLP tests run on the MFMA GEMM and again with the portable FMA GEMM
    selected (tests/python/test_performance_paths.py:89-103 re-runs the
    reference's MLP tests with its portable kernel forced)."""
    previous = vc.hip_set_gemm_kernel(request.param)
    try:
        yield request.param
    finally:
        vc.hip_set_gemm_kernel(previous)


def H(x, grad=False):
    return vc.Tensor(np.asarray(x, dtype=np.float32), requires_grad=grad, device="hip")


def build_mlp(weights, biases):
    params = []
    for w, b in zip(weights, biases):
        params += [H(w, True), H(b, True)]
    return params


def mlp_logits(params, x):
    h = x
    layers = len(params) // 2
    for i in range(layers):
        h = h @ params[2 * i] + params[2 * i + 1]
        if i + 1 < layers:
            h = h.relu()
    return h


# --- spiral classifier step (2 -> 64 -> 3, 300 points, lr 1.0) -------------------------


def test_spiral_steps_match_reference_fixture(golden, gemm_kernel):
    sp = W.spiral()
    params = build_mlp(sp["weights"], sp["biases"])
    x = H(sp["x"])
    losses = []
    for _ in range(5):
        loss = vc.cross_entropy(mlp_logits(params, x), sp["targets"])
        loss.backward()
        vc.sgd_step(params, 1.0)
        vc.zero_grad(params)
        losses.append(loss.item())
    np.testing.assert_allclose(losses, golden["spiral_losses"], rtol=1e-5)
    for i in range(2):
        np.testing.assert_allclose(params[2 * i].numpy(), golden[f"spiral_w{i}_after5"], rtol=1e-4, atol=1e-6)
        np.testing.assert_allclose(params[2 * i + 1].numpy(), golden[f"spiral_b{i}_after5"], rtol=1e-4, atol=1e-6)


# --- batched matmul backward (A, B, dC [8, 1024, 1024]; broadcast B [1, 1024, 1024]) ----


@pytest.mark.parametrize("name", ["bmm", "bmm_bcast", "bmm_bcast_rank"])
def test_bmm_backward_matches_reference_fixture(golden, name):
    a, b = H(golden[f"{name}_a"], True), H(golden[f"{name}_b"], True)
    (a @ b).backward(H(golden[f"{name}_dc"]))
    k = golden[f"{name}_a"].shape[-1]
    np.testing.assert_allclose(a.grad.numpy(), golden[f"{name}_da"], rtol=1e-4, atol=1e-4 * np.sqrt(k))
    np.testing.assert_allclose(b.grad.numpy(), golden[f"{name}_db"], rtol=1e-4, atol=1e-4 * np.sqrt(k * 3))


def _sampled_dots(got, left, right, samples, rng, trans_left=False, trans_right=False, batch_sum=False):
    """Float64 dot products at random output positions (size-independent check)."""
    for _ in range(samples):
        i = rng.integers(got.shape[-2])
        j = rng.integers(got.shape[-1])
        if batch_sum:
            want = sum(np.dot((left[z][:, i] if trans_left else left[z][i]).astype(np.float64),
                              (right[z][j] if trans_right else right[z][:, j]).astype(np.float64))
                       for z in range(left.shape[0]))
            g = got[i, j]
        else:
            z = rng.integers(got.shape[0])
            lrow = left[z][:, i] if trans_left else left[z][i]
            rcol = right[min(z, right.shape[0] - 1)][j] if trans_right else right[min(z, right.shape[0] - 1)][:, j]
            want = np.dot(lrow.astype(np.float64), rcol.astype(np.float64))
            g = got[z, i, j]
        assert abs(g - want) <= 1e-4 * abs(want) + 1e-4 * np.sqrt(left.shape[-1] * (left.shape[0] if batch_sum else 1))


def test_bmm_backward_full_size():
    bm = W.bmm()
    a, b = H(bm["a"], True), H(bm["b"], True)
    (a @ b).backward(H(bm["dc"]))
    da, db = a.grad.numpy(), b.grad.numpy()
    # batch 0 against the oracle in full, every batch by sampled float64 dots
    np.testing.assert_allclose(da[0], K.matmul2d(bm["dc"][0], bm["b"][0], False, True), rtol=1e-4, atol=1e-4 * 32)
    np.testing.assert_allclose(db[0], K.matmul2d(bm["a"][0], bm["dc"][0], True, False), rtol=1e-4, atol=1e-4 * 32)
    rng = np.random.default_rng(0)
    _sampled_dots(da, bm["dc"], bm["b"], 200, rng, trans_right=True)
    _sampled_dots(db, bm["a"], bm["dc"], 200, rng, trans_left=True)


def test_bmm_backward_broadcast_full_size():
    bm = W.bmm()
    a, b = H(bm["a"], True), H(bm["b_shared"], True)
    (a @ b).backward(H(bm["dc"]))
    db = b.grad.numpy()
    assert db.shape == (1, 1024, 1024)
    rng = np.random.default_rng(1)
    _sampled_dots(db[0], bm["a"], bm["dc"], 100, rng, trans_left=True, batch_sum=True)
    da = a.grad.numpy()
    np.testing.assert_allclose(da[3], K.matmul2d(bm["dc"][3], bm["b_shared"][0], False, True), rtol=1e-4,
                               atol=1e-4 * 32)
    # the batch-reduced product equals summing per-batch oracle products
    want = np.zeros((1024, 1024), dtype=np.float64)
    for z in range(8):
        want += K.matmul2d(bm["a"][z], bm["dc"][z], True, False)
    np.testing.assert_allclose(db[0], want, rtol=1e-4, atol=1e-4 * np.sqrt(8 * 1024))


# --- broadcast add + activation gradients (x [4096, 4096], bias [1, 4096]) -----------


def activation_hip(act):
    x, bias = H(act["x"], True), H(act["bias"], True)
    y = (x + bias).relu().sigmoid() * (x * 0.1).exp()
    y.backward(H(act["dy"]))
    return y.numpy(), x.grad.numpy(), bias.grad.numpy()


def activation_oracle(act):
    x, bias = A.T(act["x"], True), A.T(act["bias"], True)
    y = A.sigmoid(A.relu(x + bias)) * A.exp(x * 0.1)
    y.backward(A.T(act["dy"]))
    return y.data, x.grad.data, bias.grad.data


def test_activation_backward_matches_reference_fixture(golden):
    act = dict(x=golden["act_x"], bias=golden["act_bias"], dy=golden["act_dy"])
    y, dx, dbias = activation_hip(act)
    np.testing.assert_allclose(y, golden["act_y"], rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(dx, golden["act_dx"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(dbias, golden["act_dbias"], rtol=1e-4, atol=1e-5)


def test_activation_backward_full_size_and_deterministic():
    act = W.activation()
    y, dx, dbias = activation_hip(act)
    ry, rdx, rdbias = activation_oracle(act)
    np.testing.assert_allclose(y, ry, rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(dx, rdx, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(dbias, rdbias, rtol=1e-4, atol=1e-4)
    _, _, dbias2 = activation_hip(act)
    np.testing.assert_array_equal(dbias, dbias2)  # identical across runs


# --- softmax cross-entropy + argmax (logits [32768, 1000]) ---------------------------


def test_cross_entropy_full_size_and_argmax_bitexact():
    xe = W.xent()
    t = H(xe["logits"], True)
    loss = vc.cross_entropy(t, xe["targets"])
    loss.backward()
    got_loss, grad = loss.item(), t.grad.numpy()
    am = t.detach().argmax(1).numpy()
    rt = A.T(xe["logits"], True)
    ref_loss = A.cross_entropy(rt, xe["targets"])
    ref_loss.backward()
    assert np.isclose(got_loss, float(ref_loss.data), rtol=1e-6)
    np.testing.assert_allclose(grad, rt.grad.data, rtol=1e-5, atol=1e-10)
    np.testing.assert_array_equal(am, K.reduce_axis(xe["logits"], 1, K.ARGMAX))
    # gradient rows sum to zero and the target entries are negative
    assert np.abs(grad.astype(np.float64).sum(axis=1)).max() < 1e-8
    assert np.all(grad[np.arange(grad.shape[0]), xe["targets"]] < 0)


def test_cross_entropy_matches_reference_fixture(golden):
    t = H(golden["xent_logits"], True)
    loss = vc.cross_entropy(t, golden["xent_targets"])
    loss.backward()
    assert np.isclose(loss.item(), golden["xent_loss"], rtol=1e-6)
    np.testing.assert_allclose(t.grad.numpy(), golden["xent_grad"], rtol=1e-5, atol=1e-10)
    np.testing.assert_array_equal(t.detach().argmax(1).numpy(), golden["xent_argmax"])


# --- MLP train step (8192 x 1024 -> 4096 -> 4096 -> 1000) ----------------------------


def test_mlp_small_matches_reference_fixture(golden, gemm_kernel):
    n = 3
    params = build_mlp([golden[f"mlp_w{i}"] for i in range(n)], [golden[f"mlp_b{i}"] for i in range(n)])
    x, t = H(golden["mlp_x"]), golden["mlp_targets"]
    loss = vc.cross_entropy(mlp_logits(params, x), t)
    loss.backward()
    assert np.isclose(loss.item(), golden["mlp_loss"], rtol=1e-6)
    for i in range(n):
        np.testing.assert_allclose(params[2 * i].grad.numpy(), golden[f"mlp_dw{i}"], rtol=1e-4, atol=1e-7)
        np.testing.assert_allclose(params[2 * i + 1].grad.numpy(), golden[f"mlp_db{i}"], rtol=1e-4, atol=1e-7)
    vc.zero_grad(params)
    losses = []
    for _ in range(3):
        loss = vc.cross_entropy(mlp_logits(params, x), t)
        loss.backward()
        vc.sgd_step(params, 0.01)
        vc.zero_grad(params)
        losses.append(loss.item())
    np.testing.assert_allclose(losses, golden["mlp_losses"], rtol=1e-5)
    for i in range(n):
        np.testing.assert_allclose(params[2 * i].numpy(), golden[f"mlp_w{i}_after3"], rtol=1e-5, atol=1e-7)


def test_mlp_workload_architecture_against_oracle(gemm_kernel):
    """The full 1024 -> 4096 -> 4096 -> 1000 network on a 64-row batch."""
    m = W.mlp(batch=64)
    params = build_mlp(m["weights"], m["biases"])
    loss = vc.cross_entropy(mlp_logits(params, H(m["x"])), m["targets"])
    loss.backward()
    ref = A.Mlp(m["weights"], m["biases"])
    ref_loss = A.cross_entropy(ref.logits(A.T(m["x"])), m["targets"])
    ref_loss.backward()
    assert np.isclose(loss.item(), float(ref_loss.data), rtol=1e-5)
    for p, r in zip(params, ref.params()):
        np.testing.assert_allclose(p.grad.numpy(), r.grad.data, rtol=1e-4, atol=1e-6)


def test_mnist_shaped_steps_against_oracle(gemm_kernel):
    """The reference's second train benchmark, 256 x 784 -> 256 -> 10 with its
    own generator (benchmarks/train_benchmark.py:23-45): three steps of loss,
    backward and SGD at lr 0.1 against the oracle's restatement."""
    mn = W.mnist_shaped()
    params = build_mlp(mn["weights"], mn["biases"])
    x = H(mn["x"])
    ref = A.Mlp(mn["weights"], mn["biases"])
    xr = A.T(mn["x"])
    targets = [int(t) for t in mn["targets"]]
    for step in range(3):
        loss = vc.cross_entropy(mlp_logits(params, x), targets)
        loss.backward()
        grads = [p.grad.numpy() for p in params]
        vc.sgd_step(params, mn["lr"])
        vc.zero_grad(params)
        ref_loss = A.cross_entropy(ref.logits(xr), targets)
        ref_loss.backward()
        np.testing.assert_allclose(loss.item(), float(ref_loss.data), rtol=1e-5, err_msg=f"step {step}")
        for g, r in zip(grads, ref.params()):
            np.testing.assert_allclose(g, r.grad.data, rtol=1e-4, atol=1e-6, err_msg=f"step {step}")
        A.sgd_step(ref.params(), mn["lr"])
        A.zero_grad(ref.params())
    for p, r in zip(params, ref.params()):
        np.testing.assert_allclose(p.numpy(), r.data, rtol=1e-4, atol=1e-6)


def mlp_backward_float64(m, zs):
    """Float64 gradients of mean cross-entropy through the ReLU MLP, evaluated
    on the given forward pre-activations zs (so the ReLU masks are the ones the
    checked forward produced: a pre-activation within fp32 rounding of zero may
    otherwise flip its mask between precisions)."""
    ws = [w.astype(np.float64) for w in m["weights"]]
    hs = [m["x"].astype(np.float64)] + [np.maximum(z, 0) for z in zs[:-1]]
    z = zs[-1] - zs[-1].max(axis=1, keepdims=True)
    p = np.exp(z)
    p /= p.sum(axis=1, keepdims=True)
    n = p.shape[0]
    g = p
    g[np.arange(n), m["targets"]] -= 1.0
    g /= n
    grads = [None] * (2 * len(ws))
    for i in reversed(range(len(ws))):
        grads[2 * i] = hs[i].T @ g
        grads[2 * i + 1] = g.sum(axis=0)
        if i:
            g = (g @ ws[i].T) * (zs[i - 1] > 0)
    return grads


def test_mlp_full_size_step_against_float64_and_pool_reuse():
    m = W.mlp()
    params = build_mlp(m["weights"], m["biases"])
    x = H(m["x"])
    allocations, losses, grads, zs_dev = [], [], None, None
    for step in range(4):
        h, zs = x, []
        for i in range(3):
            h = h @ params[2 * i] + params[2 * i + 1]
            zs.append(h)
            if i < 2:
                h = h.relu()
        loss = vc.cross_entropy(h, m["targets"])
        loss.backward()
        if step == 0:
            grads = [p.grad.numpy() for p in params]
            zs_dev = [z.numpy().astype(np.float64) for z in zs]
        del zs, h
        vc.sgd_step(params, m["lr"])
        vc.zero_grad(params)
        losses.append(loss.item())
        allocations.append(vc.hip_pool_stats()["device_allocations"])
    # buffers are recycled: no new device allocation after the second step
    assert allocations[3] == allocations[1], allocations
    assert losses[3] < losses[0]
    # forward: every pre-activation against float64 (1e-4 relative, floor at
    # 1e-5 of the largest magnitude)
    hprev = m["x"].astype(np.float64)
    for i, (w, b) in enumerate(zip(m["weights"], m["biases"])):
        ref = hprev @ w.astype(np.float64) + b
        np.testing.assert_allclose(zs_dev[i], ref, rtol=1e-4, atol=1e-5 * np.abs(ref).max(), err_msg=f"z{i + 1}")
        hprev = np.maximum(zs_dev[i], 0)
    # backward: every parameter gradient against float64 on the same forward
    for i, (g, r) in enumerate(zip(grads, mlp_backward_float64(m, zs_dev))):
        np.testing.assert_allclose(g, r, rtol=1e-4, atol=1e-5 * np.abs(r).max(), err_msg=f"parameter {i}")


def test_mlp_train_steps_are_bitwise_reproducible():
    """No atomics and shape-fixed partitions: the same steps from the same
    start give the same losses and parameters, bit for bit (the split-K
    products, the ReLU fold and the column sums included)."""
    m = W.mlp(batch=1024, dims=(256, 2048, 512, 100))

    def run():
        params = build_mlp(m["weights"], m["biases"])
        x = H(m["x"])
        losses = []
        for _ in range(3):
            loss = vc.cross_entropy(mlp_logits(params, x), m["targets"])
            loss.backward()
            vc.sgd_step(params, 0.05)
            vc.zero_grad(params)
            losses.append(loss.item())
        return losses, [p.numpy() for p in params]

    l1, p1 = run()
    l2, p2 = run()
    assert l1 == l2 and l1[-1] < l1[0]
    for a, b in zip(p1, p2):
        np.testing.assert_array_equal(a, b)


def test_mlp_train_steps_with_and_without_deferred_products_are_bitwise_equal():
    """The full-size step with its forward products deferred (bias and ReLU in
    the GEMM epilogue, large products on a transposed B, copy-on-write for the
    updated weights) against eager products: two steps, bit for bit."""
    m = W.mlp()

    def run():
        params = build_mlp(m["weights"], m["biases"])
        x = H(m["x"])
        losses = []
        for _ in range(2):
            loss = vc.cross_entropy(mlp_logits(params, x), m["targets"])
            loss.backward()
            vc.sgd_step(params, m["lr"])
            vc.zero_grad(params)
            losses.append(loss.item())
        return losses, [p.numpy() for p in params]

    previous = vc.hip_defer_products(False)
    try:
        eager = run()
    finally:
        vc.hip_defer_products(True)
    try:
        deferred = run()
    finally:
        vc.hip_defer_products(previous)
    assert eager[0] == deferred[0]
    for a, b in zip(eager[1], deferred[1]):
        np.testing.assert_array_equal(a, b)
