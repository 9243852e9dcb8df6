"""Pins the CPU oracle before anything is checked against it:
  1. the reference's own known-answer vectors;
  2. bit-exact agreement with the reference built from source (committed
     fixtures, plus live comparisons where oracle/_ref is built);
  3. closed forms in float64 (NumPy, and torch for cross-entropy);
  4. planted mistakes (a transposed operand, a dropped 1/N, last-wins argmax,
     float32 accumulation) that these checks must catch.
"""

import numpy as np
import pytest

from oracle import autograd as A
from oracle import kernels as K
from tests.golden.make_golden import GEMM_SHAPES, gemm_inputs, sum_input
from vectorcore_amd import workloads as W


def flat(t):
    return np.asarray(t.data if isinstance(t, A.T) else t, dtype=np.float64).ravel()


# --- 1. known answers -------------------------------------------------------

def test_known_forward_answers(known):
    np.testing.assert_array_equal(flat(A.matmul(A.T(known["matmul"]["a"]), A.T(known["matmul"]["b"]))),
                                  known["matmul"]["out"])
    np.testing.assert_array_equal(flat(A.transpose(A.T(known["transpose"]["a"]))), known["transpose"]["out"])
    np.testing.assert_array_equal(flat(A.transpose(A.T(known["transpose_rank3"]["a"]))),
                                  known["transpose_rank3"]["out"])
    e = known["elementwise"]
    a, b = A.T(e["a"]), A.T(e["b"])
    np.testing.assert_array_equal(flat(a + b), e["add"])
    np.testing.assert_array_equal(flat(a - b), e["sub"])
    np.testing.assert_array_equal(flat(a * b), e["mul"])
    np.testing.assert_allclose(flat(a / b), e["div"], rtol=1e-7)
    np.testing.assert_array_equal(flat(-a), e["neg"])
    np.testing.assert_array_equal(flat(2.0 + a * 2.0), e["affine_2_plus_a_times_2"])
    br = known["broadcast_row"]
    np.testing.assert_array_equal(flat(A.T(br["a"]) + A.T(br["b"])), br["out"])
    r = known["reductions"]
    x = A.T(r["x"])
    assert A.sum_all(x).data == r["sum"] and A.mean_all(x).data == r["mean"]
    np.testing.assert_array_equal(flat(A.relu(x)), r["relu"])
    assert abs(A.sigmoid(x).data[2] - r["sigmoid_at_zero"]) < 1e-6
    ax = known["axis_reductions"]
    x = A.T(ax["x"])
    np.testing.assert_array_equal(flat(A.sum_axis(x, 0)), ax["sum0"])
    np.testing.assert_array_equal(flat(A.sum_axis(x, -1, True)), ax["sum_last_keepdim"])
    np.testing.assert_array_equal(flat(A.mean_axis(x, 1)), ax["mean1"])
    np.testing.assert_array_equal(flat(A.max_axis(x, 1)), ax["max1"])
    np.testing.assert_array_equal(flat(A.max_axis(x, 0)), ax["max0"])
    np.testing.assert_array_equal(flat(A.argmax(x, 1)), ax["argmax1"])
    assert A.max_all(x).data == ax["max_all"]
    np.testing.assert_array_equal(flat(A.argmax(A.T(known["argmax_ties"]["x"]), 1)), known["argmax_ties"]["argmax1"])


def test_known_gradient_answers(known):
    c = known["autograd_repeated"]
    x = A.T(c["x"], True)
    A.sum_all(x * x + x).backward()
    np.testing.assert_array_equal(flat(x.grad), c["grad"])
    c = known["broadcast_grad"]
    x, b = A.T(c["x"], True), A.T(c["bias"], True)
    A.sum_all(x + b).backward()
    np.testing.assert_array_equal(flat(x.grad), c["x_grad"])
    np.testing.assert_array_equal(flat(b.grad), c["bias_grad"])
    c = known["matmul_grads"]
    a, b = A.T(c["a"], True), A.T(c["b"], True)
    A.sum_all(A.matmul(a, b)).backward()
    np.testing.assert_array_equal(flat(a.grad), c["a_grad"])
    np.testing.assert_array_equal(flat(b.grad), c["b_grad"])
    c = known["grad_accumulation"]
    x = A.T(c["x"], True)
    A.sum_all(x * 3.0).backward()
    A.sum_all(x * 4.0).backward()
    np.testing.assert_array_equal(flat(x.grad), c["grad"])
    c = known["relu_bias_grads"]
    x, b = A.T(c["x"], True), A.T(c["bias"], True)
    A.sum_all(A.relu(x + b)).backward()
    np.testing.assert_array_equal(flat(x.grad), c["x_grad"])
    np.testing.assert_array_equal(flat(b.grad), c["bias_grad"])
    c = known["retain_grad"]
    a = A.T(c["a"], True)
    hidden, kept = a * 2.0, a * 3.0
    kept.retain_grad()
    (A.sum_all(hidden * hidden) + A.sum_all(kept)).backward()
    assert hidden.grad is None
    np.testing.assert_array_equal(flat(kept.grad), c["kept_grad"])
    np.testing.assert_array_equal(flat(a.grad), c["a_grad"])
    c = known["cross_entropy"]
    logits = A.T(c["logits"], True)
    loss = A.cross_entropy(logits, c["targets"])
    assert abs(float(loss.data) - c["loss"]) < 1e-6
    loss.backward()
    np.testing.assert_array_equal(flat(logits.grad), c["grad"])
    c = known["batched_broadcast_matmul"]
    a, w = A.T(c["a"], True), A.T(c["w"], True)
    y = A.matmul(a, w)
    np.testing.assert_array_equal(flat(y), c["y"])
    A.sum_all(y).backward()
    np.testing.assert_array_equal(flat(w.grad), c["w_grad"])
    np.testing.assert_array_equal(flat(a.grad), c["a_grad"])
    c = known["sgd_square"]
    p = A.T(c["p"], True)
    A.sum_all(p * p).backward()
    A.sgd_step([p], c["lr"])
    np.testing.assert_array_equal(flat(p), c["p_after"])
    c = known["max_grad_ties"]
    x = A.T(c["x"], True)
    A.sum_all(A.max_axis(x, 1)).backward()
    np.testing.assert_array_equal(x.grad.data, np.asarray(c["grad"], dtype=np.float32))


# --- 2. bit-exact against the reference built from source -------------------

@pytest.mark.parametrize("m,k,n", GEMM_SHAPES)
def test_gemm_bitexact_vs_reference_fixture(golden, m, k, n):
    for ta in (0, 1):
        for tb in (0, 1):
            a, b = gemm_inputs(m, k, n, ta, tb)
            np.testing.assert_array_equal(K.matmul2d(a, b, bool(ta), bool(tb)), golden[f"gemm_{m}_{k}_{n}_{ta}{tb}_c"])


def test_reductions_bitexact_vs_reference_fixture(golden):
    x = golden["reduce_x"]
    for axis in (0, 1, 2):
        for op, name in ((K.SUM, "sum"), (K.MAX, "max"), (K.ARGMAX, "argmax")):
            np.testing.assert_array_equal(K.reduce_axis(x, axis, op), golden[f"reduce_{name}_{axis}"])
    assert K.sum_all(sum_input()) == golden["sum_out"]


def test_matmul_backward_bitexact_vs_reference_fixture(golden):
    for name in ("bmm", "bmm_bcast", "bmm_bcast_rank"):
        a, b = A.T(golden[f"{name}_a"], True), A.T(golden[f"{name}_b"], True)
        A.matmul(a, b).backward(A.T(golden[f"{name}_dc"]))
        np.testing.assert_array_equal(a.grad.data, golden[f"{name}_da"])
        np.testing.assert_array_equal(b.grad.data, golden[f"{name}_db"])


def test_activation_backward_bitexact_vs_reference_fixture(golden):
    x, b = A.T(golden["act_x"], True), A.T(golden["act_bias"], True)
    y = A.relu(x + b)
    y = A.sigmoid(y) * A.exp(x * 0.1)
    np.testing.assert_array_equal(y.data, golden["act_y"])
    y.backward(A.T(golden["act_dy"]))
    np.testing.assert_array_equal(x.grad.data, golden["act_dx"])
    np.testing.assert_array_equal(b.grad.data, golden["act_dbias"])


def test_cross_entropy_bitexact_vs_reference_fixture(golden):
    logits = A.T(golden["xent_logits"], True)
    loss = A.cross_entropy(logits, golden["xent_targets"])
    assert loss.data == golden["xent_loss"]
    loss.backward()
    np.testing.assert_array_equal(logits.grad.data, golden["xent_grad"])
    np.testing.assert_array_equal(A.argmax(A.T(golden["xent_logits"]), 1).data, golden["xent_argmax"])


def test_mlp_bitexact_vs_reference_fixture(golden):
    n = 3
    net = A.Mlp([golden[f"mlp_w{i}"] for i in range(n)], [golden[f"mlp_b{i}"] for i in range(n)])
    x, t = A.T(golden["mlp_x"]), golden["mlp_targets"]
    loss = A.cross_entropy(net.logits(x), t)
    assert loss.data == golden["mlp_loss"]
    loss.backward()
    for i in range(n):
        np.testing.assert_array_equal(net.weights[i].grad.data, golden[f"mlp_dw{i}"])
        np.testing.assert_array_equal(net.biases[i].grad.data, golden[f"mlp_db{i}"])
    A.zero_grad(net.params())
    losses = [net.step(x, t, 0.01) for _ in range(3)]
    np.testing.assert_array_equal(np.asarray(losses, dtype=np.float32), golden["mlp_losses"])
    for i in range(n):
        np.testing.assert_array_equal(net.weights[i].data, golden[f"mlp_w{i}_after3"])
        np.testing.assert_array_equal(net.biases[i].data, golden[f"mlp_b{i}_after3"])


def test_spiral_steps_bitexact_vs_reference_fixture(golden):
    sp = W.spiral()
    net = A.Mlp(sp["weights"], sp["biases"])
    x = A.T(sp["x"])
    losses = [net.step(x, sp["targets"], 1.0) for _ in range(5)]
    np.testing.assert_array_equal(np.asarray(losses, dtype=np.float32), golden["spiral_losses"])
    for i in range(2):
        np.testing.assert_array_equal(net.weights[i].data, golden[f"spiral_w{i}_after5"])


def test_live_oracle_vs_reference(reference):
    """Fresh random inputs (not the fixtures) through both implementations."""
    rng = np.random.default_rng(99)
    for (m, k, n) in [(33, 700, 47), (5, 1030, 9), (70, 256, 13)]:
        for ta in (0, 1):
            for tb in (0, 1):
                a = rng.standard_normal((k, m) if ta else (m, k)).astype(np.float32)
                b = rng.standard_normal((n, k) if tb else (k, n)).astype(np.float32)
                np.testing.assert_array_equal(K.matmul2d(a, b, bool(ta), bool(tb)),
                                              reference.matmul2d(a, b, bool(ta), bool(tb)))
    x = rng.standard_normal((40, 3, 50)).astype(np.float32)
    y = rng.standard_normal((3, 1)).astype(np.float32)
    for op in (K.ADD, K.SUB, K.MUL, K.DIV):
        np.testing.assert_array_equal(K.binary(x, y, op), reference.binary(x, y, op))
    for op in (K.NEG, K.RELU, K.SIGMOID, K.RELU_GRAD, K.EXP):
        np.testing.assert_array_equal(K.unary(x, op), reference.unary(x, op))
    np.testing.assert_array_equal(K.unary(np.abs(x) + 0.1, K.LOG), reference.unary(np.abs(x) + 0.1, K.LOG))
    xe = W.xent(rows=300, classes=37, seed=11)
    logits = A.T(xe["logits"], True)
    loss = A.cross_entropy(logits, xe["targets"])
    loss.backward()
    rl, rg, ra = reference.cross_entropy(xe["logits"], xe["targets"])
    assert loss.data == rl
    np.testing.assert_array_equal(logits.grad.data, rg)


# --- 3. closed forms ---------------------------------------------------------

def softmax64(x):
    x = x.astype(np.float64)
    e = np.exp(x - x.max(axis=1, keepdims=True))
    return e / e.sum(axis=1, keepdims=True)


@pytest.mark.parametrize("m,k,n", [(65, 300, 95), (9, 257, 13), (1, 300, 60)])
def test_gemm_against_float64(m, k, n):
    for ta in (0, 1):
        for tb in (0, 1):
            a, b = gemm_inputs(m, k, n, ta, tb)
            ref = (a.T if ta else a).astype(np.float64) @ (b.T if tb else b).astype(np.float64)
            np.testing.assert_allclose(K.matmul2d(a, b, bool(ta), bool(tb)), ref, rtol=1e-4, atol=1e-4 * np.sqrt(k))


def test_reductions_against_float64():
    x = np.random.default_rng(5).normal(size=(64, 50, 33)).astype(np.float32)
    for axis in (0, 1, 2):
        np.testing.assert_allclose(K.reduce_axis(x, axis, K.SUM), x.astype(np.float64).sum(axis), rtol=1e-6, atol=1e-6)
        np.testing.assert_array_equal(K.reduce_axis(x, axis, K.MAX), x.max(axis))
        np.testing.assert_array_equal(K.reduce_axis(x, axis, K.ARGMAX), x.argmax(axis))
    s = sum_input()
    assert np.isclose(K.sum_all(s), s.astype(np.float64).sum(), rtol=1e-7, atol=1e-4)


def test_argmax_nan_semantics_closed_form():
    """A NaN first element wins (nothing compares greater); a later NaN never replaces."""
    x = np.array([[np.nan, 1.0, 5.0], [1.0, np.nan, 5.0], [3.0, np.nan, 2.0], [-np.inf, -np.inf, -np.inf]],
                 dtype=np.float32)
    np.testing.assert_array_equal(K.reduce_axis(x, 1, K.ARGMAX), [0, 2, 0, 0])
    got = K.reduce_axis(x, 1, K.MAX)
    assert np.isnan(got[0]) and got[1] == 5 and got[2] == 3 and got[3] == -np.inf


def test_cross_entropy_against_torch_and_closed_form():
    torch = pytest.importorskip("torch")
    xe = W.xent(rows=512, classes=100, seed=3)
    logits = A.T(xe["logits"], True)
    loss = A.cross_entropy(logits, xe["targets"])
    loss.backward()
    tt = torch.tensor(xe["logits"], dtype=torch.float64, requires_grad=True)
    ref = torch.nn.functional.cross_entropy(tt, torch.tensor(xe["targets"]))
    ref.backward()
    assert np.isclose(float(loss.data), ref.item(), rtol=1e-6)
    np.testing.assert_allclose(logits.grad.data, tt.grad.numpy(), rtol=1e-4, atol=1e-7)
    closed = softmax64(xe["logits"])
    closed[np.arange(512), xe["targets"]] -= 1.0
    np.testing.assert_allclose(logits.grad.data, closed / 512, rtol=1e-4, atol=1e-7)


def test_activation_backward_closed_form():
    act = W.activation(rows=32, cols=48)
    x, bias, dy = (act[k].astype(np.float64) for k in ("x", "bias", "dy"))
    z = np.maximum(x + bias, 0)
    s = 1 / (1 + np.exp(-z))
    e = np.exp(0.1 * x)
    dz = dy * e * s * (1 - s) * (x + bias > 0)
    dx_ref = dz + dy * s * e * 0.1
    tx, tb = A.T(act["x"], True), A.T(act["bias"], True)
    y = A.sigmoid(A.relu(tx + tb)) * A.exp(tx * 0.1)
    y.backward(A.T(act["dy"]))
    np.testing.assert_allclose(tx.grad.data, dx_ref, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(tb.grad.data, dz.sum(axis=0, keepdims=True), rtol=1e-5, atol=1e-5)


def test_mlp_gradients_closed_form():
    m = W.mlp(batch=48, dims=(20, 30, 25, 7), seed=4)
    net = A.Mlp(m["weights"], m["biases"])
    loss = A.cross_entropy(net.logits(A.T(m["x"])), m["targets"])
    loss.backward()
    hs = [m["x"].astype(np.float64)]
    zs = []
    for i, (w, b) in enumerate(zip(m["weights"], m["biases"])):
        z = hs[-1] @ w.astype(np.float64) + b
        zs.append(z)
        hs.append(np.maximum(z, 0) if i < 2 else z)
    g = softmax64(zs[-1])
    g[np.arange(48), m["targets"]] -= 1
    g /= 48
    for i in (2, 1, 0):
        np.testing.assert_allclose(net.weights[i].grad.data, hs[i].T @ g, rtol=1e-4, atol=1e-6)
        np.testing.assert_allclose(net.biases[i].grad.data, g.sum(0), rtol=1e-4, atol=1e-6)
        g = (g @ m["weights"][i].astype(np.float64).T) * (zs[i - 1] > 0) if i else None


# --- 4. planted mistakes must be caught --------------------------------------

def test_planted_transposed_operand_is_caught():
    a, b = gemm_inputs(65, 300, 95, 0, 1)
    good = a.astype(np.float64) @ b.T.astype(np.float64)
    wrong = K.matmul2d(np.ascontiguousarray(a), np.ascontiguousarray(b.T.reshape(95, 300)), False, True)
    with pytest.raises(AssertionError):
        np.testing.assert_allclose(wrong, good, rtol=1e-4, atol=1e-4 * np.sqrt(300))


def test_planted_missing_batch_scale_is_caught():
    xe = W.xent(rows=64, classes=10, seed=1)
    closed = softmax64(xe["logits"])
    closed[np.arange(64), xe["targets"]] -= 1.0
    logits = A.T(xe["logits"], True)
    A.cross_entropy(logits, xe["targets"]).backward()
    with pytest.raises(AssertionError):
        np.testing.assert_allclose(logits.grad.data * 64, closed / 64, rtol=1e-4, atol=1e-7)


def test_planted_last_wins_argmax_is_caught(known):
    x = np.asarray(known["argmax_ties"]["x"], dtype=np.float32)
    last_wins = x.shape[1] - 1 - np.argmax(x[:, ::-1], axis=1)
    assert not np.array_equal(last_wins, known["argmax_ties"]["argmax1"])
    np.testing.assert_array_equal(K.reduce_axis(x, 1, K.ARGMAX), known["argmax_ties"]["argmax1"])


def test_planted_float32_accumulation_is_caught(golden):
    s = sum_input()
    f32_sum = np.float32(0)
    for chunk in np.array_split(s, 64):
        f32_sum = np.float32(f32_sum + np.add.reduce(chunk, dtype=np.float32))
    naive = np.cumsum(s, dtype=np.float32)[-1]
    assert naive != golden["sum_out"] or f32_sum != golden["sum_out"]
