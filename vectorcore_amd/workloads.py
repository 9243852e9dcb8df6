"""Seeded synthetic inputs for the backward-pass workloads.

Every input is drawn from NumPy's PCG64 ``default_rng(seed)`` and converted to
float32, so the GPU run, the parity checks and the CPU baseline all see the
same bytes. Shapes default to the full workload sizes; tests pass smaller ones.

Workloads (seed in brackets):
  spiral   [0] 3 classes x 100 points, 2 -> 64 -> 3 MLP, SGD lr 1.0
  bmm      [1] batched matmul backward, A, B, dC [8, 1024, 1024] ~ N(0, 1)
  act      [2] y = sigmoid(relu(x + bias)) * exp(0.1 x), x [4096, 4096]
  xent     [3] softmax cross-entropy + argmax, logits [32768, 1000] ~ N(0, 2^2)
  mlp      [4] 8192 x 1024 -> 4096 -> 4096 -> 1000 MLP train step, SGD lr 0.01
  mnist_shaped [0] 256 x 784 -> 256 -> 10 MLP train step, SGD lr 0.1 (the
           reference's own train benchmark generator)
"""

from __future__ import annotations

import numpy as np


def _normal(rng, shape, scale=1.0):
    x = rng.standard_normal(size=shape, dtype=np.float32)
    if scale != 1.0:
        x *= np.float32(scale)
    return x


def linear_weights(rng, dims):
    """W_i [in, out] ~ U(-1/sqrt(in), 1/sqrt(in)); biases zero."""
    weights, biases = [], []
    for fan_in, fan_out in zip(dims[:-1], dims[1:]):
        bound = 1.0 / np.sqrt(fan_in)
        weights.append(rng.uniform(-bound, bound, size=(fan_in, fan_out)).astype(np.float32))
        biases.append(np.zeros(fan_out, dtype=np.float32))
    return weights, biases


def spiral(points=100, classes=3, hidden=64, seed=0):
    """Point = r (sin t, cos t), r = linspace(0, 1, points), t = 4k + 4r + N(0, 0.2^2)."""
    rng = np.random.default_rng(seed)
    feats, labels = [], []
    r = np.linspace(0.0, 1.0, points)
    for k in range(classes):
        theta = 4.0 * k + 4.0 * r + rng.normal(0.0, 0.2, size=points)
        feats.append(np.stack([r * np.sin(theta), r * np.cos(theta)], axis=1))
        labels += [k] * points
    x = np.concatenate(feats).astype(np.float32)
    weights, biases = linear_weights(rng, [2, hidden, classes])
    return dict(x=x, targets=np.asarray(labels, dtype=np.int64), weights=weights, biases=biases, lr=1.0)


def bmm(batch=8, m=1024, k=1024, n=1024, seed=1):
    rng = np.random.default_rng(seed)
    a = _normal(rng, (batch, m, k))
    b = _normal(rng, (batch, k, n))
    dc = _normal(rng, (batch, m, n))
    b_shared = _normal(rng, (1, k, n))
    return dict(a=a, b=b, dc=dc, b_shared=b_shared)


def activation(rows=4096, cols=4096, seed=2):
    rng = np.random.default_rng(seed)
    return dict(x=_normal(rng, (rows, cols)), bias=_normal(rng, (1, cols)), dy=_normal(rng, (rows, cols)))


def xent(rows=32768, classes=1000, seed=3):
    rng = np.random.default_rng(seed)
    logits = _normal(rng, (rows, classes), scale=2.0)
    targets = rng.integers(0, classes, size=rows, dtype=np.int64)
    return dict(logits=logits, targets=targets)


def mlp(batch=8192, dims=(1024, 4096, 4096, 1000), seed=4):
    rng = np.random.default_rng(seed)
    x = _normal(rng, (batch, dims[0]))
    targets = rng.integers(0, dims[-1], size=batch, dtype=np.int64)
    weights, biases = linear_weights(rng, list(dims))
    return dict(x=x, targets=targets, weights=weights, biases=biases, lr=0.01)


def mnist_shaped(batch=256, features=784, hidden=256, classes=10, seed=0):
    """The reference's second train benchmark (benchmarks/train_benchmark.py:
    23-26, 29-45): x ~ N(0, 1) [batch, features], uniform int targets, then
    each parameter drawn as N(0, 1) * scale in float64 and cast (W1 scale
    features^-0.5, b1 0, W2 scale hidden^-0.5, b2 0), in that order; SGD lr 0.1."""
    rng = np.random.default_rng(seed)
    x = rng.normal(size=(batch, features)).astype(np.float32)
    targets = rng.integers(0, classes, size=batch)

    def param(shape, scale):
        return (rng.normal(size=shape) * scale).astype(np.float32)

    w1, b1 = param((features, hidden), features ** -0.5), param((hidden,), 0.0)
    w2, b2 = param((hidden, classes), hidden ** -0.5), param((classes,), 0.0)
    return dict(x=x, targets=targets.astype(np.int64), weights=[w1, w2], biases=[b1, b2], lr=0.1)


def mlp_gemm_flops(batch, dims):
    """Algorithmic GEMM FLOPs of one train step: forward x@W per layer, and in
    backward dH = dY @ W^T for every layer but the first plus dW = H^T @ dY
    for every layer (the first layer's input needs no gradient)."""
    fwd = sum(2 * batch * i * o for i, o in zip(dims[:-1], dims[1:]))
    bwd_dw = sum(2 * batch * i * o for i, o in zip(dims[:-1], dims[1:]))
    bwd_dh = sum(2 * batch * i * o for i, o in zip(dims[1:-1], dims[2:]))
    return fwd, bwd_dw + bwd_dh
