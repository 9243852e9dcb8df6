"""ORACLE — test infrastructure only.

A restatement of the reference's reverse-mode engine and backward rules over
the C oracle kernels, so composite results (cross-entropy, activation chains,
MLP train steps) can be checked without the product. It follows:
  * the engine: src/tensor.cpp:251-301 (DFS topological order over
    grad_fn parents, reverse walk, gradient map with early erase, .grad on
    leaves and retain_grad nodes, accumulation with ``+``);
  * graph recording: src/autograd.cpp:15-48;
  * sum_to_shape / broadcast_to: src/autograd.cpp:50-91;
  * the op rules: src/ops.cpp:98-413; Linear/cross_entropy/sgd: src/nn.cpp.

Values are numpy float32 arrays; every arithmetic step calls the C oracle
kernel the reference would run, in the reference's order, so the result is
bit-identical to the reference library on the same inputs.
"""

from __future__ import annotations

import contextlib

import numpy as np

from oracle import kernels as K

_grad_enabled = True


@contextlib.contextmanager
def no_grad():
    """NoGradGuard (src/autograd.cpp:15-19)."""
    global _grad_enabled
    previous = _grad_enabled
    _grad_enabled = False
    try:
        yield
    finally:
        _grad_enabled = previous


class GradFn:
    __slots__ = ("parents", "backward")

    def __init__(self, parents, backward):
        self.parents = parents
        self.backward = backward


class T:
    """A tensor node: float32 value plus autograd state (detail/tensor_impl.hpp:20-31)."""

    __slots__ = ("data", "requires_grad", "leaf", "retains_grad", "grad_fn", "grad")

    def __init__(self, data, requires_grad=False):
        self.data = K.f32(data)
        self.requires_grad = requires_grad
        self.leaf = True
        self.retains_grad = False
        self.grad_fn = None
        self.grad = None

    @property
    def shape(self):
        return self.data.shape

    def detach(self):
        return T(self.data)

    def retain_grad(self):
        if not self.requires_grad:
            raise RuntimeError("retain_grad() requires a tensor that requires gradients")
        if not self.leaf:
            self.retains_grad = True

    # operators (src/tensor.cpp:318-330): a float operand becomes a scalar tensor
    def __add__(self, o): return add(self, _t(o))
    def __radd__(self, o): return add(_t(o), self)
    def __sub__(self, o): return sub(self, _t(o))
    def __rsub__(self, o): return sub(_t(o), self)
    def __mul__(self, o): return mul(self, _t(o))
    def __rmul__(self, o): return mul(_t(o), self)
    def __truediv__(self, o): return div(self, _t(o))
    def __rtruediv__(self, o): return div(_t(o), self)
    def __neg__(self): return neg(self)
    def __matmul__(self, o): return matmul(self, o)

    def backward(self, gradient=None):
        backward(self, gradient)


def _t(x):
    return x if isinstance(x, T) else T(np.float32(x))


def attach(out: T, parents, fn) -> T:
    """attach_grad_fn (src/autograd.cpp:36-48)."""
    if not _grad_enabled:
        return out
    if not any(p.requires_grad for p in parents):
        return out
    out.grad_fn = GradFn(list(parents), fn)
    out.requires_grad = True
    out.leaf = False
    return out


def backward(root: T, gradient: T | None = None) -> None:
    """Tensor::backward (src/tensor.cpp:244-301)."""
    if gradient is None:
        if root.data.size != 1:
            raise RuntimeError("backward() without a gradient requires a scalar tensor")
        gradient = T(np.ones(root.shape, dtype=np.float32))
    if not root.requires_grad:
        raise RuntimeError("cannot call backward on a tensor without gradients")
    order, visited = [], set()

    def visit(node):
        if id(node) in visited:
            return
        visited.add(id(node))
        if node.grad_fn is not None:
            for parent in node.grad_fn.parents:
                visit(parent)
        order.append(node)

    visit(root)
    with no_grad():
        grads = {id(root): gradient.detach()}
        for node in reversed(order):
            upstream = grads.pop(id(node), None)
            if upstream is None:
                continue
            if node.requires_grad and (node.leaf or node.retains_grad):
                node.grad = upstream.detach() if node.grad is None else (node.grad + upstream).detach()
            if node.grad_fn is None:
                continue
            parent_grads = node.grad_fn.backward(upstream)
            for parent, g in zip(node.grad_fn.parents, parent_grads):
                if not parent.requires_grad:
                    continue
                if id(parent) in grads:
                    grads[id(parent)] = grads[id(parent)] + g
                else:
                    grads[id(parent)] = g.detach()


def sum_to_shape(g: T, target) -> T:
    """src/autograd.cpp:50-72: sum each stretched or leading axis (keepdim), in axis order."""
    target = tuple(target)
    if g.shape == target:
        return g
    lead = len(g.shape) - len(target)
    current = g
    for axis in range(len(g.shape)):
        tdim = 1 if axis < lead else target[axis - lead]
        if tdim == g.shape[axis]:
            continue
        current = sum_axis(current, axis, keepdim=True)
    return reshape(current, target)


def broadcast_to(v: T, target) -> T:
    """src/autograd.cpp:74-91: binary add of a scalar zero with an explicit
    output shape (so -0.0 becomes +0.0, as in the reference)."""
    target = tuple(target)
    if v.shape == target:
        return v
    K.broadcast_shape(v.shape, target)  # validates compatibility
    return T(K.binary(v.data, np.float32(0.0), K.ADD, out_shape=target))


def _binary(a: T, b: T, op: int) -> T:
    return T(K.binary(a.data, b.data, op))


def add(a: T, b: T) -> T:
    out = _binary(a, b, K.ADD)
    sa, sb, na, nb = a.shape, b.shape, a.requires_grad, b.requires_grad
    return attach(out, [a, b], lambda g: [sum_to_shape(g, sa) if na else None,
                                          sum_to_shape(g, sb) if nb else None])


def sub(a: T, b: T) -> T:
    out = _binary(a, b, K.SUB)
    sa, sb, na, nb = a.shape, b.shape, a.requires_grad, b.requires_grad
    return attach(out, [a, b], lambda g: [sum_to_shape(g, sa) if na else None,
                                          sum_to_shape(neg(g), sb) if nb else None])


def mul(a: T, b: T) -> T:
    out = _binary(a, b, K.MUL)
    sa, sb, na, nb = a.shape, b.shape, a.requires_grad, b.requires_grad
    ad, bd = a.detach(), b.detach()
    return attach(out, [a, b], lambda g: [sum_to_shape(mul(g, bd), sa) if na else None,
                                          sum_to_shape(mul(g, ad), sb) if nb else None])


def div(a: T, b: T) -> T:
    out = _binary(a, b, K.DIV)
    sa, sb, na, nb = a.shape, b.shape, a.requires_grad, b.requires_grad
    ad, bd = a.detach(), b.detach()

    def rule(g):
        ga = sum_to_shape(div(g, bd), sa) if na else None
        gb = sum_to_shape(div(neg(mul(g, ad)), mul(bd, bd)), sb) if nb else None
        return [ga, gb]

    return attach(out, [a, b], rule)


def neg(a: T) -> T:
    out = T(K.unary(a.data, K.NEG))
    return attach(out, [a], lambda g: [neg(g)])


def _matmul_kernel(a: T, b: T, ta: bool, tb: bool) -> T:
    return T(K.matmul(a.data, b.data, ta, tb))


def matmul(a: T, b: T) -> T:
    """src/ops.cpp:244-262: dA = dY @ B^T, dB = A^T @ dY, then sum_to_shape."""
    out = _matmul_kernel(a, b, False, False)
    sa, sb, na, nb = a.shape, b.shape, a.requires_grad, b.requires_grad
    ad, bd = a.detach(), b.detach()
    return attach(out, [a, b], lambda g: [
        sum_to_shape(_matmul_kernel(g, bd, False, True), sa) if na else None,
        sum_to_shape(_matmul_kernel(ad, g, True, False), sb) if nb else None])


def transpose(a: T) -> T:
    out = T(K.transpose_last2(a.data))
    return attach(out, [a], lambda g: [transpose(g)])


def reshape(a: T, shape) -> T:
    shape = tuple(shape)
    out = T(a.data.reshape(shape))
    original = a.shape
    return attach(out, [a], lambda g: [reshape(g, original)])


def sum_all(a: T) -> T:
    out = T(K.sum_all(a.data))
    shape = a.shape
    return attach(out, [a], lambda g: [broadcast_to(g, shape)])


def sum_axis(a: T, axis: int, keepdim=False) -> T:
    _, _, _, _, kept, removed = K.split_axis(a.shape, axis)
    out = T(K.reduce_axis(a.data, axis, K.SUM, keepdim))
    shape = a.shape
    return attach(out, [a], lambda g: [broadcast_to(reshape(g, kept), shape)])


def mean_all(a: T) -> T:
    if a.data.size == 0:
        raise ValueError("mean of an empty tensor is undefined")
    return sum_all(a) / float(a.data.size)


def mean_axis(a: T, axis: int, keepdim=False) -> T:
    _, _, length, _, _, _ = K.split_axis(a.shape, axis)
    if length == 0:
        raise ValueError("mean over an empty axis is undefined")
    return sum_axis(a, axis, keepdim) / float(length)


def max_axis(a: T, axis: int, keepdim=False) -> T:
    """src/ops.cpp:323-347: gradient goes to the first maximum (scatter)."""
    ax, _, _, _, kept, removed = K.split_axis(a.shape, axis)
    out = T(K.reduce_axis(a.data, axis, K.MAX, keepdim))
    if not _grad_enabled or not a.requires_grad:
        return out
    idx = K.reduce_axis(a.data, axis, K.ARGMAX, keepdim)
    shape = a.shape
    return attach(out, [a], lambda g: [T(K.scatter_axis(g.data, idx, shape, ax))])


def max_all(a: T) -> T:
    if a.data.size == 0:
        raise ValueError("max of an empty tensor is undefined")
    return max_axis(reshape(a, (a.data.size,)), 0)


def argmax(a: T, axis: int, keepdim=False) -> T:
    return T(K.reduce_axis(a.data, axis, K.ARGMAX, keepdim))


def exp(a: T) -> T:
    out = T(K.unary(a.data, K.EXP))
    saved = out.detach()
    return attach(out, [a], lambda g: [mul(g, saved)])


def log(a: T) -> T:
    out = T(K.unary(a.data, K.LOG))
    saved = a.detach()
    return attach(out, [a], lambda g: [div(g, saved)])


def relu(a: T) -> T:
    out = T(K.unary(a.data, K.RELU))
    saved = a.detach()
    return attach(out, [a], lambda g: [mul(g, T(K.unary(saved.data, K.RELU_GRAD)))])


def sigmoid(a: T) -> T:
    out = T(K.unary(a.data, K.SIGMOID))
    y = out.detach()
    return attach(out, [a], lambda g: [mul(mul(g, y), sub(T(np.float32(1.0)), y))])


def log_softmax(a: T, axis=-1) -> T:
    """src/ops.cpp:378-384."""
    shifted = sub(a, max_axis(a.detach(), axis, True))
    return sub(shifted, log(sum_axis(exp(shifted), axis, True)))


def softmax(a: T, axis=-1) -> T:
    return exp(log_softmax(a, axis))


def cross_entropy(logits: T, targets) -> T:
    """src/nn.cpp:31-53: -(log_softmax(logits, 1) * one_hot).sum() / batch."""
    if logits.data.ndim != 2:
        raise ValueError("cross_entropy expects [batch, classes] logits")
    batch, classes = logits.shape
    targets = [int(t) for t in targets]
    if len(targets) != batch:
        raise ValueError("cross_entropy target count does not match the batch")
    if batch == 0:
        raise ValueError("cross_entropy of an empty batch is undefined")
    mask = np.zeros((batch, classes), dtype=np.float32)
    for row, t in enumerate(targets):
        if t >= classes or t < 0:
            raise IndexError(f"target class {t} is out of range for {classes} classes")
    mask[np.arange(batch), targets] = 1.0
    return div(neg(sum_all(mul(log_softmax(logits, 1), T(mask)))), T(np.float32(batch)))


def sgd_step(params, lr: float) -> None:
    """src/nn.cpp:55-76."""
    for p in params:
        if p.grad is None:
            continue
        K.sgd_(p.data, p.grad.data, lr)


def zero_grad(params) -> None:
    for p in params:
        p.grad = None


class Mlp:
    """x @ W + b layers (W stored [in, out], src/nn.cpp:14-24) with ReLU between."""

    def __init__(self, weights, biases):
        self.weights = [T(w, requires_grad=True) for w in weights]
        self.biases = [T(b, requires_grad=True) for b in biases]

    def params(self):
        out = []
        for w, b in zip(self.weights, self.biases):
            out += [w, b]
        return out

    def logits(self, x: T) -> T:
        h = x
        for i, (w, b) in enumerate(zip(self.weights, self.biases)):
            h = add(matmul(h, w), b)
            if i + 1 < len(self.weights):
                h = relu(h)
        return h

    def step(self, x: T, targets, lr: float) -> float:
        """One train step as in benchmarks/train_benchmark.py:43-48."""
        loss = cross_entropy(self.logits(x), targets)
        loss.backward()
        sgd_step(self.params(), lr)
        zero_grad(self.params())
        return float(loss.data)
