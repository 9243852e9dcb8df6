"""Random programs on the hip device, run with deferred products on and off.

Each program builds MLP-like layers (products, row-bias adds, ReLU or
sigmoid) over random shapes (1 to 257 wide, up to 4096 rows), takes a sum or
cross-entropy loss, runs backward and SGD, reads intermediates before and
after the parameter updates, and keeps products recorded before later
updates to read at the end. Deferred products must give every value read the
same bits as eager ones (same kernels, same order), including products whose
operands were updated in place while they waited.
"""

import numpy as np
import pytest

import vectorcore_amd as vc

pytestmark = pytest.mark.gpu

DIMS = [1, 3, 17, 64, 130, 257]


def program(seed):
    """A list of ops; tensors are named by their index in the order they are made."""
    rng = np.random.default_rng(seed)
    ops, shapes, params = [], [], []

    def make(op, shape):
        ops.append(op)
        shapes.append(tuple(shape))
        return len(shapes) - 1

    def leaf(shape, param):
        idx = make(("new", tuple(shape), int(rng.integers(0, 2**31)), param), shape)
        if param:
            params.append(idx)
        return idx

    x = leaf((int(rng.choice(DIMS + [4096])), int(rng.choice(DIMS))), False)
    for _ in range(int(rng.integers(1, 4))):  # train steps
        cur = x
        for _ in range(int(rng.integers(1, 4))):  # layers
            width = int(rng.choice(DIMS))
            w = leaf((shapes[cur][1], width), True)
            cur = make(("matmul", cur, w), (shapes[cur][0], width))
            if rng.random() < 0.7:
                cur = make(("add", cur, leaf((width,), True)), shapes[cur])
            r = rng.random()
            if r < 0.6:
                cur = make(("relu", cur), shapes[cur])
            elif r < 0.7:
                cur = make(("sigmoid", cur), shapes[cur])
            if rng.random() < 0.3:
                ops.append(("read", cur))
        if rng.random() < 0.5:
            loss = make(("ce", cur, int(rng.integers(0, 2**31))), ())
        else:
            loss = make(("sum", cur), ())
        if rng.random() < 0.5:
            ops.append(("read", loss))
        ops.append(("backward", loss))
        if rng.random() < 0.5:
            ops.append(("read_grads",))
        ops.append(("sgd", float(rng.choice([0.01, 0.1, 1.0]))))
        if rng.random() < 0.7:
            ops.append(("read", cur))  # recorded before the update, read after it
        ops.append(("zero_grad",))
        if rng.random() < 0.5:  # a product recorded now, read only after the later updates
            w = params[int(rng.integers(0, len(params)))]
            if len(shapes[w]) == 2 and shapes[w][0] == shapes[x][1]:
                ops.append(("hold", make(("matmul", x, w), (shapes[x][0], shapes[w][1]))))
    ops.append(("read_params",))
    return ops


def run(ops, defer):
    vc.hip_defer_products(defer)
    t, params, reads, held = [], [], [], []
    for op in ops:
        kind = op[0]
        if kind == "new":
            _, shape, seed, param = op
            r = np.random.default_rng(seed)
            data = (r.standard_normal(shape) / np.sqrt(max(1, shape[0]))).astype(np.float32)
            v = vc.Tensor(data, requires_grad=param, device="hip")
            t.append(v)
            if param:
                params.append(v)
        elif kind == "matmul":
            t.append(t[op[1]] @ t[op[2]])
        elif kind == "add":
            t.append(t[op[1]] + t[op[2]])
        elif kind == "relu":
            t.append(t[op[1]].relu())
        elif kind == "sigmoid":
            t.append(t[op[1]].sigmoid())
        elif kind == "ce":
            logits = t[op[1]]
            r = np.random.default_rng(op[2])
            targets = [int(v) for v in r.integers(0, logits.shape[1], size=logits.shape[0])]
            t.append(vc.cross_entropy(logits, targets))
        elif kind == "sum":
            t.append(t[op[1]].sum())
        elif kind == "read":
            reads.append(np.array(t[op[1]].numpy(), copy=True))
        elif kind == "backward":
            t[op[1]].backward()
        elif kind == "read_grads":
            for p in params:
                if p.grad is not None:
                    reads.append(np.array(p.grad.numpy(), copy=True))
        elif kind == "sgd":
            vc.sgd_step(params, op[1])
        elif kind == "zero_grad":
            vc.zero_grad(params)
        elif kind == "hold":
            held.append(t[op[1]])
        elif kind == "read_params":
            for h in held:
                reads.append(np.array(h.numpy(), copy=True))
            for p in params:
                reads.append(np.array(p.numpy(), copy=True))
    vc.synchronize()
    return reads


@pytest.fixture(autouse=True)
def restore_deferred_mode():
    previous = vc.hip_defer_products()
    yield
    vc.hip_defer_products(previous)


@pytest.mark.parametrize("first", [0, 20])
def test_random_programs_read_the_same_bits_with_and_without_deferred_products(first):
    assert vc.hip_available()
    for seed in range(first, first + 20):
        ops = program(seed)
        deferred, eager = run(ops, True), run(ops, False)
        assert len(deferred) == len(eager), f"seed {seed}"
        for i, (x, y) in enumerate(zip(deferred, eager)):
            assert x.shape == y.shape and np.array_equal(x.view(np.uint32), y.view(np.uint32)), \
                f"seed {seed}: read {i} differs"
