"""Fused elementwise programs (vc_hip_map) and the backward pass that builds them.

The ABI tests evaluate random straight-line programs with numpy in float32
(whose +, -, *, / are the IEEE operations the kernel performs, so the bits
must agree) and column sums in float64. The engine tests run backward passes
with fusion on and off (hip_fuse_elementwise) and on the cpu device: the
gradients of fused chains must be the same bits as the eager kernels', and a
chain must become one program.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

import vectorcore_amd as vc
from vectorcore_amd import cabi as C

pytestmark = pytest.mark.gpu

OPS = (C.MAP_ADD, C.MAP_SUB, C.MAP_MUL, C.MAP_DIV, C.MAP_NEG, C.MAP_STEP)


def eval_program(inputs, constants, code):
    """numpy restatement of the interpreter: float32 slots, one op each."""
    slots = [None] * C.MAP_SLOTS
    for j, x in enumerate(inputs):
        slots[j] = x.astype(np.float32)
    for c, v in enumerate(constants):
        slots[len(inputs) + c] = np.float32(v)
    with np.errstate(all="ignore"):
        for op, a, b, d in code:
            x, y = slots[a], slots[b]
            if op == C.MAP_ADD:
                r = x + y
            elif op == C.MAP_SUB:
                r = x - y
            elif op == C.MAP_MUL:
                r = x * y
            elif op == C.MAP_DIV:
                r = x / y
            elif op == C.MAP_NEG:
                r = -x
            else:
                r = np.where(x > 0, np.float32(1), np.float32(0))
            slots[d] = np.broadcast_to(np.asarray(r, dtype=np.float32), inputs[0].shape).copy()
    return slots


def random_program(rng, n_in, n_const, n_code):
    """A valid program: reads only written slots, never writes a constant."""
    first_temp = n_in + n_const
    written = set(range(first_temp))
    writable = [s for s in range(C.MAP_SLOTS) if s < n_in or s >= first_temp]
    code = []
    for _ in range(n_code):
        op = int(rng.choice(OPS))
        a, b = (int(rng.choice(sorted(written))) for _ in range(2))
        if op in (C.MAP_NEG, C.MAP_STEP):
            b = a
        d = int(rng.choice(writable))
        code.append((op, a, b, d))
        written.add(d)
    temps = sorted(written - set(range(n_in, first_temp)))
    return code, temps


def run(inputs, constants, code, out_slots, sum_slots, rows, cols, offset=0):
    """Uploads inputs (each shifted by `offset` elements), runs the program, downloads."""
    bufs = []
    for x in inputs:
        flat = np.concatenate([np.zeros(offset, np.float32), x.ravel()])
        bufs.append(C.Buffer.of(flat))
    outs = [C.Buffer((offset + rows * cols,)) for _ in out_slots]
    sums = [C.Buffer((max(cols, 1),)) for _ in sum_slots]
    p = C.map_program([b.ptr + 4 * offset for b in bufs], constants, code,
                      [(o.ptr + 4 * offset, s) for o, s in zip(outs, out_slots)],
                      [(o.ptr, s) for o, s in zip(sums, sum_slots)], rows, cols)
    C.check(C.lib().vc_hip_map(ctypes.byref(p)))
    got = [o.numpy()[offset:].reshape(rows, cols) for o in outs]
    got_sums = [o.numpy()[:cols] for o in sums]
    return got, got_sums


def bits(x):
    return np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)


def assert_same_values(got, want):
    """Bit equality, except that a NaN's payload is free (0/0 and inf-inf
    give the host's and the device's default NaNs, which differ in sign)."""
    got, want = np.asarray(got, np.float32), np.asarray(want, np.float32)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
    keep = ~np.isnan(want)
    np.testing.assert_array_equal(bits(got[keep]), bits(want[keep]))


@pytest.mark.parametrize("rows,cols,offset", [(1, 4096 * 4 + 3, 0), (1, 1001, 1), (37, 256, 0), (5, 7, 3)])
@pytest.mark.parametrize("seed", range(6))
def test_random_programs_bitexact(rows, cols, offset, seed):
    rng = np.random.default_rng(100 + seed)
    n_in = int(rng.integers(1, 9))
    n_const = int(rng.integers(0, min(8, 16 - n_in) + 1))
    n_code = int(rng.integers(1, 33)) if seed % 2 else int(rng.integers(1, 17))
    code, temps = random_program(rng, n_in, n_const, n_code)
    inputs = [rng.standard_normal((rows, cols)).astype(np.float32) for _ in range(n_in)]
    inputs[0][0, : min(cols, 4)] = [0.0, -0.0, np.inf, np.nan][: min(cols, 4)]
    constants = [float(np.float32(v)) for v in rng.standard_normal(n_const)]
    out_slots = [int(s) for s in rng.choice(temps, size=min(len(temps), 4), replace=False)]
    want = eval_program(inputs, constants, code)
    got, _ = run(inputs, constants, code, out_slots, [], rows, cols, offset)
    for g, s in zip(got, out_slots):
        assert_same_values(g, want[s])


# Vector and scalar loads, one to 2048 partial rows per column, and a row
# too wide for one column block's partial row count to matter (2, 300001).
@pytest.mark.parametrize("rows,cols", [(4096, 4096), (1000, 256), (37, 1000), (50, 130), (3, 64), (1, 5), (9, 1),
                                       (4000, 130), (2, 300001)])
def test_column_sums(rows, cols):
    rng = np.random.default_rng(rows * 7 + cols)
    inputs = [rng.standard_normal((rows, cols)).astype(np.float32) for _ in range(3)]
    # slot 3 = constant 0.5; t4 = x0 * x1; t5 = t4 + x2 * 0.5; sums of t4 and t5, output t5
    code = [(C.MAP_MUL, 0, 1, 4), (C.MAP_MUL, 2, 3, 5), (C.MAP_ADD, 4, 5, 5)]
    want = eval_program(inputs, [0.5], code)
    got, sums = run(inputs, [0.5], code, [5], [4, 5], rows, cols)
    np.testing.assert_array_equal(bits(got[0]), bits(want[5]))
    for s, slot in zip(sums, (4, 5)):
        exact = want[slot].astype(np.float64).sum(axis=0)
        np.testing.assert_allclose(s, exact, rtol=1e-6, atol=1e-6 * np.sqrt(rows))


def test_column_sums_are_deterministic():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((2048, 1000)).astype(np.float32)
    code = [(C.MAP_MUL, 0, 0, 1)]
    first = run([x], [], code, [], [1], 2048, 1000)[1][0]
    for _ in range(3):
        np.testing.assert_array_equal(bits(run([x], [], code, [], [1], 2048, 1000)[1][0]), bits(first))


def test_empty_column_sums_are_zero():
    x = C.Buffer((4,))
    s = C.Buffer.of(np.full(64, 7.0, np.float32))
    p = C.map_program([x.ptr], [], [(C.MAP_NEG, 0, 0, 1)], [], [(s.ptr, 1)], 0, 64)
    C.check(C.lib().vc_hip_map(ctypes.byref(p)))
    np.testing.assert_array_equal(s.numpy(), np.zeros(64, np.float32))


@pytest.mark.parametrize("bad,message", [
    (dict(code=[(C.MAP_ADD, 0, 5, 2)]), "before it is written"),
    (dict(code=[(C.MAP_ADD, 0, 0, 16)]), "out of range"),
    (dict(code=[(C.MAP_ADD, 0, 0, 1)], constants=[1.0]), "overwrites a constant"),
    (dict(code=[(9, 0, 0, 2)]), "unknown opcode"),
    (dict(outputs=[]), "nothing to compute"),
])
def test_invalid_programs_are_rejected(bad, message):
    x, y = C.Buffer((16,)), C.Buffer((16,))
    args = dict(inputs=[x.ptr], constants=[], code=[(C.MAP_NEG, 0, 0, 2)], outputs=[(y.ptr, 2)], sums=[],
                rows=4, cols=4)
    args.update(bad)
    if "outputs" in bad:
        args["outputs"] = bad["outputs"]
    p = C.map_program(**args)
    with pytest.raises(ValueError, match=message):
        C.check(C.lib().vc_hip_map(ctypes.byref(p)))


def test_too_many_inputs_are_rejected():
    bufs = [C.Buffer((4,)) for _ in range(9)]
    p = C.map_program([b.ptr for b in bufs[:8]], [], [(C.MAP_NEG, 0, 0, 8)], [(bufs[8].ptr, 8)], [], 1, 4)
    p.n_inputs = 9
    with pytest.raises(ValueError, match="1 to 8 inputs"):
        C.check(C.lib().vc_hip_map(ctypes.byref(p)))


# ---- the backward pass -----------------------------------------------------------


def T(a, device, grad=False):
    return vc.Tensor(np.ascontiguousarray(a, dtype=np.float32), requires_grad=grad, device=device)


def npy(t):
    return t.to("cpu").numpy()


@pytest.fixture
def fuse():
    previous = vc.hip_fuse_elementwise()
    yield vc.hip_fuse_elementwise
    vc.hip_fuse_elementwise(previous)


def activation_chain(device, xs, bs, dys, profile_labels=None):
    """y = sigmoid(relu(x + bias)) * exp(0.1 x); backward with dy."""
    x, bias = T(xs, device, True), T(bs, device, True)
    y = (x + bias).relu().sigmoid() * (x * 0.1).exp()
    if profile_labels is not None:
        vc.synchronize()
        vc.hip_profile_reset()
        vc.hip_profile(True)
    y.backward(T(dys, device))
    out = [npy(x.grad), npy(bias.grad)]
    if profile_labels is not None:
        vc.hip_profile(False)
        return out, vc.hip_profile_read()
    return out


def test_activation_chain_is_one_program(fuse):
    rng = np.random.default_rng(3)
    xs = rng.standard_normal((512, 1024)).astype(np.float32)
    bs = rng.standard_normal((1, 1024)).astype(np.float32)
    dys = rng.standard_normal((512, 1024)).astype(np.float32)
    fuse(True)
    (dx, db), prof = activation_chain("hip", xs, bs, dys, profile_labels=True)
    assert prof.get("fused_map_columns", {}).get("launches") == 1, prof
    assert prof.get("column_sum_combine", {}).get("launches") == 1, prof
    assert set(prof) == {"fused_map_columns", "column_sum_combine"}, prof
    fuse(False)
    dx_e, db_e = activation_chain("hip", xs, bs, dys)
    np.testing.assert_array_equal(bits(dx), bits(dx_e))
    np.testing.assert_allclose(db, db_e, rtol=1e-6, atol=1e-6)
    dx_c, db_c = activation_chain("cpu", xs, bs, dys)
    np.testing.assert_allclose(dx, dx_c, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(db, db_c, rtol=1e-4, atol=1e-4)


def random_graph(rng, depth):
    """A random program of elementwise ops over two leaves; returns a builder."""
    plan = []
    for _ in range(depth):
        plan.append((int(rng.integers(0, 9)), int(rng.integers(0, 1 << 30))))

    def build(a, b):
        vals = [a, b]
        for kind, pick in plan:
            u = vals[pick % len(vals)]
            v = vals[(pick >> 8) % len(vals)]
            if kind == 0:
                r = u + v
            elif kind == 1:
                r = u - v
            elif kind == 2:
                r = u * v
            elif kind == 3:
                r = u / (v * v + 1.0)
            elif kind == 4:
                r = u.relu()
            elif kind == 5:
                r = u.sigmoid()
            elif kind == 6:
                r = (u * 0.25).exp()
            elif kind == 7:
                r = (u * u + 1.0).log()
            else:
                r = -u
            vals.append(r)
        total = vals[-1]
        for v in vals[2:-1:3]:  # more than one consumer for some nodes
            total = total + v
        return total

    return build


@pytest.mark.parametrize("seed", range(12))
def test_random_elementwise_graphs(fuse, seed):
    rng = np.random.default_rng(seed)
    build = random_graph(rng, int(rng.integers(3, 14)))
    shape = (96, 130) if seed % 3 else (64, 256)
    av = rng.standard_normal(shape).astype(np.float32)
    bv = rng.standard_normal((1, shape[1]) if seed % 2 else shape).astype(np.float32)
    g = rng.standard_normal(shape).astype(np.float32)

    def grads(device):
        a, b = T(av, device, True), T(bv, device, True)
        out = build(a, b)
        out.backward(T(g, device))
        return [None if t.grad is None else npy(t.grad) for t in (a, b)]  # None: the output ignores t

    fuse(True)
    fused = grads("hip")
    fuse(False)
    eager = grads("hip")
    cpu = grads("cpu")
    for k in range(2):
        assert (fused[k] is None) == (eager[k] is None) == (cpu[k] is None)
        if fused[k] is None:
            continue
        if k == 1 and seed % 2:  # b is a row bias: its gradient is a column sum
            np.testing.assert_allclose(fused[k], eager[k], rtol=1e-5, atol=1e-5)
        else:
            assert_same_values(fused[k], eager[k])
        np.testing.assert_allclose(fused[k], cpu[k], rtol=1e-4, atol=1e-4)


def test_gradient_accumulation_and_retained_gradients(fuse):
    # A retained intermediate gradient and a leaf gradient accumulated over two
    # passes are read after the pass, so both are computed; the values match
    # the eager path's bits.
    rng = np.random.default_rng(9)
    xs = rng.standard_normal((128, 256)).astype(np.float32)

    def run_twice():
        x = T(xs, "hip", True)
        outs = []
        for _ in range(2):
            h = (x * 3.0).sigmoid()
            h.retain_grad()
            (h * x).backward(T(np.ones_like(xs), "hip"))
            outs.append(npy(h.grad))
        return outs + [npy(x.grad)]

    fuse(True)
    fused = run_twice()
    fuse(False)
    eager = run_twice()
    for f, e in zip(fused, eager):
        np.testing.assert_array_equal(bits(f), bits(e))
