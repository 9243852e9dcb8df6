"""Writes tests/golden/ref_vectors.npz from the reference VectorCore built from
its own sources (oracle/_ref, see oracle/build_oracle.py).

Each case stores its inputs and the reference's outputs, at sizes small enough
to commit. Run from the repository root:  python tests/golden/make_golden.py
"""

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import kernels as K  # noqa: E402
from vectorcore_amd import workloads as W  # noqa: E402

# m, k, n: small path, ragged edges, k over several 256-deep panels, m < 4,
# k = 1, n = 1 (after tests/python/test_performance_paths.py:26-33)
GEMM_SHAPES = [(3, 5, 7), (4, 33, 33), (9, 257, 13), (65, 300, 95), (127, 513, 129), (1, 300, 300),
               (300, 1, 60), (8, 3, 410), (200, 37, 1), (128, 64, 70)]


def gemm_inputs(m, k, n, ta, tb):
    """Inputs of one GEMM case, regenerated from a per-case seed (not stored)."""
    rng = np.random.default_rng(m * 1_000_003 + k * 1009 + n * 17 + ta * 2 + tb)
    a = rng.uniform(-1, 1, size=(k, m) if ta else (m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, size=(n, k) if tb else (k, n)).astype(np.float32)
    return a, b


def sum_input():
    return np.random.default_rng(77).standard_normal(300_001).astype(np.float32)


def main():
    if not K.Reference.available():
        raise SystemExit("oracle/_ref/libvc_ref.so is not built (python oracle/build_oracle.py)")
    ref = K.Reference()
    out = {}
    rng = np.random.default_rng(2024)
    for (m, k, n) in GEMM_SHAPES:
        for ta in (0, 1):
            for tb in (0, 1):
                a, b = gemm_inputs(m, k, n, ta, tb)
                out[f"gemm_{m}_{k}_{n}_{ta}{tb}_c"] = ref.matmul2d(a, b, bool(ta), bool(tb))
    # batched and batch-broadcast matmul backward (autograd through the reference)
    for name, ashape, bshape in [("bmm", (2, 33, 40), (2, 40, 24)), ("bmm_bcast", (3, 17, 19), (1, 19, 18)),
                                 ("bmm_bcast_rank", (2, 1, 9, 12), (3, 12, 5))]:
        a = rng.standard_normal(ashape).astype(np.float32)
        b = rng.standard_normal(bshape).astype(np.float32)
        y_shape = K.broadcast_shape(ashape[:-2], bshape[:-2]) + (ashape[-2], bshape[-1])
        dc = rng.standard_normal(y_shape).astype(np.float32)
        da, db = ref.matmul_backward(a, b, dc)
        out.update({f"{name}_a": a, f"{name}_b": b, f"{name}_dc": dc, f"{name}_da": da, f"{name}_db": db})
    # activation chain backward
    act = W.activation(rows=64, cols=96, seed=2)
    y, dx, dbias = ref.activation_backward(act["x"], act["bias"], act["dy"])
    out.update(act_x=act["x"], act_bias=act["bias"], act_dy=act["dy"], act_y=y, act_dx=dx, act_dbias=dbias)
    # cross-entropy + argmax, with a few ties
    xe = W.xent(rows=256, classes=100, seed=3)
    logits = xe["logits"]
    logits[5, 7] = logits[5, 9] = np.float32(50.0)
    loss, grad, am = ref.cross_entropy(logits, xe["targets"])
    out.update(xent_logits=logits, xent_targets=xe["targets"], xent_loss=np.float32(loss), xent_grad=grad,
               xent_argmax=am)
    # reductions, with NaNs placed first and inside the axis
    x = rng.standard_normal((5, 300, 7)).astype(np.float32)
    x[0, 0, 0] = np.nan
    x[1, 10, 2] = np.nan
    x[2, 0, 3] = np.float32(-np.inf)
    out["reduce_x"] = x
    for axis in (0, 1, 2):
        for op, opname in ((K.SUM, "sum"), (K.MAX, "max"), (K.ARGMAX, "argmax")):
            out[f"reduce_{opname}_{axis}"] = ref.reduce_axis(x, axis, op)
    out["sum_out"] = np.float32(ref.sum_all(sum_input()))
    # small MLP: gradients of one step, then parameters after three SGD steps
    m = W.mlp(batch=64, dims=(32, 48, 40, 10), seed=4)
    net = ref.mlp(m["weights"], m["biases"], m["x"], m["targets"])
    loss, dws, dbs = net.grads()
    out.update(mlp_x=m["x"], mlp_targets=m["targets"], mlp_loss=np.float32(loss))
    for i, (w, b, dw, db) in enumerate(zip(m["weights"], m["biases"], dws, dbs)):
        out.update({f"mlp_w{i}": w, f"mlp_b{i}": b, f"mlp_dw{i}": dw, f"mlp_db{i}": db})
    losses = [net.step(0.01) for _ in range(3)]
    ws, bs = net.params()
    out["mlp_losses"] = np.asarray(losses, dtype=np.float32)
    for i, (w, b) in enumerate(zip(ws, bs)):
        out[f"mlp_w{i}_after3"], out[f"mlp_b{i}_after3"] = w, b
    # spiral workload (full size): five steps at lr 1.0
    sp = W.spiral()
    net = ref.mlp(sp["weights"], sp["biases"], sp["x"], sp["targets"])
    out["spiral_losses"] = np.asarray([net.step(1.0) for _ in range(5)], dtype=np.float32)
    ws, bs = net.params()
    for i, (w, b) in enumerate(zip(ws, bs)):
        out[f"spiral_w{i}_after5"], out[f"spiral_b{i}_after5"] = w, b
    path = Path(__file__).with_name("ref_vectors.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({path.stat().st_size / 1e6:.2f} MB, {len(out)} arrays)")


if __name__ == "__main__":
    main()
