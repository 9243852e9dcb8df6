#!/usr/bin/env python3
"""Train-step benchmark of the MI355X backend.

Workload: one SGD train step of the fp32 MLP 8192 x 1024 -> 4096 -> 4096 -> 1000
(ReLU between layers, softmax cross-entropy over int targets, full reverse-mode
backward through the autograd graph, SGD at lr 0.01; W ~ U(+-1/sqrt(fan_in)),
biases 0, x ~ N(0, 1), seed 4), all on the hip device with inputs resident in
HBM. Each step ends with loss.item(), as the reference's train benchmark does
(benchmarks/train_benchmark.py:43-48). Parameter, activation and gradient
buffers are recycled through the device pool.

Prints one JSON line: whole-job train-steps/s, the backward-GEMM roofline
(MFMA-bound; HIP events carried by the backward-GEMM dispatches on the library
stream over the timed region, the only kernels timed there), the forward-GEMM
rate and the bias-gradient sums from a short breakdown pass that times every
kernel, the standalone reduction kernel on the step's bias-gradient shapes, the
other configurations (--config runs one of them alone), and the reference CPU
path timed on this host on the same full-batch step.
vs_baseline stays null: no published figure exists for this metric (the
reference publishes Apple M4 numbers at other shapes only).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

DIMS = (1024, 4096, 4096, 1000)
BATCH = 8192
FP32_MFMA_PEAK_TFLOPS = 157.3  # MI355X dense fp32 matrix peak
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
CPU_BASELINE_STEPS = 3         # CPU baseline: full 8192-row steps after one warm-up
BWD_GEMM_LABELS = ("gemm_nt", "gemm_tn")  # dH = dY W^T and dW = H^T dY
BREAKDOWN_STEPS = 5


def log(*args):
    print(*args, file=sys.stderr, flush=True)


def copy_calibration_pass(vc):
    """A plain streaming pass of known size (read 256 MiB, write 256 MiB) whose
    FETCH_SIZE/WRITE_SIZE counters calibrate rocprofv3's traffic readings."""
    src = vc.Tensor.zeros([64 << 20], device="hip")
    for _ in range(3):
        _ = -src
    vc.synchronize()


def mlp_step(vc, m):
    """One train step of the MLP `m` (workloads.mlp) on the hip device:
    x @ W + b per layer, ReLU between layers, cross-entropy, backward, SGD,
    gradients zeroed, the loss read."""
    params = []
    for w, b in zip(m["weights"], m["biases"]):
        params += [vc.Tensor(w, requires_grad=True, device="hip"), vc.Tensor(b, requires_grad=True, device="hip")]
    x = vc.Tensor(m["x"], device="hip")
    targets = m["targets"]
    lr = m["lr"]
    layers = len(m["weights"])

    def step():
        h = x
        for i in range(layers):
            h = h @ params[2 * i] + params[2 * i + 1]
            if i < layers - 1:
                h = h.relu()
        loss = vc.cross_entropy(h, targets)
        loss.backward()
        vc.sgd_step(params, lr)
        vc.zero_grad(params)
        return loss.item()

    return step


def gpu_bench(steps: int, warmup: int, copy_calibration: bool = False):
    import numpy as np

    import vectorcore_amd as vc
    from vectorcore_amd import workloads as W

    if not vc.hip_available():
        raise SystemExit("bench.py: the hip device is unavailable: the MI355X backend needs a gfx950 GPU")
    step = mlp_step(vc, W.mlp(batch=BATCH, dims=DIMS))

    if copy_calibration:
        copy_calibration_pass(vc)
    losses = [step() for _ in range(warmup)]
    allocs_before = vc.hip_pool_stats()["device_allocations"]
    # Timed region. Only the backward GEMMs carry HIP events (as dispatch
    # timestamps on the library stream), for the roofline.
    vc.synchronize()
    vc.hip_profile(True, labels=list(BWD_GEMM_LABELS))
    vc.hip_profile_reset()
    t0 = time.perf_counter()
    for _ in range(steps):
        losses.append(step())
    vc.synchronize()
    elapsed = time.perf_counter() - t0
    prof = vc.hip_profile_read()
    allocs_after = vc.hip_pool_stats()["device_allocations"]
    # Breakdown pass after the timed region: every kernel carries events.
    vc.hip_profile(True)
    vc.hip_profile_reset()
    breakdown_steps = max(1, min(steps, BREAKDOWN_STEPS))
    for _ in range(breakdown_steps):
        losses.append(step())
    breakdown = vc.hip_profile_read()
    vc.hip_profile(False)
    if not np.isfinite(losses[-1]) or not losses[-1] < losses[0]:
        raise SystemExit(f"bench.py: training did not make progress: {losses[0]} -> {losses[-1]}")
    return dict(elapsed=elapsed, prof=prof, breakdown=breakdown, breakdown_steps=breakdown_steps, losses=losses,
                new_allocations=allocs_after - allocs_before, device=vc.hip_device_name(),
                gemm_kernel=vc.hip_gemm_kernel())


def cpu_baseline():
    """The reference VectorCore (built from its own sources into oracle/_ref)
    running the same full-batch step on this host's cores: one warm-up step,
    then the median of CPU_BASELINE_STEPS timed steps, each ending with the
    loss read as in benchmarks/train_benchmark.py:71-79."""
    import statistics

    import numpy as np

    from oracle import kernels as K
    from vectorcore_amd import workloads as W

    m = W.mlp(batch=BATCH, dims=DIMS)
    nproc = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    if K.Reference.available():
        ref = K.Reference()
        net = ref.mlp(m["weights"], m["biases"], m["x"], m["targets"])
        t0 = time.perf_counter()
        net.step(m["lr"])  # warm-up (thread pool, first touch of the buffers)
        log(f"  cpu baseline: warm-up step {time.perf_counter() - t0:.1f} s")
        times = []
        for i in range(CPU_BASELINE_STEPS):
            t0 = time.perf_counter()
            net.step(m["lr"])
            times.append(time.perf_counter() - t0)
            log(f"  cpu baseline: step {i + 1}/{CPU_BASELINE_STEPS} {times[-1]:.2f} s")
        per_step = statistics.median(times)
        return dict(value=1.0 / per_step, unit="train-steps/s", cores=ref.threads(), kind="reference",
                    hardware_concurrency=ref.threads(), nproc=nproc, step_seconds=[round(t, 3) for t in times],
                    sample=f"reference VectorCore CPU path (oracle/_ref, -O3, no -march), the full 8192-row "
                           f"1024-4096-4096-1000 step (forward, cross-entropy, backward, SGD, loss read), "
                           f"median of {CPU_BASELINE_STEPS} steps after 1 warm-up, "
                           f"{ref.threads()} pool threads (std::thread::hardware_concurrency), nproc {nproc}")
    from oracle import autograd as A
    net = A.Mlp(m["weights"], m["biases"])
    rows = 256
    x = A.T(m["x"][:rows])
    t0 = time.perf_counter()
    net.step(x, m["targets"][:rows], m["lr"])
    per_full_step = (time.perf_counter() - t0) * (BATCH / rows)
    return dict(value=1.0 / per_full_step, unit="train-steps/s", cores=1, kind="port", nproc=nproc,
                sample=f"C oracle (the reference library is not built here), {rows}-row slice, one step, "
                       f"scaled x{BATCH // rows}")


def _median_ms(fn, reps):
    import statistics
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append((time.perf_counter() - t0) * 1e3)
    return statistics.median(times)


# Untimed calls before a configuration's timed ones. The part raises its
# clock over the first tens of milliseconds of sustained load (batched matmul
# backward: 0.69 of peak on its first calls, 0.83 after 50 more, 25 ms), so
# each configuration first runs its call for this long, as a training loop
# would have before.
CONFIG_WARM_S = 0.1


def _warm_up(fn, seconds=CONFIG_WARM_S):
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        fn()


def _profiled(vc, fn, labels=None, repeats=20, setup=None):
    """Per-label kernel aggregates of one call of fn (events on the kernels'
    dispatches), averaged over `repeats` calls; `setup` runs untimed before each."""
    vc.synchronize()
    vc.hip_profile_reset()
    for _ in range(repeats):
        if setup:
            setup()
            vc.synchronize()
        vc.hip_profile(True, labels=labels)
        fn()
        vc.hip_profile(False)
    out = vc.hip_profile_read()
    return {k: {f: (v[f] / repeats if f in ("ms", "flops", "bytes", "launches") else v[f]) for f in v}
            for k, v in out.items()}


def _reference(cpu: bool):
    if not cpu:
        return None
    from oracle import kernels as K
    return K.Reference() if K.Reference.available() else None


def _small_mlp_step(vc, m):
    """One train step of a one-hidden-layer classifier m (workloads.spiral or
    workloads.mnist_shaped) on the hip device, ending with loss.item() as
    benchmarks/train_benchmark.py:40-45 does."""
    ps = []
    for w, b in zip(m["weights"], m["biases"]):
        ps += [vc.Tensor(w, requires_grad=True, device="hip"), vc.Tensor(b, requires_grad=True, device="hip")]
    xs = vc.Tensor(m["x"], device="hip")
    targets = [int(t) for t in m["targets"]]

    def step():
        loss = vc.cross_entropy((xs @ ps[0] + ps[1]).relu() @ ps[2] + ps[3], targets)
        loss.backward()
        vc.sgd_step(ps, m["lr"])
        vc.zero_grad(ps)
        return loss.item()

    return step


def _small_mlp_figures(vc, step, warmup):
    """Throughput over 200 steps drained at both ends (median of 5), and the
    reference's own per-step measure: the median of 30 step times, each ending
    with loss.item(), after 5 warm-up steps (benchmarks/train_benchmark.py:
    71-79). loss.item() waits for the loss kernel only, so a step's host time
    can end while its backward and update still run; the throughput figure
    covers the device's whole work."""
    # Untimed warm-up long enough to reach the steady rate: the first few
    # hundred steps of a process run up to ~30% slower.
    for _ in range(warmup):
        step()

    def steps():
        vc.synchronize()
        for _ in range(200):
            step()
        vc.synchronize()

    steps_per_s = 200e3 / _median_ms(steps, 5)
    for _ in range(5):
        step()
    return {"hip_steps_per_s": round(steps_per_s, 1), "hip_median_step_ms": round(_median_ms(step, 30), 4)}


def measure_spiral(vc, W, ref):
    """Spiral classifier train step (launch-bound; no roofline)."""
    sp = W.spiral()
    c1 = {"workload": "spiral 300x2->64->3 train step, lr 1.0", "bound": "launch/latency",
          **_small_mlp_figures(vc, _small_mlp_step(vc, sp), 500)}
    if ref:
        net = ref.mlp(sp["weights"], sp["biases"], sp["x"], sp["targets"])
        net.step(sp["lr"])
        c1["cpu_reference_steps_per_s"] = round(1e3 / _median_ms(lambda: net.step(sp["lr"]), 50), 1)
    c1["published_reference_ms_per_step"] = {
        "apple_m4_cpu": 0.749, "apple_m4_metal": 0.964,
        "source": "docs/benchmarks.md:16-17 (benchmarks/train_benchmark.py, spiral_2-64-3_b300: the same shapes on "
                  "N(0,1) inputs; Apple M4 under heavy load, per that file); context, not a target"}
    return c1


def measure_mnist_shaped(vc, W, ref):
    """The reference's MNIST-shaped train step, 256 x 784 -> 256 -> 10
    (benchmarks/train_benchmark.py:23-26), with its own generator."""
    mn = W.mnist_shaped()
    out = {"workload": "MLP 784->256->10 fp32 (ReLU), batch 256: forward, softmax cross-entropy, backward, SGD lr 0.1",
           "bound": "launch/latency", **_small_mlp_figures(vc, _small_mlp_step(vc, mn), 300)}
    if ref:
        net = ref.mlp(mn["weights"], mn["biases"], mn["x"], mn["targets"])
        for _ in range(5):
            net.step(mn["lr"])
        ms = _median_ms(lambda: net.step(mn["lr"]), 30)
        out["cpu_reference_median_step_ms"] = round(ms, 3)
        out["cpu_reference_steps_per_s"] = round(1e3 / ms, 1)
    out["published_reference_ms_per_step"] = {
        "apple_m4_cpu": 6.346, "apple_m4_metal": 1.756,
        "source": "docs/benchmarks.md:18-19 (benchmarks/train_benchmark.py, mnist_784-256-10_b256; Apple M4 under "
                  "heavy load, per that file); context, not a target"}
    return out


def measure_bmm(vc, W, ref, bkey):
    """Batched matmul backward, dA = dC B^T (NT) and dB = A^T dC (TN)."""
    bm = W.bmm()
    flops = 2.0 * 8 * 1024 ** 3
    a = vc.Tensor(bm["a"], requires_grad=True, device="hip")
    b = vc.Tensor(bm[bkey], requires_grad=True, device="hip")
    dc = vc.Tensor(bm["dc"], device="hip")

    def fwd_bwd():
        (a @ b).backward(dc)
        vc.zero_grad([a, b])
        vc.synchronize()

    _warm_up(fwd_bwd)
    prof = _profiled(vc, fwd_bwd, labels=list(BWD_GEMM_LABELS))
    ms = sum(v["ms"] for v in prof.values())
    tflops = 2 * flops / ms / 1e9
    c2 = {"workload": f"A [8,1024,1024] @ B {list(bm[bkey].shape)}, backward dA and dB",
          "bound": "mfma", "bwd_gemm_tflops": round(tflops, 1), "frac": round(tflops / FP32_MFMA_PEAK_TFLOPS, 3),
          "bwd_gemm_ms": round(ms, 3), "per_kernel_us": {k: round(v["ms"] * 1e3, 1) for k, v in prof.items()},
          "hip_ms_forward_backward": round(_median_ms(fwd_bwd, 10), 3)}
    if ref:
        c2["cpu_reference_ms_forward_backward"] = round(
            _median_ms(lambda: ref.matmul_backward(bm["a"], bm[bkey], bm["dc"]), 1), 1)
    return c2


def measure_activation(vc, W, ref):
    """Activation chain y = sigmoid(relu(x + bias)) * exp(0.1 x); backward for dx, dbias."""
    ac = W.activation()
    x = vc.Tensor(ac["x"], requires_grad=True, device="hip")
    bias = vc.Tensor(ac["bias"], requires_grad=True, device="hip")
    dy = vc.Tensor(ac["dy"], device="hip")
    holder = {}

    def forward():
        holder["y"] = (x + bias).relu().sigmoid() * (x * 0.1).exp()
        vc.synchronize()

    def backward():
        holder["y"].backward(dy)
        vc.synchronize()

    def fwd_bwd():
        forward(); backward(); vc.zero_grad([x, bias])

    _warm_up(fwd_bwd)

    def fresh_forward():
        vc.zero_grad([x, bias])
        forward()

    prof = _profiled(vc, backward, setup=fresh_forward)
    vc.zero_grad([x, bias])
    kms = sum(v["ms"] for v in prof.values())
    kbytes = sum(v["bytes"] for v in prof.values())
    min_bytes = 3 * 4096 * 4096 * 4 + 2 * 4096 * 4
    c3 = {"workload": "x [4096,4096] + bias [1,4096]: sigmoid(relu) * exp(0.1 x), backward dx and dbias",
          "bound": "hbm", "bwd_kernel_gbs": round(kbytes / kms / 1e6, 1),
          "frac": round(kbytes / kms / 1e6 / HBM_PEAK_GBS, 3), "bwd_kernels_ms": round(kms, 3),
          "bwd_kernel_launches": int(sum(v["launches"] for v in prof.values())),
          "bwd_bytes_mb": round(kbytes / 1e6, 1),
          "min_bytes_rate_gbs": round(min_bytes / kms / 1e6, 1),
          "per_label_us": {k: round(v["ms"] * 1e3, 1) for k, v in prof.items()},
          "hip_ms_forward_backward": round(_median_ms(fwd_bwd, 10), 3)}
    if ref:
        c3["cpu_reference_ms_forward_backward"] = round(
            _median_ms(lambda: ref.activation_backward(ac["x"], ac["bias"], ac["dy"]), 1), 1)
    return c3


def measure_xent(vc, W, ref):
    """Mean softmax cross-entropy forward + backward, argmax over classes."""
    xe = W.xent()
    lg = vc.Tensor(xe["logits"], requires_grad=True, device="hip")
    tg = xe["targets"]

    def ce_calls():
        loss = vc.cross_entropy(lg, tg)
        loss.backward()
        lg.detach().argmax(1)
        vc.zero_grad([lg])

    def ce():
        ce_calls()
        vc.synchronize()

    _warm_up(ce)
    # The kernels are timed over calls enqueued back to back, as a training
    # loop runs them (a call that starts on an idle device measured ~1 us
    # longer in the forward); hip_ms times whole calls, each synchronised.
    prof = _profiled(vc, ce_calls)
    c4 = {"workload": "logits [32768,1000] N(0,4): loss, dlogits, argmax(1)", "bound": "hbm",
          "hip_ms": round(_median_ms(ce, 10), 3)}
    for label in ("xent_forward", "xent_backward", "reduce_axis_argmax"):
        v = prof.get(label)
        if v and v["ms"]:
            gbs = v["bytes"] / v["ms"] / 1e6
            c4[label] = {"ms": round(v["ms"], 4), "gbs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 3)}
    if ref:
        c4["cpu_reference_ms"] = round(_median_ms(lambda: ref.cross_entropy(xe["logits"], tg), 1), 1)
    return c4


ONE_HIDDEN_DIMS = (1024, 4096, 1000)
ONE_HIDDEN_STEPS = 20


def measure_mlp_one_hidden(vc, W, ref):
    """The one-hidden-layer network 8192 x 1024 -> 4096 -> 1000 (the headline
    runs 1024 -> 4096 -> 4096 -> 1000): the same train step, seed and
    initialisation; steps/s over ONE_HIDDEN_STEPS steps after CONFIG_WARM_S of untimed steps,
    and the backward GEMMs' rate from events on their dispatches."""
    m = W.mlp(batch=BATCH, dims=ONE_HIDDEN_DIMS)
    step = mlp_step(vc, m)
    _warm_up(step)
    vc.synchronize()
    vc.hip_profile(True, labels=list(BWD_GEMM_LABELS))
    vc.hip_profile_reset()
    t0 = time.perf_counter()
    losses = [step() for _ in range(ONE_HIDDEN_STEPS)]
    vc.synchronize()
    elapsed = time.perf_counter() - t0
    prof = vc.hip_profile_read()
    vc.hip_profile(False)
    _, bwd_flops = W.mlp_gemm_flops(BATCH, ONE_HIDDEN_DIMS)
    gemm_ms = sum(v["ms"] for v in prof.values()) / ONE_HIDDEN_STEPS
    tflops = bwd_flops / gemm_ms / 1e9
    out = {"workload": "MLP 1024->4096->1000 fp32 (ReLU), batch 8192: forward, softmax cross-entropy, backward, "
                       "SGD lr 0.01", "bound": "mfma", "hip_steps_per_s": round(ONE_HIDDEN_STEPS / elapsed, 2),
           "ms_per_step": round(elapsed * 1e3 / ONE_HIDDEN_STEPS, 3), "bwd_gemm_tflops": round(tflops, 1),
           "frac": round(tflops / FP32_MFMA_PEAK_TFLOPS, 4), "loss_first_last": [round(losses[0], 5),
                                                                                round(losses[-1], 5)]}
    if ref:
        net = ref.mlp(m["weights"], m["biases"], m["x"], m["targets"])
        net.step(m["lr"])
        times = []
        for _ in range(2):
            t0 = time.perf_counter()
            net.step(m["lr"])
            times.append(time.perf_counter() - t0)
        out["cpu_reference_steps_per_s"] = round(1.0 / min(times), 4)
        out["cpu_reference_sample"] = "full 8192-row steps: 1 warm-up, then the faster of 2"
    return out


def measure_column_sums(vc):
    """The standalone column-sum reduction (axis-0 sum) on the train step's
    bias-gradient shapes: the kernel a bias gradient takes when its producer
    cannot keep the sums (inside the step they come from the producers)."""
    import numpy as np
    rng = np.random.default_rng(5)
    out = {}
    total_bytes = total_ms = 0.0
    for rows, cols, times in ((BATCH, 4096, 2), (BATCH, 1000, 1)):
        t = vc.Tensor(rng.standard_normal((rows, cols)).astype(np.float32), device="hip")

        def colsum():
            t.sum(0)
            vc.synchronize()

        _warm_up(colsum)
        prof = _profiled(vc, lambda: t.sum(0), labels=["reduce_axis_sum"], repeats=10)["reduce_axis_sum"]
        gbs = prof["bytes"] / prof["ms"] / 1e6
        out[f"{rows}x{cols}"] = {"us": round(prof["ms"] * 1e3, 2), "gbs": round(gbs, 1),
                                 "frac": round(gbs / HBM_PEAK_GBS, 3)}
        total_bytes += times * prof["bytes"]
        total_ms += times * prof["ms"]
    out["step_shapes_gbs"] = round(total_bytes / total_ms / 1e6, 1)
    return out


CONFIGS = ("spiral_train_step", "mnist_shaped_train_step", "batched_matmul_backward",
           "batched_matmul_backward_broadcast_b", "activation_backward", "cross_entropy", "column_sums",
           "mlp_one_hidden_layer")


def config_measurements(cpu: bool, only=None):
    """The reference's other configurations on the hip device: throughput, the
    roofline fraction of their kernels, and the reference CPU path on the same
    inputs (whole calls, including the harness's host copies), in this run."""
    import vectorcore_amd as vc
    from vectorcore_amd import workloads as W
    ref = _reference(cpu)
    run = {
        "spiral_train_step": lambda: measure_spiral(vc, W, ref),
        "mnist_shaped_train_step": lambda: measure_mnist_shaped(vc, W, ref),
        "batched_matmul_backward": lambda: measure_bmm(vc, W, ref, "b"),
        "batched_matmul_backward_broadcast_b": lambda: measure_bmm(vc, W, ref, "b_shared"),
        "activation_backward": lambda: measure_activation(vc, W, ref),
        "cross_entropy": lambda: measure_xent(vc, W, ref),
        "column_sums": lambda: measure_column_sums(vc),
        "mlp_one_hidden_layer": lambda: measure_mlp_one_hidden(vc, W, ref),
    }
    out = {}
    for name in (only or CONFIGS):
        # One configuration failing is reported in its entry (and on stderr)
        # instead of taking the train-step line down with it.
        try:
            out[name] = run[name]()
        except Exception as e:  # noqa: BLE001
            import traceback
            traceback.print_exc()
            out[name] = {"error": f"{type(e).__name__}: {e}"}
    if ref:
        out["cpu_reference_threads"] = ref.threads()
    return out


def load_traffic():
    """HBM bytes per launch of the dominant kernels, measured with rocprofv3
    FETCH_SIZE/WRITE_SIZE runs and kept in profiles/ (None when absent)."""
    path = ROOT / "profiles" / "hbm_traffic.json"
    if not path.exists():
        return None
    try:
        return json.loads(path.read_text())
    except (OSError, ValueError):
        return None


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-configs", action="store_true", help="skip the other configurations' measurements")
    ap.add_argument("--config", choices=CONFIGS,
                    help="run only this configuration's measurement (no train-step bench) and print it as JSON")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first stream 256 MiB through a negate kernel (counter calibration for rocprofv3 --pmc)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (the data-parallel sharding of "
              "this workload is a design note, not a launched path)", file=sys.stderr)
        sys.exit(2)

    if args.config:
        if args.copy_calibration:
            import vectorcore_amd as vc
            copy_calibration_pass(vc)
        print(json.dumps({args.config: config_measurements(cpu=not args.no_cpu_baseline, only=[args.config])[args.config]}),
              flush=True)
        return

    r = gpu_bench(args.steps, args.warmup, args.copy_calibration)
    prof = r["prof"]
    ms_per_step = r["elapsed"] * 1e3 / args.steps
    bwd = [v for k, v in prof.items() if k in BWD_GEMM_LABELS]
    bwd_flops = sum(v["flops"] for v in bwd)
    bwd_ms = sum(v["ms"] for v in bwd)
    bwd_launches = sum(v["launches"] for v in bwd)
    bwd_tflops = bwd_flops / bwd_ms / 1e9 if bwd_ms else None
    # Per-kernel figures from the breakdown pass.
    bd, nb = r["breakdown"], r["breakdown_steps"]
    combine = bd.get("column_sum_combine", {})
    fwd = bd.get("gemm_nn", {})
    fwd_tflops = fwd["flops"] / fwd["ms"] / 1e9 if fwd.get("ms") else None
    device_ms = sum(v["ms"] for v in bd.values()) / nb
    log(f"  breakdown pass ({nb} steps, every kernel timed):")
    for k, v in sorted(bd.items(), key=lambda kv: -kv[1]["ms"]):
        rate = (f"{v['flops'] / v['ms'] / 1e9:7.1f} TFLOP/s" if v["flops"] and "gemm" in k
                else f"{v['bytes'] / v['ms'] / 1e6:7.0f} GB/s")
        log(f"  {k:22s} {v['launches'] / nb:5.1f}/step {v['ms'] / nb:8.3f} ms/step  {rate}")
    log(f"  device time {device_ms:.3f} ms/step; timed region {ms_per_step:.3f} ms/step wall")

    traffic = load_traffic()
    roofline = {
        "bound": "mfma",
        "kernel": "backward GEMMs (gemm_nt dH = dY W^T, gemm_tn dW = H^T dY), fp32 V_MFMA_F32_32X32X2_F32",
        "achieved": round(bwd_tflops, 2) if bwd_tflops else None,
        "peak": FP32_MFMA_PEAK_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(bwd_tflops / FP32_MFMA_PEAK_TFLOPS, 4) if bwd_tflops else None,
        "traffic": traffic.get("bwd_gemm_bytes_per_launch") if traffic else None,
        "launches_per_step": bwd_launches / args.steps,
        "flops_per_step": bwd_flops / args.steps,
    }
    out = {
        "metric": "MLP train-steps/s (8192x1024->4096->4096->1000 fp32); bwd GEMM TFLOP/s; reduce GB/s",
        "value": round(1e3 / ms_per_step, 3),
        "unit": "train-steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0,1) inputs, U(+-1/sqrt(fan_in)) weights, uniform int targets)",
        "config": {"workload": "MLP 1024->4096->4096->1000 fp32 (ReLU), batch 8192: forward, softmax cross-entropy, "
                               "backward, SGD lr 0.01",
                   "global_batch": BATCH, "layers": list(DIMS), "parallelism": "single GPU"},
        "bwd_gemm_tflops": round(bwd_tflops, 2) if bwd_tflops else None,
        "fwd_gemm_tflops": round(fwd_tflops, 2) if fwd_tflops else None,
        "bias_grad_sums": {
            "how": "partial column sums left pending by the producing kernels (masked NT product epilogue for "
                   "db1 and db2, cross-entropy backward for db3) and finished inside the SGD launch; a separate "
                   "combine launch would show here",
            "combine_launches_per_step": round(combine.get("launches", 0) / nb, 2),
            "combine_us_per_step": round(combine.get("ms", 0.0) * 1e3 / nb, 2),
        },
        "device_ms_per_step": round(device_ms, 3),
        "timing": "value and roofline: the timed steps, with events on the backward GEMMs only; "
                  "fwd_gemm_tflops, bias_grad_sums, device_ms_per_step: a breakdown pass of "
                  f"{r['breakdown_steps']} further steps with every kernel timed; reduce_gbs: the standalone "
                  "column-sum kernel on the step's bias-gradient shapes (configs.column_sums)",
        "pool_new_allocations_in_timed_steps": r["new_allocations"],
        "loss_first_last": [round(r["losses"][0], 5), round(r["losses"][-1], 5)],
        "device": r["device"],
        "roofline": roofline,
    }
    if not args.no_cpu_baseline:
        t0 = time.perf_counter()
        out["cpu_baseline"] = cpu_baseline()
        out["speedup_vs_cpu_baseline"] = round(out["value"] / out["cpu_baseline"]["value"], 1)
        log(f"  cpu baseline took {time.perf_counter() - t0:.1f} s")
    if not args.no_configs:
        t0 = time.perf_counter()
        out["configs"] = config_measurements(cpu=not args.no_cpu_baseline)
        log(f"  other configurations took {time.perf_counter() - t0:.1f} s")
        sums = out["configs"]["column_sums"]
        # The reduction kernel on the step's bias-gradient shapes ([8192, 4096] twice, [8192, 1000]).
        if "step_shapes_gbs" in sums:
            out["reduce_gbs"] = sums["step_shapes_gbs"]
            out["reduce_hbm_frac"] = round(sums["step_shapes_gbs"] / HBM_PEAK_GBS, 4)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
