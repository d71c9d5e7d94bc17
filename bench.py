"""Benchmark of the MLP training step on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
                    [--only all|step|small|bwd|splitk|mixed|tape|pcie|copy]

Workload (one "step"): MLP 512->1024(ReLU)->1024(ReLU)->10, f32, batch 2048,
softmax cross-entropy, Adam(1e-3, 0.9, 0.999, 1e-8): forward, backward and the
optimizer update, on synthetic N(0,1) batches with uniform labels in [0,10)
that are resident in HBM before timing starts (one fresh batch per step).

Prints ONE JSON line.  `value` is ms/step over K timed steps (lower is
better), timed after the W warmup steps and a further ~100 ms of steps that
let the device settle at its sustained clock (settle_steps in the line).
Next to it:
  roofline      the dominant kernel of the step: algorithmic FLOPs per launch
                over its average duration, from HIP events that the kernel's
                own dispatch carries (hipExtLaunchKernel), against the f32
                MFMA peak
  small_batch   the same MLP at batch 32 with SGD(0.01), one step = forward,
                backward, update: ms/step, per-launch µs, the HBM roofline of
                its compulsory bytes, and its own CPU baseline
  bwd_gemm      Linear 4096->4096 backward at batch 8192 in bf16 (dX = dY·Wᵀ,
                dW = Xᵀ·dY with db fused), TFLOP/s against the bf16 MFMA peak
  splitk_dw     dW = Xᵀ·dY, K = 262144, f16 in / f32 out, db fused, against
                the HBM roofline
  mixed_mlp     8 x 4096 ReLU MLP -> 1000 classes, batch 4096, bf16 with f32
                master weights, loss scale 1024, Adam: ms/step and TFLOP/s
  pcie_inclusive  the same step with every batch copied from host memory:
                synchronous writes vs. the overlapped loader (not `value`)
  tape_mlp      examples/bench_grande.rs (N 4096, D 128, H 512, minibatch
                256, Adam) trained through the device autodiff tape, one
                HIP launch per recorded op, against the oracle's CPU tape
  cpu_baseline  the CPU oracle (C++ restatement of rtensor's single-threaded
                CPU path) timed on a bounded sample of the same workload, on
                one host thread; bwd_gemm, splitk_dw and mixed_mlp carry
                their own, from row samples scaled to the whole workload
"""
from __future__ import annotations

import argparse
import itertools
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_F32_TFLOPS = 157.3   # MI355X dense f32 matrix
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 matrix
PEAK_HBM_GBS = 8000.0
REF_GPU_MS_B2048 = 6.89   # rtensor GPU step at batch 2048 (README.md:53), RTX 4070 Laptop

DIMS = [512, 1024, 1024, 10]
BATCH = 2048


def kaiming(rng, fan_in, fan_out):
    bound = np.sqrt(6.0 / fan_in)
    return rng.uniform(-bound, bound, size=(fan_in, fan_out)).astype(np.float32)


def step_flops(dims, batch):
    """Algorithmic FLOPs of one step: forward + dW per layer + dX for layers > 0."""
    f = 0
    for l in range(len(dims) - 1):
        mk = dims[l] * dims[l + 1]
        f += 2 * batch * mk * (3 if l > 0 else 2)
    return f


def label_flops(label, dims, batch):
    """FLOPs per launch of a plan kernel label (fwd_l*, dw_l*, dx_l*, and
    dwdx_l*: a layer's dW and dX in one launch)."""
    if label.startswith("dwdx_l"):
        l = int(label[len("dwdx_l"):])
        return 2 * 2 * batch * dims[l] * dims[l + 1]
    for pre in ("fwd_l", "dw_l", "dx_l"):
        if label.startswith(pre):
            l = int(label[len(pre):])
            return 2 * batch * dims[l] * dims[l + 1]
    return 0


def traffic_for(label, section=None, key="bytes_per_launch"):
    """HBM bytes measured by rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE, scaled by
    a copy of known size) from the committed summary profiles/pmc_traffic.json,
    if present: per launch of a batch-2048 step label, or under `section`
    (small_batch: the batch-32 SGD step)."""
    path = os.path.join(ROOT, "profiles", "pmc_traffic.json")
    try:
        with open(path) as f:
            doc = json.load(f)
    except (OSError, ValueError):
        return None
    if section is not None:
        doc = doc.get(section, {})
    if label is None:
        return doc.get(key)
    return doc.get(label, {}).get(key)


def bench_step(gpu, G, steps, warmup):
    rng = np.random.default_rng(2048)
    params = []
    for l in range(len(DIMS) - 1):
        params += [kaiming(rng, DIMS[l], DIMS[l + 1]), np.zeros((1, DIMS[l + 1]), np.float32)]
    mlp = G.GpuMlp.from_params(gpu, params, BATCH, 1e-3)
    nb = min(steps + warmup, 64)
    xs = [gpu.upload(rng.standard_normal((BATCH, DIMS[0]), dtype=np.float32)) for _ in range(nb)]
    ys = [G.upload_labels(gpu, rng.integers(0, DIMS[-1], BATCH)) for _ in range(nb)]
    gpu.sync()
    for i in range(warmup):
        mlp.step(xs[i % nb], ys[i % nb])
    gpu.sync()
    settle = settle_clock(gpu, lambda i: mlp.step(xs[i % nb], ys[i % nb]))
    t0 = time.perf_counter()
    for i in range(steps):
        mlp.step(xs[(warmup + i) % nb], ys[(warmup + i) % nb])
    gpu.sync()
    wall = time.perf_counter() - t0
    loss = mlp.last_loss()

    # Second pass of the same steps with HIP events around every launch (on
    # the library's stream) for per-kernel durations.
    gpu.profile_reset()
    gpu.profile(True)
    for i in range(steps):
        mlp.step(xs[(warmup + i) % nb], ys[(warmup + i) % nb])
    gpu.sync()
    gpu.profile(False)
    prof = gpu.perfilar()
    gpu.profile_reset()
    return wall, loss, prof, mlp.dispatches_por_passo(), settle


def settle_clock(gpu, work, ms=100.0):
    """Runs work(i) in batches until ~ms of device load have passed: the
    device takes ~25 ms of sustained load to settle at its clock (~1.95 GHz
    at the ~1.35 kW socket limit), and the first launches run up to 15%
    slower.  Returns {settle_ms, settle_steps}."""
    t0 = time.perf_counter()
    n = 0
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(10):
            work(n)
            n += 1
        gpu.sync()
    return {"settle_ms": round((time.perf_counter() - t0) * 1e3, 1), "settle_steps": n}


def c1_bytes(dims):
    """Compulsory HBM bytes of one SGD step: W read by the forward and again
    by dX (layers > 0), dW written, and the update reading θ and g and
    writing θ (12 B per parameter)."""
    w = sum(dims[l] * dims[l + 1] for l in range(len(dims) - 1))
    b = sum(dims[1:])
    w_dx = sum(dims[l] * dims[l + 1] for l in range(1, len(dims) - 1))
    return 4 * (w + b) + 4 * w_dx + 4 * (w + b) + 12 * (w + b)


def bench_small(gpu, G, steps=2000, warmup=100):
    """MLP 512-1024-1024-10, f32, batch 32, SGD(0.01): the one-step config of
    README.md:50, timed over many steps (one fresh resident batch each)."""
    B = 32
    rng = np.random.default_rng(32)
    params = []
    for l in range(len(DIMS) - 1):
        params += [kaiming(rng, DIMS[l], DIMS[l + 1]), np.zeros((1, DIMS[l + 1]), np.float32)]
    mlp = G.GpuMlp.from_params(gpu, params, B, 0.01, optimizer="sgd")
    nb = 64
    xs = [gpu.upload(rng.standard_normal((B, DIMS[0]), dtype=np.float32)) for _ in range(nb)]
    ys = [G.upload_labels(gpu, rng.integers(0, DIMS[-1], B)) for _ in range(nb)]
    for i in range(warmup):
        mlp.step(xs[i % nb], ys[i % nb])
    gpu.sync()
    settle = settle_clock(gpu, lambda i: mlp.step(xs[i % nb], ys[i % nb]))
    t0 = time.perf_counter()
    for i in range(steps):
        mlp.step(xs[i % nb], ys[i % nb])
    gpu.sync()
    ms = (time.perf_counter() - t0) / steps * 1e3
    gpu.timer_begin()
    for i in range(steps):
        mlp.step(xs[i % nb], ys[i % nb])
    dev_ms = gpu.timer_end() / steps
    gpu.profile_reset()
    gpu.profile(True)
    for i in range(200):
        mlp.step(xs[i % nb], ys[i % nb])
    gpu.sync()
    gpu.profile(False)
    prof = gpu.perfilar()
    gpu.profile_reset()
    launches = mlp.dispatches_por_passo()
    mlp.destroy()
    byts = c1_bytes(DIMS)
    gbs = byts / (ms * 1e-3) / 1e9
    kern = {n: round(t / c * 1e3, 2) for n, c, t in prof}
    return {"config": "MLP 512-1024(ReLU)-1024(ReLU)-10, f32, batch 32, SGD(0.01); one step = forward, "
                      "backward, update", "ms_per_step": round(ms, 4), "device_ms_per_step": round(dev_ms, 4),
            "launches_per_step": launches, "kernels_us": kern,
            "kernel_sum_us": round(sum(kern.values()), 2),
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": round(gbs / PEAK_HBM_GBS, 4),
                         "traffic": traffic_for(None, "small_batch", "bytes_per_step"),
                         "traffic_unit": "bytes per step (the 6 launches)",
                         "traffic_source": "profiles/pmc_traffic.json small_batch: rocprofv3 --pmc FETCH_SIZE and "
                                           "WRITE_SIZE of bench.py --only small, scaled by a copy kernel of known size",
                         "bytes_per_step": byts,
                         "note": "a chain of dependent launches: the step is bound by launch latency, "
                                 "not by these bytes"},
            "vs_published": {"ref_gpu_ms": 0.73, "ref_cpu_ms": 14.01,
                             "source": "README.md:50, rtensor wgpu on an RTX 4070 Laptop and its CPU path"},
            **settle}


def bench_bwd_gemm(gpu, G, reps=10, rounds=20):
    """Linear 4096->4096 backward at batch 8192, bf16 operands, f32 accumulate."""
    B, D = 8192, 4096
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((B, D), dtype=np.float32) / np.float32(64.0))
    dy = (rng.standard_normal((B, D), dtype=np.float32) / np.float32(64.0))
    w = rng.uniform(-np.sqrt(6.0 / D), np.sqrt(6.0 / D), size=(D, D)).astype(np.float32)
    gx, gdy, gw = gpu.upload(x, G.BF16), gpu.upload(dy, G.BF16), gpu.upload(w, G.BF16)
    dx = gpu.zeros((B, D), G.BF16)
    dw = gpu.zeros((D, D), G.F32)
    db = gpu.zeros((1, D), G.F32)
    # The device takes ~25 ms of this load to settle at its sustained clock
    # (~1.95 GHz at the ~1.35 kW socket limit); the first rounds run up to
    # 15% slower.  Warm up for ~80 ms before timing.
    for _ in range(100):
        gpu.gemm(G.NT, gdy, gw, dx)
        gpu.gemm(G.TN, gx, gdy, dw, colsum=db)
    gpu.sync()
    # Back-to-back launches between two HIP events on the library stream,
    # dX and dW alternating in rounds, median over the rounds.
    t_dx, t_dw = [], []
    for _ in range(rounds):
        gpu.timer_begin()
        for _ in range(reps):
            gpu.gemm(G.NT, gdy, gw, dx)
        t_dx.append(gpu.timer_end() / reps)
        gpu.timer_begin()
        for _ in range(reps):
            gpu.gemm(G.TN, gx, gdy, dw, colsum=db)
        t_dw.append(gpu.timer_end() / reps)
    t_dx, t_dw = float(np.median(t_dx)), float(np.median(t_dw))
    flops = 2.0 * B * D * D
    tf_dx = flops / (t_dx * 1e-3) / 1e12
    tf_dw = flops / (t_dw * 1e-3) / 1e12
    tf = 2 * flops / ((t_dx + t_dw) * 1e-3) / 1e12
    return {
        "config": "Linear 4096->4096 backward, batch 8192, bf16 in / f32 accumulate; dX bf16, dW f32, db fused",
        "dX_ms": round(t_dx, 4), "dW_db_ms": round(t_dw, 4),
        "dX_tflops": round(tf_dx, 1), "dW_tflops": round(tf_dw, 1),
        "tflops": round(tf, 1), "peak_tflops": PEAK_BF16_TFLOPS, "frac": round(tf / PEAK_BF16_TFLOPS, 4),
    }


def bench_splitk(gpu, G, reps=50, slices=64):
    """Split-K weight gradient over a 262144-long batch, f16 operands."""
    K, M, N = 262144, 512, 512
    rng = np.random.default_rng(4)
    x = gpu.upload(rng.standard_normal((K, M), dtype=np.float32) / np.float32(16.0), G.F16)
    dy = gpu.upload(rng.standard_normal((K, N), dtype=np.float32) / np.float32(16.0), G.F16)
    dw, db = gpu.zeros((M, N)), gpu.zeros((1, N))
    part = gpu.zeros((slices * (M * N + N),))
    for _ in range(200):  # ~40 ms: past the device's clock ramp
        gpu.split_k(x, dy, dw, part, slices, True, colsum=db)
    gpu.sync()
    gpu.timer_begin()
    for _ in range(reps):
        gpu.split_k(x, dy, dw, part, slices, True, colsum=db)
    t = gpu.timer_end() / reps
    # Second pass with per-launch events for the GEMM / reduction split.
    gpu.profile_reset()
    gpu.profile(True)
    for _ in range(reps):
        gpu.split_k(x, dy, dw, part, slices, True, colsum=db)
    gpu.sync()
    gpu.profile(False)
    prof = {n: ms / c for n, c, ms in gpu.perfilar()}
    gpu.profile_reset()
    bytes_ = 2 * K * M * 2 + M * N * 4 + N * 4  # compulsory: read X, dY; write dW, db
    gbs = bytes_ / (t * 1e-3) / 1e9
    flops = 2.0 * K * M * N
    return {"config": "dW = X^T dY, K=262144, X,dY f16 [262144,512] ~N(0,1)/16, f32 out [512,512], db fused",
            "slices": slices, "gemm_ms": round(prof["splitk_gemm"], 4),
            "reduce_ms": round(prof.get("splitk_reduce", 0.0), 4), "ms": round(t, 4),
            "bound": "hbm", "achieved_gbs": round(gbs, 1), "peak_gbs": PEAK_HBM_GBS,
            "frac": round(gbs / PEAK_HBM_GBS, 4), "tflops": round(flops / (t * 1e-3) / 1e12, 1)}


def bench_colsum(gpu, G, reps=50):
    """The bias gradient on its own (rt_colsum, the reference's COLSUM):
    db = colsum(dY) for the Linear 4096 backward's dY (bf16 [8192, 4096]) and
    the split-K dW's dY (f16 [262144, 512]), against the HBM roofline."""
    out = {"config": "db = colsum(dY), f32 out; dY bf16 [8192,4096] ~N(0,1)/64 and f16 [262144,512] ~N(0,1)/16",
           "bound": "hbm", "peak_gbs": PEAK_HBM_GBS}
    rng = np.random.default_rng(5)
    for name, rows, cols, dt, scale in (("bf16_8192x4096", 8192, 4096, G.BF16, 64.0),
                                        ("f16_262144x512", 262144, 512, G.F16, 16.0)):
        a = gpu.upload(rng.standard_normal((rows, cols), dtype=np.float32) / np.float32(scale), dt)
        d = gpu.zeros((1, cols))
        for _ in range(100):  # past the clock ramp
            gpu.colsum(a, d)
        gpu.sync()
        ts = []
        for _ in range(5):
            gpu.timer_begin()
            for _ in range(reps):
                gpu.colsum(a, d)
            ts.append(gpu.timer_end() / reps)
        t = float(np.median(ts))
        bytes_ = rows * cols * 2 + cols * 4  # compulsory: read dY, write db
        gbs = bytes_ / (t * 1e-3) / 1e9
        out[name] = {"us": round(t * 1e3, 2), "achieved_gbs": round(gbs, 1), "frac": round(gbs / PEAK_HBM_GBS, 4)}
    return out


def bench_mixed(gpu, G, steps=20, warmup=10):
    """8 x 4096 ReLU layers -> 1000 classes, batch 4096, bf16 + f32 master, Adam."""
    dims = [4096] * 9 + [1000]
    B = 4096
    rng = np.random.default_rng(5)
    params = []
    for l in range(len(dims) - 1):
        params += [kaiming(rng, dims[l], dims[l + 1]), np.zeros((1, dims[l + 1]), np.float32)]
    mlp = G.GpuMlp.from_params(gpu, params, B, 1e-3, precision="bf16", loss_scale=1024.0)
    del params
    xs = [gpu.upload(rng.standard_normal((B, dims[0]), dtype=np.float32), G.BF16) for _ in range(4)]
    ys = [G.upload_labels(gpu, rng.integers(0, dims[-1], B)) for _ in range(4)]
    for i in range(warmup):
        mlp.step(xs[i % 4], ys[i % 4])
    gpu.sync()
    settle = settle_clock(gpu, lambda i: mlp.step(xs[i % 4], ys[i % 4]))
    t0 = time.perf_counter()
    for i in range(steps):
        mlp.step(xs[i % 4], ys[i % 4])
    gpu.sync()
    ms = (time.perf_counter() - t0) / steps * 1e3
    flops = step_flops(dims, B)
    loss = mlp.last_loss()
    mlp.destroy()
    return {"config": "MLP 8x4096(ReLU) -> 1000, batch 4096, bf16 weights/activations, f32 master, "
                      "loss scale 1024, Adam(1e-3)", "ms_per_step": round(ms, 3),
            "tflops": round(flops / (ms * 1e-3) / 1e12, 1), "peak_tflops": PEAK_BF16_TFLOPS,
            "frac": round(flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4), "final_loss": round(float(loss), 4),
            **settle}


# examples/bench_grande.rs: N samples of D features, two ReLU layers of H,
# 10 classes, minibatches of LOTE, Adam(1e-3), softmax cross-entropy.
TAPE_N, TAPE_D, TAPE_H, TAPE_LOTE, TAPE_C = 4096, 128, 512, 256, 10


def tape_data():
    """bench_grande.rs:27-35: x[i][j] = sin(0.01 i + 0.03 j) (f32), label i % 10."""
    i = np.arange(TAPE_N, dtype=np.float32)[:, None]
    j = np.arange(TAPE_D, dtype=np.float32)[None, :]
    x = np.sin(i * np.float32(0.01) + j * np.float32(0.03)).astype(np.float32)
    y = np.zeros((TAPE_N, TAPE_C), np.float32)
    y[np.arange(TAPE_N), np.arange(TAPE_N) % TAPE_C] = 1.0
    return x, y


def tape_step_flops(rows):
    """bench_grande.rs:63-65: (D*H + H*H + H*C) MACs per sample, x3 fwd+bwd, x2."""
    return (TAPE_D * TAPE_H + TAPE_H * TAPE_H + TAPE_H * TAPE_C) * 3 * 2 * rows


def bench_tape(gpu, G, epochs=3):
    """bench_grande.rs on the device tape: a Sequential model recorded op by op
    (matmul, broadcast add, relu, softmax-xent) and Adam, every op a HIP
    launch; minibatches resident in HBM before the timed epochs."""
    from rgpu_amd import autograd as A

    x, y = tape_data()
    rng = np.random.default_rng(7)

    def glorot(d, h):
        lim = np.sqrt(6.0 / (d + h))
        return rng.uniform(-lim, lim, (d, h)).astype(np.float32)

    dims = [TAPE_D, TAPE_H, TAPE_H, TAPE_C]
    acts = ["relu", "relu", "linear"]
    model = A.Sequential([A.Dense(gpu, dims[k], dims[k + 1], acts[k], weights=glorot(dims[k], dims[k + 1]))
                          for k in range(3)])
    params = model.params()
    opt = A.Adam(1e-3)
    batches = [(gpu.upload(x[i:i + TAPE_LOTE]), gpu.upload(y[i:i + TAPE_LOTE]))
               for i in range(0, TAPE_N, TAPE_LOTE)]

    def epoch():
        loss = None
        for bx, by in batches:
            t = A.Tape(gpu)
            loss = A.softmax_cross_entropy(model.forward(t.constant(bx)), by)
            opt.step(params, loss.backward())
        return loss

    epoch()  # warm-up
    gpu.sync()
    t0 = time.perf_counter()
    for _ in range(epochs):
        loss = epoch()
    gpu.sync()
    wall = time.perf_counter() - t0
    steps = epochs * len(batches)
    # device time of the same work, and the per-kernel split, in one more epoch
    gpu.timer_begin()
    epoch()
    dev_ms = gpu.timer_end() / len(batches)
    gpu.profile_reset()
    gpu.profile(True)
    epoch()
    gpu.sync()
    prof = gpu.perfilar()
    gpu.profile(False)
    flops = tape_step_flops(TAPE_LOTE)
    ms = wall / steps * 1e3
    kern = sorted(((n, c, t) for n, c, t in prof), key=lambda r: -r[2])
    return {"config": f"bench_grande: N={TAPE_N} D={TAPE_D} H={TAPE_H} lote={TAPE_LOTE}, Sequential "
                      "Dense(relu) x2 + Dense(linear) -> softmax-xent, Adam(1e-3), device tape",
            "steps": steps, "ms_per_step": round(ms, 4), "device_ms_per_step": round(dev_ms, 4),
            "gflops": round(flops / (ms * 1e-3) / 1e9, 1), "launches_per_step": sum(c for _, c, _ in prof) // len(batches),
            "final_loss": round(loss.item(), 4),
            "kernels_ms_per_step": {n: round(t / len(batches), 4) for n, _, t in kern[:8]}}


def cpu_tape_baseline(budget_s=10.0):
    """bench_grande.rs on the oracle's tape (the reference's CPU path), 1 thread."""
    from oracle import oracle as O

    O.set_threads(1)
    x, y = tape_data()
    rng = O.Rng(7)
    layers = [O.Dense(TAPE_D, TAPE_H, "relu", rng), O.Dense(TAPE_H, TAPE_H, "relu", rng),
              O.Dense(TAPE_H, TAPE_C, "linear", rng)]
    model = O.Sequential(layers)
    params = model.params()
    opt = O.Optimizer("adam", 1e-3)
    t0 = time.perf_counter()
    n = 0
    for i in itertools.cycle(range(0, TAPE_N, TAPE_LOTE)):
        t = O.Tape()
        O.loss("softmax_cross_entropy", model.forward(t.constant(x[i:i + TAPE_LOTE])), y[i:i + TAPE_LOTE]).backward()
        opt.step(params, t)
        n += 1
        if time.perf_counter() - t0 > budget_s or n >= 48:
            break
    ms = (time.perf_counter() - t0) / n * 1e3
    return {"value": round(ms, 3), "unit": "ms/step", "cores": 1, "kind": "port",
            "sample": f"{n} minibatch steps of bench_grande (lote {TAPE_LOTE}) on the oracle tape, 1 thread"}


def bench_pcie(gpu, G, steps=50):
    """The batch-2048 f32 step with each batch coming from host memory
    (PCIe-inclusive; `value` never includes this): (a) rt_write of x and the
    labels into the batch buffers, then the step (the write waits for the
    previous step); (b) rt_mlp_load + rt_mlp_step_loaded, the copy of batch
    i+1 overlapping step i."""
    rng = np.random.default_rng(11)
    params = []
    for l in range(len(DIMS) - 1):
        params += [kaiming(rng, DIMS[l], DIMS[l + 1]), np.zeros((1, DIMS[l + 1]), np.float32)]
    xs = [rng.standard_normal((BATCH, DIMS[0]), dtype=np.float32) for _ in range(4)]
    ys = [rng.integers(0, DIMS[-1], BATCH) for _ in range(4)]
    ys32 = [y.astype(np.uint32) for y in ys]
    out = {}
    for mode in ("write_then_step", "overlapped_load"):
        mlp = G.GpuMlp.from_params(gpu, params, BATCH, 1e-3)
        xb, yb = gpu.zeros((BATCH, DIMS[0])), gpu.zeros((BATCH,), G.U32)

        def one(i):
            if mode == "write_then_step":
                gpu.write(xb, xs[i % 4])
                gpu.write(yb, ys32[i % 4])
                mlp.step(xb, yb)
            else:
                mlp.carregar(xs[i % 4], ys[i % 4])
                mlp.step_loaded()

        for i in range(5):
            one(i)
        gpu.sync()
        t0 = time.perf_counter()
        for i in range(steps):
            one(i)
        gpu.sync()
        out[mode + "_ms"] = round((time.perf_counter() - t0) / steps * 1e3, 4)
        mlp.destroy()
    out["batch_bytes"] = BATCH * DIMS[0] * 4 + BATCH * 4
    return out


def bench_copy(gpu, G, mib=256, reps=5):
    """A plain device copy of known size (f32 -> f32 through the convert
    kernel): reads and writes exactly mib MiB per launch.  Used to calibrate
    the FETCH_SIZE / WRITE_SIZE counters."""
    n = mib * 1024 * 1024 // 4
    src, dst = gpu.zeros((n,)), gpu.zeros((n,))
    for _ in range(reps):
        gpu.convert(src, dst)
    gpu.sync()
    return {"bytes_read_per_launch": n * 4, "bytes_written_per_launch": n * 4, "launches": reps}


def host_cpu():
    cpu = platform.processor() or platform.machine()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return cpu


def cpu_small_baseline(budget_s=3.0):
    """The oracle's batch-32 SGD step (tests/gpu.rs:116-121 order), 1 thread."""
    from oracle import oracle as O

    O.set_threads(1)
    rng = np.random.default_rng(32)
    params = []
    for l in range(len(DIMS) - 1):
        params += [kaiming(rng, DIMS[l], DIMS[l + 1]), np.zeros((1, DIMS[l + 1]), np.float32)]
    m = O.CpuMlp(params[0::2], params[1::2])
    m.set_optimizer("sgd", 0.01)
    x = rng.standard_normal((32, DIMS[0]), dtype=np.float32)
    y = rng.integers(0, DIMS[-1], 32).astype(np.uint32)
    t0 = time.perf_counter()
    n = 0
    while time.perf_counter() - t0 < budget_s and n < 400:
        m.step(x, y)
        n += 1
    ms = (time.perf_counter() - t0) / n * 1e3
    return {"value": round(ms, 3), "unit": "ms/step", "cores": 1, "kind": "port",
            "sample": f"{n} batch-32 SGD steps on the oracle, 1 thread on {host_cpu()}"}


def cpu_bwd_baseline(rows=512):
    """The CPU path of a Linear 4096->4096 backward (ops.rs:125-129: g·Wᵀ and
    Xᵀ·g, then reduce_to for db) on `rows` of the 8192 batch rows, 1 thread,
    scaled by 8192 / rows (every term is linear in the batch).  f32 on the
    same values (the CPU path has no bf16)."""
    from oracle import oracle as O

    O.set_threads(1)
    B, D = 8192, 4096
    rng = np.random.default_rng(3)
    x = rng.standard_normal((rows, D), dtype=np.float32) / np.float32(64.0)
    g = rng.standard_normal((rows, D), dtype=np.float32) / np.float32(64.0)
    w = rng.uniform(-np.sqrt(6.0 / D), np.sqrt(6.0 / D), size=(D, D)).astype(np.float32)
    wt = np.ascontiguousarray(w.T)
    t0 = time.perf_counter()
    O.matmul(g, wt)
    O.matmul(np.ascontiguousarray(x.T), g)
    O.reduce_to(g, (1, D))
    s = time.perf_counter() - t0
    ms = s * B / rows * 1e3
    return {"value": round(ms, 1), "unit": "ms per backward (dX + dW + db)", "cores": 1, "kind": "port",
            "sample": f"{rows} of the 8192 rows on the oracle (g·Wᵀ, Xᵀ·g, reduce_to), 1 thread, "
                      f"{s:.2f} s scaled x{B // rows}"}


def cpu_splitk_baseline(rows=16384):
    """dW = Xᵀ·dY and db = reduce_to(dY) on the oracle over `rows` of the
    262144 reduction rows, 1 thread, scaled by 262144 / rows."""
    from oracle import oracle as O

    O.set_threads(1)
    K, M, N = 262144, 512, 512
    rng = np.random.default_rng(4)
    x = rng.standard_normal((rows, M), dtype=np.float32) / np.float32(16.0)
    dy = rng.standard_normal((rows, N), dtype=np.float32) / np.float32(16.0)
    t0 = time.perf_counter()
    O.matmul(np.ascontiguousarray(x.T), dy)
    O.reduce_to(dy, (1, N))
    s = time.perf_counter() - t0
    return {"value": round(s * K / rows * 1e3, 1), "unit": "ms per dW + db", "cores": 1, "kind": "port",
            "sample": f"{rows} of the 262144 rows on the oracle, 1 thread, {s:.2f} s scaled x{K // rows}"}


def cpu_colsum_baseline(rows=32768):
    """reduce_to(dY, (1, 512)) on the oracle over `rows` of the 262144 rows
    (f32; the CPU path has no f16), 1 thread, scaled by 262144 / rows."""
    from oracle import oracle as O

    O.set_threads(1)
    K, N = 262144, 512
    dy = np.random.default_rng(5).standard_normal((rows, N), dtype=np.float32) / np.float32(16.0)
    t0 = time.perf_counter()
    O.reduce_to(dy, (1, N))
    s = time.perf_counter() - t0
    return {"value": round(s * K / rows * 1e3, 2), "unit": "ms per db of [262144, 512]", "cores": 1, "kind": "port",
            "sample": f"{rows} of the 262144 rows on the oracle, 1 thread, {s:.3f} s scaled x{K // rows}"}


def cpu_mixed_baseline(batches=(16, 48)):
    """One training step of the 8 x 4096 -> 1000 MLP on the oracle (f32, the
    CPU path has no bf16), 1 thread, at two small batches; the step time is
    a + b·batch (the Adam sweep over 138.3 M parameters and the per-step
    copies of the weights do not scale with the batch, the GEMMs do),
    extrapolated to batch 4096, after one untimed step."""
    from oracle import oracle as O

    O.set_threads(1)
    dims = [4096] * 9 + [1000]
    rng = np.random.default_rng(5)
    params = []
    for l in range(len(dims) - 1):
        params += [kaiming(rng, dims[l], dims[l + 1]), np.zeros((1, dims[l + 1]), np.float32)]
    m = O.CpuMlp(params[0::2], params[1::2])
    del params
    m.set_optimizer("adam", 1e-3)
    # the first step also allocates Adam's m and v (1.1 GB): not timed
    m.step(rng.standard_normal((batches[0], dims[0]), dtype=np.float32),
           rng.integers(0, dims[-1], batches[0]).astype(np.uint32))
    ts = []
    for b in batches:
        x = rng.standard_normal((b, dims[0]), dtype=np.float32)
        y = rng.integers(0, dims[-1], b).astype(np.uint32)
        t0 = time.perf_counter()
        m.step(x, y)
        ts.append(time.perf_counter() - t0)
    del m
    slope = (ts[1] - ts[0]) / (batches[1] - batches[0])
    fixed = ts[0] - slope * batches[0]
    full = fixed + slope * 4096
    return {"value": round(full * 1e3, 0), "unit": "ms/step", "cores": 1, "kind": "port",
            "sample": f"one oracle step at batch {batches[0]} ({ts[0]:.2f} s) and {batches[1]} ({ts[1]:.2f} s), "
                      f"1 thread; a + b·batch extrapolated to 4096 (a = {fixed:.2f} s, b = {slope * 1e3:.1f} ms/row)"}


def cpu_baseline(budget_s=12.0):
    """The oracle's single-threaded training step on the host, bounded sample."""
    from oracle import oracle as O

    O.set_threads(1)
    rng = np.random.default_rng(7)
    params = []
    for l in range(len(DIMS) - 1):
        params += [kaiming(rng, DIMS[l], DIMS[l + 1]), np.zeros((1, DIMS[l + 1]), np.float32)]
    m = O.CpuMlp(params[0::2], params[1::2])
    m.set_optimizer("adam", 1e-3)
    x = rng.standard_normal((BATCH, DIMS[0]), dtype=np.float32)
    y = rng.integers(0, DIMS[-1], BATCH).astype(np.uint32)
    t0 = time.perf_counter()
    n = 0
    while True:
        m.step(x, y)
        n += 1
        if time.perf_counter() - t0 > budget_s or n >= 20:
            break
    ms = (time.perf_counter() - t0) / n * 1e3
    cpu = host_cpu()
    return {"value": round(ms, 2), "unit": "ms/step", "cores": 1, "kind": "port",
            "sample": f"{n} steps of the batch-2048 Adam step, oracle C++ port of rtensor's CPU path, "
                      f"1 thread on {cpu} ({os.cpu_count()} logical CPUs visible)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", choices=["all", "step", "small", "bwd", "splitk", "colsum", "mixed", "copy", "tape",
                                       "pcie"],
                    default="all",
                    help="restrict the GPU work (for profiler passes); the JSON line needs 'all' or 'step'")
    ap.add_argument("--rounds", type=int, default=20,
                    help="rounds of the bf16 backward pair for --only bwd (more rounds hold the load for "
                         "power and clock sampling)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (the data-parallel "
              "all-reduce is not built).", file=sys.stderr)
        sys.exit(2)

    from rgpu_amd import gpu as G

    gpu = G.Gpu(0)
    if args.only in ("small", "bwd", "splitk", "colsum", "mixed", "copy", "tape", "pcie"):
        fn = {"small": bench_small, "bwd": bench_bwd_gemm, "splitk": bench_splitk, "colsum": bench_colsum,
              "mixed": bench_mixed, "copy": bench_copy, "tape": bench_tape, "pcie": bench_pcie}[args.only]
        if args.only == "bwd":
            res = fn(gpu, G, rounds=args.rounds)
        elif args.only == "small" and (args.steps, args.warmup) != (500, 200):  # explicit: a short leg for counters
            res = fn(gpu, G, steps=args.steps, warmup=args.warmup)
        else:
            res = fn(gpu, G)
        print(json.dumps({args.only: res}), flush=True)
        return
    wall, loss, prof, launches, settle = bench_step(gpu, G, args.steps, args.warmup)
    ms = wall / args.steps * 1e3
    total_flops = step_flops(DIMS, BATCH)

    kernels = {}
    dom = None
    for name, count, tot in prof:
        avg = tot / count
        kernels[name] = round(avg * 1e3, 2)  # µs per launch
        if dom is None or tot > dom[2]:
            dom = (name, count, tot)
    name, count, tot = dom
    avg_ms = tot / count
    flops = label_flops(name, DIMS, BATCH)
    if flops:
        achieved = flops / (avg_ms * 1e-3) / 1e12
        roof = {"kernel": name, "bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_F32_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / PEAK_F32_TFLOPS, 4), "traffic": traffic_for(name),
                "traffic_source": "profiles/pmc_traffic.json: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE of "
                                  "bench.py --only step, scaled by a copy kernel of known size",
                "flops_per_launch": flops, "avg_us": round(avg_ms * 1e3, 2)}
    else:
        roof = {"kernel": name, "bound": "hbm", "achieved": None, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": None, "traffic": traffic_for(name), "avg_us": round(avg_ms * 1e3, 2)}

    out = {
        "metric": "ms/step MLP 512-1024-1024-10 train @B=2048; bwd GEMM TFLOP/s % of peak",
        "value": round(ms, 4),
        "unit": "ms/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": round(ms / REF_GPU_MS_B2048, 4),
        "vs_baseline_ref": "rtensor wgpu step 6.89 ms at batch 2048 on an RTX 4070 Laptop (README.md:53)",
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "MLP 512-1024(ReLU)-1024(ReLU)-10 softmax-xent train step, f32, Adam",
                   "global_batch": BATCH, "dims": DIMS, "optimizer": "adam(1e-3,0.9,0.999,1e-8)",
                   "parallelism": "single GPU"},
        "step_tflops": round(total_flops / (ms * 1e-3) / 1e12, 2),
        "launches_per_step": launches,
        "final_loss": round(float(loss), 5),
        "roofline": roof,
        "kernels_us": kernels,
        "kernel_sum_us": round(sum(kernels.values()), 2),
        **settle,
    }
    if args.only == "all":
        out["small_batch"] = bench_small(gpu, G)
        out["bwd_gemm"] = bench_bwd_gemm(gpu, G)
        out["splitk_dw"] = bench_splitk(gpu, G)
        out["colsum"] = bench_colsum(gpu, G)
        out["mixed_mlp"] = bench_mixed(gpu, G)
        out["tape_mlp"] = bench_tape(gpu, G)
        out["pcie_inclusive"] = bench_pcie(gpu, G)
    if not args.no_cpu:
        cb = cpu_baseline()
        out["cpu_baseline"] = cb
        out["speedup_vs_cpu"] = round(cb["value"] / ms, 1)
        if "tape_mlp" in out:
            ct = cpu_tape_baseline()
            out["tape_mlp"]["cpu_baseline"] = ct
            out["tape_mlp"]["speedup_vs_cpu"] = round(ct["value"] / out["tape_mlp"]["ms_per_step"], 1)
        if "small_batch" in out:
            c = cpu_small_baseline()
            out["small_batch"]["cpu_baseline"] = c
            out["small_batch"]["speedup_vs_cpu"] = round(c["value"] / out["small_batch"]["ms_per_step"], 1)
        if "bwd_gemm" in out:
            c = cpu_bwd_baseline()
            out["bwd_gemm"]["cpu_baseline"] = c
            out["bwd_gemm"]["speedup_vs_cpu"] = round(c["value"] / (out["bwd_gemm"]["dX_ms"] +
                                                                    out["bwd_gemm"]["dW_db_ms"]), 1)
        if "splitk_dw" in out:
            c = cpu_splitk_baseline()
            out["splitk_dw"]["cpu_baseline"] = c
            out["splitk_dw"]["speedup_vs_cpu"] = round(c["value"] / out["splitk_dw"]["ms"], 1)
        if "colsum" in out:
            c = cpu_colsum_baseline()
            out["colsum"]["cpu_baseline"] = c
            out["colsum"]["speedup_vs_cpu"] = round(c["value"] / (out["colsum"]["f16_262144x512"]["us"] * 1e-3), 1)
        if "mixed_mlp" in out:
            c = cpu_mixed_baseline()
            out["mixed_mlp"]["cpu_baseline"] = c
            out["mixed_mlp"]["speedup_vs_cpu"] = round(c["value"] / out["mixed_mlp"]["ms_per_step"], 1)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
