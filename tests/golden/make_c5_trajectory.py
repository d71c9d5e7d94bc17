"""Writes c5_trajectory.json: the oracle's per-step losses of 100 Adam steps of
the 8-hidden-layer 4096-wide ReLU MLP -> 1000 classes at batch 4096, the
configuration the bf16 training plan is measured on.  The GPU test runs the
same 100 steps in bf16 (f32 master weights, loss scale 1024) and checks every
loss against these.

Inputs (all from rtensor's Rng, whose stream is pinned by rng_vectors.json):
* weights: Kaiming-uniform U(±sqrt(6/fan_in)) drawn row-major layer by layer
  from Rng(6), then rounded to bf16 (round to nearest even), as the bf16
  plan holds them; biases zero;
* step s (0-based): x = Rng(7000 + s) normals [4096, 4096] rounded to bf16,
  labels = Rng(8000 + s) below(1000).
The oracle trains in f32 from these rounded values: tape forward, softmax
cross-entropy, backward, Adam(1e-3, 0.9, 0.999, 1e-8) (tests/gpu.rs:116-121).
Its matmul is row-parallel, which is bit-identical to the single-threaded
one (each element's k order is unchanged), so any thread count gives these
losses.

The conditioning of that trajectory: the same 100 steps through two
independent numpy restatements of the bf16 plan's rounding points
(tests/gpu_common.numpy_bf16_trajectory, float32 and float64 accumulation).
Early on the loss spikes (7.96 -> 26 -> 13.8 -> 7.3) and the spike amplifies
step-1 differences ~100x: valid bf16 implementations land several percent
apart there, so the GPU test bounds each step by max(2e-2, 2 x the farther
restatement's distance from the oracle).

Run: python tests/golden/make_c5_trajectory.py [threads]        (~30 s per step on 8)
     python tests/golden/make_c5_trajectory.py --restatements   (adds them, ~45 min)
"""
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as O  # noqa: E402
from rgpu_amd.gpu import bf16_bits_to_f32, f32_to_bf16_bits  # noqa: E402
from tests.gpu_common import kaiming_model, normal_batch, uniform_labels  # noqa: E402

DIMS = [4096] * 9 + [1000]
BATCH = 4096
STEPS = 100
LR = 1e-3
WEIGHT_SEED = 6
X_SEED0, LABEL_SEED0 = 7000, 8000
OUT = os.path.join(HERE, "c5_trajectory.json")


def bf16_round(a):
    return bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(a, np.float32)))


def initial_params():
    params = kaiming_model(WEIGHT_SEED, DIMS)
    return [bf16_round(p) if i % 2 == 0 else p for i, p in enumerate(params)]


def batch(s):
    x = bf16_round(normal_batch(X_SEED0 + s, BATCH, DIMS[0]))
    return x, uniform_labels(LABEL_SEED0 + s, BATCH, DIMS[-1])


def main(threads):
    O.set_threads(threads)
    params = initial_params()
    cpu = O.CpuMlp(params[0::2], params[1::2])
    cpu.set_optimizer("adam", LR)
    losses = []
    t0 = time.time()
    for s in range(STEPS):
        x, lab = batch(s)
        losses.append(float(cpu.step(x, lab)))
        print(f"step {s}: loss {losses[-1]:.6f} ({time.time() - t0:.0f} s)", flush=True)
    doc = {
        "config": {"dims": DIMS, "batch": BATCH, "steps": STEPS, "optimizer": "adam", "lr": LR,
                   "beta1": 0.9, "beta2": 0.999, "eps": 1e-8, "weight_seed": WEIGHT_SEED,
                   "x_seed0": X_SEED0, "label_seed0": LABEL_SEED0,
                   "rounding": "weights and inputs rounded to bf16 (RNE); oracle in f32"},
        # f32 bits of each loss, and the decimal value for reading
        "loss_bits": [int(np.float32(v).view(np.uint32)) for v in losses],
        "loss": losses,
    }
    with open(OUT, "w") as f:
        json.dump(doc, f, indent=1)
    print("wrote", OUT)


def restatements():
    from tests.gpu_common import numpy_bf16_trajectory

    with open(OUT) as f:
        doc = json.load(f)
    params = initial_params()
    for acc in ("f32", "f64"):
        t0 = time.time()
        losses = numpy_bf16_trajectory(params, (batch(s) for s in range(STEPS)), LR, acc=acc)
        doc[f"bf16_restatement_{acc}_acc"] = losses
        print(f"bf16 restatement, {acc} accumulation: {time.time() - t0:.0f} s", flush=True)
    with open(OUT, "w") as f:
        json.dump(doc, f, indent=1)
    print("wrote", OUT)


if __name__ == "__main__":
    if len(sys.argv) > 1 and sys.argv[1] == "--restatements":
        restatements()
    else:
        main(int(sys.argv[1]) if len(sys.argv) > 1 else (os.cpu_count() or 1))
