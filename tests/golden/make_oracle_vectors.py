"""Writes oracle_vectors.json: the oracle's outputs on the MLP cases the GPU
tests use, as regression fixtures.

Cases (inputs from rtensor's Rng, whose stream is pinned by rng_vectors.json):

* ``gpu_rs_tiny``: the model of crates/rtensor/tests/gpu.rs:13-37, 8 -> 16 -> 16
  -> 4 (ReLU hidden, linear output) with Glorot weights from Rng(42) and the
  quadrant data of gpu.rs:21-30 (64 rows); one step without an update.
* ``gpu_rs_split_k``: gpu.rs:147-170's 8 -> 128 -> 4 model on 512 quadrant
  rows, Glorot from Rng(7), one Adam(0.05) step.
* ``config_b32_sgd``: MLP 512 -> 1024 -> 1024 -> 10 at batch 32, Kaiming-
  uniform weights from Rng(1), zero biases, x = Rng(101) normals, labels =
  Rng(102) below(10), one SGD(0.01) step.

For each: the loss (f32 bits), and per gradient (and, after an update, per
updated parameter) its shape, the SHA-256 of its f32 bytes and up to 64
strided samples (index, f32 bits).  The digests pin the oracle bit for bit
against later changes to it; the samples are what the GPU tests compare
their own results against, at the tolerances the reference's tests use.

Run: python tests/golden/make_oracle_vectors.py
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as O  # noqa: E402
from tests.gpu_common import glorot_model, kaiming_model, normal_batch, quadrant_data, uniform_labels  # noqa: E402


def cases():
    """(name, params, x, labels, optimizer, lr) for every case."""
    x, lab = quadrant_data()
    yield "gpu_rs_tiny", glorot_model(42, [8, 16, 16, 4]), x, lab, "none", 0.0
    x, lab = quadrant_data(512, 8)
    yield "gpu_rs_split_k", glorot_model(7, [8, 128, 4]), x, lab, "adam", 0.05
    dims = [512, 1024, 1024, 10]
    yield ("config_b32_sgd", kaiming_model(1, dims), normal_batch(101, 32, 512), uniform_labels(102, 32, 10),
           "sgd", 0.01)


def bits(v) -> str:
    return "%08x" % int(np.float32(v).view(np.uint32))


def describe(a: np.ndarray) -> dict:
    a = np.ascontiguousarray(a, np.float32)
    flat = a.reshape(-1)
    stride = max(1, flat.size // 64)
    idx = list(range(0, flat.size, stride))[:64]
    return {"shape": list(a.shape), "sha256": hashlib.sha256(flat.tobytes()).hexdigest(),
            "samples": [[i, bits(flat[i])] for i in idx]}


def run_case(params, x, lab, opt, lr) -> dict:
    m = O.CpuMlp(params[0::2], params[1::2])
    m.set_optimizer(opt, lr)
    loss = m.step(x, lab)
    out = {"loss": bits(loss), "grads": [describe(g) for g in m.grads()]}
    if opt != "none":
        out["weights"] = [describe(w) for w in m.weights()]
    out["inputs_sha256"] = hashlib.sha256(b"".join(np.ascontiguousarray(a, np.float32).tobytes()
                                                   for a in list(params) + [x])
                                          + np.ascontiguousarray(lab, np.uint32).tobytes()).hexdigest()
    return out


def build() -> dict:
    return {name: dict(run_case(p, x, lab, opt, lr), optimizer=opt, lr=lr)
            for name, p, x, lab, opt, lr in cases()}


def main():
    with open(os.path.join(HERE, "oracle_vectors.json"), "w") as f:
        json.dump(build(), f, indent=1)
        f.write("\n")


if __name__ == "__main__":
    main()
