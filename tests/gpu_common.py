"""Shared data builders for the GPU parity tests (seeded exactly like the
reference tests, tests/gpu.rs, and the configs the backend is measured on)."""
import os

import numpy as np

from oracle import oracle as O


def oracle_threads() -> int:
    # Row-parallel oracle is bit-identical for any thread count; the GPU box
    # gives a 16-CPU share.
    return max(1, min(16, os.cpu_count() or 1))


def quadrant_data(n=64, d=8):
    """gpu.rs:21-30: x_i = sin(0.37 i), label = quadrant of (x0, x1)."""
    x = np.sin(np.arange(n * d, dtype=np.float32) * np.float32(0.37)).astype(np.float32).reshape(n, d)
    lab = (x[:, 0] > 0).astype(np.uint32) + 2 * (x[:, 1] > 0).astype(np.uint32)
    return x, lab


def glorot_model(seed, dims):
    """Sequential of Dense layers with rtensor's Glorot init (nn.rs:122-130):
    ReLU hidden, linear output; returns the host params [W1, b1, ...]."""
    rng = O.Rng(seed)
    layers = [O.Dense(dims[i], dims[i + 1], "relu" if i < len(dims) - 2 else "linear", rng)
              for i in range(len(dims) - 1)]
    return [p.value() for l in layers for p in l.params()]


def kaiming_model(seed, dims):
    """Kaiming-uniform W ~ U(±sqrt(6/fan_in)) drawn row-major layer by layer
    from one Rng(seed); zero biases."""
    rng = O.Rng(seed)
    params = []
    for i in range(len(dims) - 1):
        params.append(O.kaiming_uniform(rng, dims[i], dims[i + 1]))
        params.append(np.zeros((1, dims[i + 1]), np.float32))
    return params


def normal_batch(seed, rows, cols):
    return O.Rng(seed).normals(rows * cols).reshape(rows, cols)


def uniform_labels(seed, rows, classes):
    return O.Rng(seed).belows(rows, classes)
