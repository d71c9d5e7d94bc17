"""Shared data builders for the GPU parity tests (seeded exactly like the
reference tests, tests/gpu.rs, and the configs the backend is measured on)."""
import os

import numpy as np

from oracle import oracle as O


def oracle_threads() -> int:
    # Row-parallel oracle is bit-identical for any thread count; at most 16
    # threads, the CPU share of a one-GPU host.
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


def numpy_f32_trajectory(params, batches, lr, beta1=0.9, beta2=0.999, eps=1e-8):
    """The same training step written directly in float32 numpy (BLAS GEMM
    order, pairwise sums): an independent f32 implementation whose distance
    from the oracle measures how much the trajectory moves under a change of
    summation order alone.  Returns final params and per-step losses."""
    Ws = [p.astype(np.float32).copy() for p in params[0::2]]
    bs = [p.astype(np.float32).reshape(1, -1).copy() for p in params[1::2]]
    ps = [a for pair in zip(Ws, bs) for a in pair]
    m = [np.zeros_like(p) for p in ps]
    v = [np.zeros_like(p) for p in ps]
    f = np.float32
    losses = []
    for t, (x, lab) in enumerate(batches, start=1):
        acts = [x.astype(np.float32)]
        for l in range(len(Ws)):
            z = acts[-1] @ Ws[l] + bs[l]
            acts.append(np.maximum(z, f(0)) if l < len(Ws) - 1 else z)
        z = acts[-1]
        e = np.exp(z - z.max(1, keepdims=True))
        p = e / e.sum(1, keepdims=True)
        B = z.shape[0]
        losses.append(float(-np.log(np.maximum(p[np.arange(B), lab], f(1e-12))).astype(np.float64).mean()))
        delta = ((p - np.eye(z.shape[1], dtype=np.float32)[lab]) * f(1.0 / B)).astype(np.float32)
        grads = [None] * len(ps)
        for l in reversed(range(len(Ws))):
            grads[2 * l] = acts[l].T @ delta
            grads[2 * l + 1] = delta.sum(0, keepdims=True)
            if l > 0:
                delta = (delta @ Ws[l].T) * (acts[l] > 0)
        c1 = f(1) - f(beta1) ** t
        c2 = f(1) - f(beta2) ** t
        for i, g in enumerate(grads):
            m[i] = m[i] * f(beta1) + g * (f(1) - f(beta1))
            v[i] = v[i] * f(beta2) + (g * g) * (f(1) - f(beta2))
            ps[i] -= ((m[i] * (f(1) / c1)) / (np.sqrt(v[i] * (f(1) / c2)) + f(eps))) * f(lr)
    return ps, losses


def bf16_pipeline_grads(params, x, lab, loss_scale=1024.0):
    """Step-1 gradients of the ReLU MLP computed in float64 with the rounding
    points of the mixed-precision plan: bf16 weights and inputs, hidden
    activations stored as bf16 (round to nearest even), δ stored as bf16 after
    the loss and after every ReLU mask; gradients unscaled at the end.  An
    independent restatement of what the bf16 training step computes."""
    from rgpu_amd.gpu import bf16_bits_to_f32, f32_to_bf16_bits

    def rb(a):
        return bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(a, np.float32))).astype(np.float64)

    Ws = [rb(p) for p in params[0::2]]
    bs = [np.asarray(p, np.float64).reshape(1, -1) for p in params[1::2]]
    acts = [rb(x)]
    for l in range(len(Ws)):
        z = acts[-1] @ Ws[l] + bs[l]
        acts.append(rb(np.maximum(z, 0)) if l < len(Ws) - 1 else z)
    z = acts[-1]
    p = np.exp(z - z.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    B = z.shape[0]
    d = rb((p - np.eye(z.shape[1])[lab]) * (loss_scale / B))
    grads = [None] * (2 * len(Ws))
    for l in reversed(range(len(Ws))):
        grads[2 * l] = acts[l].T @ d / loss_scale
        grads[2 * l + 1] = d.sum(0, keepdims=True) / loss_scale
        if l > 0:
            d = rb((d @ Ws[l].T) * (acts[l] > 0))
    return grads
