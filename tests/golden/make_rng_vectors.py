"""Writes rng_vectors.json: golden outputs of rtensor's Rng (src/rng.rs:3-49).

Computed here with Python integers and float64, independently of the C++
oracle: xorshift64* (shifts 12/25/27, multiplier 0x2545F4914F6CDD1D), the
24-bit uniform (u >> 40) / 2^24 (exact in f32), below(n) = u % n, and
Box-Muller normal values with f32 intermediates and correctly rounded
transcendentals (the oracle's libm result must agree to within 2 ulp).  Run: python tests/golden/make_rng_vectors.py
"""
import json
import math
import os

import numpy as np

MASK = (1 << 64) - 1


def stream(seed):
    s = 0x9E3779B97F4A7C15 if seed == 0 else seed
    while True:
        x = s
        x ^= x >> 12
        x ^= (x << 25) & MASK
        x ^= x >> 27
        s = x
        yield (x * 0x2545F4914F6CDD1D) & MASK


def main():
    out = {}
    for seed in (0, 1, 7, 42, 2024):
        g = stream(seed)
        u64 = [next(g) for _ in range(16)]
        g = stream(seed)
        unif = [(next(g) >> 40) / float(1 << 24) for _ in range(16)]
        g = stream(seed)
        below10 = [next(g) % 10 for _ in range(32)]
        g = stream(seed)
        normals = []
        f = np.float32
        for _ in range(16):
            # f32 at every step, as rng.rs:32-36 evaluates it; ln/cos/sqrt are
            # taken in float64 of the f32 argument and rounded back to f32.
            u1 = max(f((next(g) >> 40) / float(1 << 24)), f(1e-7))
            u2 = f((next(g) >> 40) / float(1 << 24))
            ln_u1 = f(math.log(float(u1)))
            rad = f(math.sqrt(float(f(-2.0) * ln_u1)))
            arg = (f(2.0) * f(math.pi)) * u2
            cs = f(math.cos(float(arg)))
            normals.append(float(rad * cs))
        g = stream(seed)
        # range(-λ, λ) for the Glorot bound of Dense(8, 16): λ = sqrt(6/24) in f32
        lam = np.float32(np.sqrt(np.float32(6.0) / np.float32(24.0), dtype=np.float32))
        rng_vals = []
        for _ in range(16):
            u = np.float32((next(g) >> 40) / float(1 << 24))
            rng_vals.append(float(np.float32(-lam) + u * (lam - np.float32(-lam))))
        out[str(seed)] = {"u64": [str(v) for v in u64], "uniform": unif, "below10": below10,
                          "normal_f64": normals, "glorot_8_16": rng_vals}
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "rng_vectors.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
    print(path)


if __name__ == "__main__":
    main()
