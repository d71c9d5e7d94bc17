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


def numpy_f32_trajectory(params, batches, lr, beta1=0.9, beta2=0.999, eps=1e-8, optimizer="adam", momentum=0.0,
                         return_state=False):
    """The same training step written directly in float32 numpy (BLAS GEMM
    order, pairwise sums): an independent f32 implementation whose distance
    from the oracle measures how much the trajectory moves under a change of
    summation order alone.  Adam (optim.rs:187-195 expression order) or SGD
    with momentum (optim.rs:88-103).  Returns final params and per-step
    losses, and with return_state also (m, v): Adam's moments, or the SGD
    velocity and zeros."""
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
            if optimizer == "adam":
                m[i] = m[i] * f(beta1) + g * (f(1) - f(beta1))
                v[i] = v[i] * f(beta2) + (g * g) * (f(1) - f(beta2))
                ps[i] -= ((m[i] * (f(1) / c1)) / (np.sqrt(v[i] * (f(1) / c2)) + f(eps))) * f(lr)
            elif momentum == 0.0:
                ps[i] -= g * f(lr)
            else:
                m[i] = m[i] * f(momentum) + g * f(lr)
                ps[i] -= m[i]
    if return_state:
        return ps, losses, m, v
    return ps, losses


def numpy_f32_grads(params, x, lab):
    """One step's gradients of the ReLU MLP with softmax cross-entropy in
    float32 numpy (BLAS summation order): an independent f32 implementation,
    whose distance from the oracle measures the conditioning of the step."""
    f = np.float32
    Ws = [p.astype(f) for p in params[0::2]]
    bs = [p.astype(f).reshape(1, -1) for p in params[1::2]]
    acts = [np.asarray(x, f)]
    for l in range(len(Ws)):
        z = acts[-1] @ Ws[l] + bs[l]
        acts.append(np.maximum(z, f(0)) if l < len(Ws) - 1 else z)
    z = acts[-1]
    e = np.exp(z - z.max(1, keepdims=True))
    p = e / e.sum(1, keepdims=True)
    B = z.shape[0]
    d = ((p - np.eye(z.shape[1], dtype=f)[lab]) * f(1.0 / B)).astype(f)
    grads = [None] * (2 * len(Ws))
    for l in reversed(range(len(Ws))):
        grads[2 * l] = acts[l].T @ d
        grads[2 * l + 1] = d.sum(0, keepdims=True)
        if l > 0:
            d = (d @ Ws[l].T) * (acts[l] > 0)
    return grads


def bf16_pipeline_grads(params, x, lab, loss_scale=1024.0, col_frac=None, seed=0):
    """Step-1 gradients of the ReLU MLP computed in float64 with the rounding
    points of the mixed-precision plan: bf16 weights and inputs, hidden
    activations stored as bf16 (round to nearest even), δ stored as bf16 after
    the loss and after every ReLU mask; gradients unscaled at the end.  An
    independent restatement of what the bf16 training step computes.

    With col_frac, each dW is computed only on a random subset of its
    columns (that fraction, at least 64) and returned with the column
    indices: [(dW[:, cols], cols), db, ...] -- the forward and δ chains stay
    whole."""
    from rgpu_amd.gpu import bf16_bits_to_f32, f32_to_bf16_bits

    def rb(a):
        return bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(a, np.float32))).astype(np.float64)

    rng = np.random.default_rng(seed)
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
        if col_frac is None:
            grads[2 * l] = acts[l].T @ d / loss_scale
        else:
            n = d.shape[1]
            cols = np.sort(rng.choice(n, min(n, max(64, int(n * col_frac))), replace=False))
            grads[2 * l] = (acts[l].T @ d[:, cols] / loss_scale, cols)
        grads[2 * l + 1] = d.sum(0, keepdims=True) / loss_scale
        if l > 0:
            d = rb((d @ Ws[l].T) * (acts[l] > 0))
    return grads


def bf16_pipeline_loss(params, x, lab):
    """The mean softmax cross-entropy of one forward pass of the bf16 plan,
    restated in float64: bf16 (round to nearest even) weights and inputs,
    hidden activations stored as bf16 after the ReLU, float64 accumulation,
    logits and softmax, and rtensor's row loss −ln(max(p_y, 1e-12))
    (losses.rs:99-115), which caps a row at 27.63 once the logits are large.
    params are f32 master weights; x f32."""
    from rgpu_amd.gpu import bf16_bits_to_f32, f32_to_bf16_bits

    def rb(a):
        return bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(a, np.float32))).astype(np.float64)

    Ws = [rb(p) for p in params[0::2]]
    bs = [np.asarray(p, np.float64).reshape(1, -1) for p in params[1::2]]
    a = rb(x)
    for l in range(len(Ws)):
        z = a @ Ws[l] + bs[l]
        a = rb(np.maximum(z, 0)) if l < len(Ws) - 1 else z
    m = a.max(1, keepdims=True)
    lse = m[:, 0] + np.log(np.exp(a - m).sum(1))
    p_y = np.exp(a[np.arange(a.shape[0]), lab] - lse)
    return float((-np.log(np.maximum(p_y, 1e-12))).mean())


def bf16_plan_layer_checks(mlp, params, x, lab, loss_scale, n_rows=64, n_entries=256, seed=0):
    """Checks each GEMM and rounding point of one bf16 training step of the
    plan on the plan's OWN stored inputs (rt_mlp_activation / rt_mlp_delta),
    per element against float64, so that no perturbation is carried from one
    layer to the next (the ReLU masks are the plan's own):

    * forward, sampled rows: A_l = bf16(ReLU(A_{l-1}·W_l + b_l)) within one
      bf16 rounding (2⁻⁸ relative) plus f32 accumulation (1e-5 of the sum
      of |terms|); the f32 logits within the accumulation bound;
    * loss: δ_L = bf16((softmax(z) − onehot)·scale/B) from the plan's logits;
    * backward, sampled rows: δ_{l-1} = bf16((δ_l·W_lᵀ) ⊙ 1[A_{l-1} > 0]),
      exactly 0 where the mask is 0;
    * dW_l = A_{l-1}ᵀ·δ_l / scale on sampled entries and db_l = 1ᵀ·δ_l / scale
      whole, within the accumulation bound.
    params are the f32 master weights the step started from (W rounded to
    bf16 here, as the plan's copy is); x the f32 batch (rounded here)."""
    from rgpu_amd.gpu import bf16_bits_to_f32, f32_to_bf16_bits

    def rb(a):
        return bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(a, np.float32))).astype(np.float64)

    u, acc = 2.0 ** -8, 1e-5
    rng = np.random.default_rng(seed)
    Ws = [rb(p) for p in params[0::2]]
    bs = [np.asarray(p, np.float64).reshape(1, -1) for p in params[1::2]]
    L, B = len(Ws), x.shape[0]
    A = [rb(x)] + [mlp.activation(l).astype(np.float64) for l in range(L)]
    D = [mlp.delta(l).astype(np.float64) for l in range(L)]
    grads = mlp.grads()
    rows = np.sort(rng.choice(B, min(B, n_rows), replace=False))
    worst = {}

    def check(tag, got, want, bound):
        r = np.abs(got - want) / np.maximum(bound, 1e-300)
        worst[tag] = float(r.max()) if r.size else 0.0
        assert np.all(np.abs(got - want) <= bound), f"{tag}: worst |err|/bound {worst[tag]:.2f}"

    for l in range(L):
        a = A[l][rows]
        z = a @ Ws[l] + bs[l]
        s = np.abs(a) @ np.abs(Ws[l]) + np.abs(bs[l])
        got = A[l + 1][rows]
        if l < L - 1:
            want = np.maximum(z, 0.0)
            check(f"fwd{l}", got, want, u * want + 2 * acc * s)
        else:
            check(f"logits", got, z, acc * s)
    z = A[L]
    p = np.exp(z - z.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    want = (p - np.eye(z.shape[1])[lab]) * (loss_scale / B)
    check("xent", D[L - 1], want, u * np.abs(want) + 1e-5 * loss_scale / B)
    for l in range(L - 1, 0, -1):
        d = D[l][rows]
        g = d @ Ws[l].T
        s = np.abs(d) @ np.abs(Ws[l]).T
        mask = A[l][rows] > 0
        got = D[l - 1][rows]
        check(f"bwd{l}", got, g * mask, (u * np.abs(g) + 2 * acc * s) * mask)
    for l in range(L):
        din, dout = Ws[l].shape
        pi, qi = rng.integers(0, din, n_entries), rng.integers(0, dout, n_entries)
        prod = A[l][:, pi] * D[l][:, qi]
        check(f"dW{l}", grads[2 * l].astype(np.float64)[pi, qi], prod.sum(0) / loss_scale,
              acc * np.abs(prod).sum(0) / loss_scale)
        check(f"db{l}", grads[2 * l + 1].astype(np.float64).reshape(-1), D[l].sum(0) / loss_scale,
              acc * np.abs(D[l]).sum(0) / loss_scale + 1e-30)
    print("layer-local checks, worst |err|/bound:", {k: round(v, 3) for k, v in worst.items()}, flush=True)
    return worst


def gate_rows(want, got, floor=1e-3):
    """Per tensor: (norm-wise, max-relative, elementwise over |want| >
    floor·max|want|, erro_rel) distance of got from want."""
    rows = []
    for a, b in zip(want, got):
        a64 = np.asarray(a, np.float64)
        b64 = np.asarray(b, np.float64).reshape(a64.shape)
        d = np.abs(b64 - a64)
        na, ma = float(np.linalg.norm(a64)), float(np.abs(a64).max()) if a64.size else 0.0
        nd, md = float(np.linalg.norm(d)), float(d.max()) if d.size else 0.0
        nw = nd / na if na > 0 else (0.0 if nd == 0 else float("inf"))
        mx = md / ma if ma > 0 else (0.0 if md == 0 else float("inf"))
        big = np.abs(a64) > floor * ma
        el = float((d[big] / np.abs(a64[big])).max()) if big.any() else 0.0
        rows.append((nw, mx, el, O.erro_rel(a64, b64)))
    return rows


def grad_gate(name, want, got, norm_bound, max_bound, erro_bound=None, floor=1e-3, ref=None, ref_factor=3.0):
    """Scale-aware parity gate, per tensor of the lists want (reference) and
    got: norm-wise ‖got − want‖/‖want‖ <= norm_bound and max|got − want| /
    max|want| <= max_bound.  Unlike the reference's erro_rel
    (|x − y|/(1 + max(|x|, |y|)), gpu.rs:53-60), which is an absolute error for
    values far below 1, a wrong or zeroed tensor scores ~1 on both, whatever
    its scale.  Bounds may be scalars or per-tensor lists; erro_bound (scalar
    or list), if given, also gates erro_rel.  Also reports the elementwise relative error
    over the entries with |want| > floor·max|want|.

    ref, if given, is an independent implementation of the same computation
    (another summation order): where the problem itself is ill-conditioned
    (ReLU pre-activations within rounding of zero flip their mask under any
    reordering) each bound becomes max(bound, ref_factor x ref's own distance
    from want).  Returns the rows (norm, max, elementwise, erro_rel)."""
    n = len(want)
    nb = norm_bound if isinstance(norm_bound, (list, tuple)) else [norm_bound] * n
    mb = max_bound if isinstance(max_bound, (list, tuple)) else [max_bound] * n
    eb = erro_bound if isinstance(erro_bound, (list, tuple)) else [erro_bound] * n
    if ref is not None:
        rr = gate_rows(want, ref, floor)
        nb = [max(b, ref_factor * r[0]) for b, r in zip(nb, rr)]
        mb = [max(b, ref_factor * r[1]) for b, r in zip(mb, rr)]
        print(f"{name}: conditioning (independent implementation vs reference): norm-wise",
              ["%.1e" % r[0] for r in rr], "max-relative", ["%.1e" % r[1] for r in rr], flush=True)
    rows = gate_rows(want, got, floor)
    print(f"{name}: norm-wise", ["%.1e" % r[0] for r in rows], "\n  max-relative", ["%.1e" % r[1] for r in rows],
          "\n  elementwise (|y| > %.0e max)" % floor, ["%.1e" % r[2] for r in rows],
          "\n  erro_rel", ["%.1e" % r[3] for r in rows], flush=True)
    for i, r in enumerate(rows):
        assert r[0] <= nb[i], f"{name}[{i}]: norm-wise {r[0]:.3e} > {nb[i]:.1e}"
        assert r[1] <= mb[i], f"{name}[{i}]: max-relative {r[1]:.3e} > {mb[i]:.1e}"
        if eb[i] is not None:
            assert r[3] <= eb[i], f"{name}[{i}]: erro_rel {r[3]:.3e} > {eb[i]:.1e}"
    return rows


def numpy_bf16_trajectory(params, batches, lr, loss_scale=1024.0, acc="f32", beta1=0.9, beta2=0.999, eps=1e-8):
    """The bf16 mixed-precision training step restated in numpy: f32 master
    weights and Adam (optim.rs:187-195 order), bf16 (round to nearest even)
    copies of the weights, the inputs, the hidden activations (after ReLU)
    and δ (after the loss, scaled by loss_scale, and after every ReLU mask),
    f32 logits and softmax, gradients unscaled by 1/loss_scale.  The GEMMs
    accumulate in float32 (acc="f32", BLAS order) or float64 (acc="f64") and
    round to f32: two independent implementations of the plan's rounding
    points that differ only in accumulation order.  Returns the per-step
    losses."""
    from rgpu_amd.gpu import bf16_bits_to_f32, f32_to_bf16_bits

    def rb(a):
        return bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(a, np.float32)))

    def mm(a, b):
        if acc == "f64":
            return (a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32)
        return a @ b

    f = np.float32
    S = f(loss_scale)
    ps = [np.asarray(p, np.float32).copy() for p in params]
    for i in range(1, len(ps), 2):
        ps[i] = ps[i].reshape(1, -1)
    m = [np.zeros_like(p) for p in ps]
    v = [np.zeros_like(p) for p in ps]
    losses = []
    for t, (x, lab) in enumerate(batches, start=1):
        Wh = [rb(W) for W in ps[0::2]]
        acts = [rb(x)]
        for l in range(len(Wh)):
            z = mm(acts[-1], Wh[l]) + ps[2 * l + 1]
            acts.append(rb(np.maximum(z, f(0))) if l < len(Wh) - 1 else z)
        z = acts[-1]
        e = np.exp(z - z.max(1, keepdims=True))
        p = e / e.sum(1, keepdims=True)
        B = z.shape[0]
        losses.append(float(-np.log(np.maximum(p[np.arange(B), lab], f(1e-12))).astype(np.float64).mean()))
        d = rb((p - np.eye(z.shape[1], dtype=f)[lab]) * f(S / B))
        g = [None] * len(ps)
        for l in reversed(range(len(Wh))):
            g[2 * l] = mm(acts[l].T, d) * f(1 / S)
            g[2 * l + 1] = d.sum(0, keepdims=True) * f(1 / S)
            if l > 0:
                d = rb(mm(d, Wh[l].T) * (acts[l] > 0))
        c1 = f(1) - f(beta1) ** t
        c2 = f(1) - f(beta2) ** t
        for i, gi in enumerate(g):
            m[i] = m[i] * f(beta1) + gi * (f(1) - f(beta1))
            v[i] = v[i] * f(beta2) + (gi * gi) * (f(1) - f(beta2))
            ps[i] -= ((m[i] * (f(1) / c1)) / (np.sqrt(v[i] * (f(1) / c2)) + f(eps))) * f(lr)
    return losses
