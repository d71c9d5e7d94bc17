"""The half-precision configurations the backend is measured on:
  * split-K weight gradient: dW = Xᵀ·dY with reduction length 262144, X and dY
    f16 ~N(0,1)/16 [262144, 512], f32 accumulate and output, db = colsum(dY);
  * Linear 4096->4096 backward at batch 8192 in bf16: dX = dY·Wᵀ, dW = Xᵀ·dY,
    db = colsum(dY), f32 accumulate;
  * the 8-layer 4096-wide ReLU MLP -> 1000 classes, batch 4096, bf16
    activations/weights with f32 master weights, static loss scale 1024 and
    fused Adam.
The CPU reference is the oracle in f32 on the same rounded inputs
(crates/rtensor/src/tensor.rs:318-373 order); half paths must stay within
2e-2 relative of it and loss trajectories must track it."""
import time

import numpy as np
import pytest

from oracle import oracle as O
from rgpu_amd import gpu as G
from tests.gpu_common import (bf16_pipeline_grads, bf16_pipeline_loss, bf16_plan_layer_checks, grad_gate,
                              kaiming_model, normal_batch, oracle_threads, uniform_labels)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gpu():
    O.set_threads(oracle_threads())
    g = G.Gpu(0)
    yield g
    g.close()
    O.set_threads(1)


def f16_round(a):
    return a.astype(np.float16).astype(np.float32)


def bf16_round(a):
    return G.bf16_bits_to_f32(G.f32_to_bf16_bits(a))


@pytest.mark.parametrize("K,slices", [(262144, 32), (262144, 64), (8192, 8), (70001, 16)])
def test_splitk_dw_f16(gpu, K, slices):
    M = N = 512
    t0 = time.time()
    x = f16_round(normal_batch(31, K, M) / np.float32(16))
    dy = f16_round(normal_batch(32, K, N) / np.float32(16))
    gx, gdy = gpu.upload(x, G.F16), gpu.upload(dy, G.F16)
    dw, db = gpu.zeros((M, N)), gpu.zeros((1, N))
    part = gpu.zeros((slices * (M * N + N),))
    gpu.split_k(gx, gdy, dw, part, slices, True, colsum=db)
    got_w, got_b = gpu.download(dw), gpu.download(db)
    # the oracle on the same f16-rounded inputs, in f32 (sequential k)
    want_w = O.matmul(np.ascontiguousarray(x.T), dy)
    want_b = O.reduce_to(dy, (1, N))
    ex_w = x.T.astype(np.float64) @ dy.astype(np.float64)
    ex_b = dy.astype(np.float64).sum(0, keepdims=True)
    e_w, e_b = O.erro_rel(want_w, got_w), O.erro_rel(want_b, got_b)
    xw, xb = O.erro_rel(ex_w, got_w), O.erro_rel(ex_b, got_b)
    cw, cb = O.erro_rel(ex_w, want_w), O.erro_rel(ex_b, want_b)
    print(f"K={K} slices={slices}: dW vs oracle {e_w:.2e} (vs exact {xw:.2e}, oracle vs exact {cw:.2e}); "
          f"db vs oracle {e_b:.2e} (vs exact {xb:.2e}, oracle {cb:.2e}); {time.time() - t0:.1f}s")
    assert e_w < 1e-4 and e_b < 1e-4
    assert xw <= max(1e-5, 3 * cw) and xb <= max(1e-5, 3 * cb)
    # deterministic
    dw2 = gpu.zeros((M, N))
    gpu.split_k(gx, gdy, dw2, part, slices, True)
    assert np.array_equal(gpu.download(dw2), got_w)


def bf16_gates(mlp, cpu, params_r, x, lab, col_frac=None, emu_bound=None):
    """Gradient gates of one step of the bf16 plan.

    1. Layer-local: every GEMM and rounding point of the step on the plan's
       own stored inputs, per element against float64 (pins the kernels).
    2. Against the f32 oracle (the 2e-2 bar), scale-aware: per tensor
       norm-wise and max-relative distance.  bf16 activation storage alone
       flips ReLU masks (~0.1% of them at these sizes), which moves the first
       layers' gradients up to ~12% norm-wise from f32; the float64
       restatement of the bf16 pipeline measures that inherent distance for
       each tensor, and the plan may deviate from f32 by at most
       max(2e-2, 2 x) it.  A zeroed or wrong tensor scores ~1.  erro_rel
       (tests/gpu.rs:53-60) is gated the same way: it is an absolute error
       while gradients are far below 1, so the 2e-2 floor decides at step 0,
       but in the loss spike of the 8 x 4096 model (step 1: loss 26) the
       gradients are O(1) and the restatement itself is up to ~0.19 from f32
       on it.
    3. Optionally (small widths, where f32-vs-float64 accumulation does not
       flip masks) norm-wise against that restatement itself."""
    gg, gc = mlp.grads(), cpu.grads()
    bf16_plan_layer_checks(mlp, params_r, x, lab, 1024.0)
    emu = bf16_pipeline_grads(params_r, x, lab, col_frac=col_frac)
    inh_n, inh_m, inh_e = [], [], []
    for i, (e, c) in enumerate(zip(emu, gc)):
        if isinstance(e, tuple):
            e, cols = e
            c = c[:, cols]
        c = c.astype(np.float64)
        inh_n.append(float(np.linalg.norm(e - c) / np.linalg.norm(c)))
        inh_m.append(float(np.abs(e - c).max() / np.abs(c).max()))
        inh_e.append(O.erro_rel(c, e))
    print("inherent bf16 distance from f32 (float64 restatement): norm-wise", ["%.1e" % v for v in inh_n],
          "\n  max-relative", ["%.1e" % v for v in inh_m], "\n  erro_rel", ["%.1e" % v for v in inh_e], flush=True)
    grad_gate("bf16 grads vs the f32 oracle", gc, gg, [max(2e-2, 2 * v) for v in inh_n],
              [max(2e-2, 2 * v) for v in inh_m], erro_bound=[max(2e-2, 2 * v) for v in inh_e])
    if emu_bound is not None:
        ne = [float(np.linalg.norm(a - b) / max(np.linalg.norm(a), 1e-30)) for a, b in zip(emu, gg)]
        print("  norm-wise vs the bf16 restatement", ["%.1e" % r for r in ne], flush=True)
        assert max(ne) < emu_bound


def _mixed_step_check(gpu, dims, B, steps, lr, seed, emu_bound=1e-2, col_frac=None):
    params = kaiming_model(seed, dims)
    # the CPU reference runs in f32 from the bf16-rounded initial weights and inputs
    params_r = [bf16_round(p) if i % 2 == 0 else p for i, p in enumerate(params)]
    cpu = O.CpuMlp(params_r[0::2], params_r[1::2])
    cpu.set_optimizer("adam", lr)
    mlp = G.GpuMlp.from_params(gpu, params_r, B, lr, precision="bf16", loss_scale=1024.0)
    losses = []
    for s in range(steps):
        x = bf16_round(normal_batch(5000 + s, B, dims[0]))
        lab = uniform_labels(6000 + s, B, dims[-1])
        mlp.step(gpu.upload(x, G.BF16), G.upload_labels(gpu, lab))
        lc = cpu.step(x, lab)
        lg = mlp.last_loss()
        if s == 0:
            bf16_gates(mlp, cpu, params_r, x, lab, col_frac=col_frac, emu_bound=emu_bound)
            assert not mlp.overflow()
        losses.append((lc, lg))
    return losses, cpu, mlp


def test_mixed_precision_mlp_trajectory_small(gpu):
    # The 8-hidden-layer ReLU structure at width 256 (batch 512, 32 classes):
    # 100 steps of bf16 training against the f32 oracle.
    dims = [256] * 9 + [32]
    losses, cpu, mlp = _mixed_step_check(gpu, dims, 512, 100, 1e-3, 5)
    d = [abs(a - b) / max(abs(a), 1e-6) for a, b in losses]
    print("loss cpu/gpu first", losses[0], "last", losses[-1], "max rel diff %.2e" % max(d))
    assert max(d) < 2e-2
    assert losses[-1][1] < losses[0][1]
    ew = [O.erro_rel(a, b) for a, b in zip(cpu.weights(), mlp.weights())]
    moved = [float(np.linalg.norm(b - a) / max(np.linalg.norm(a - p0.reshape(a.shape)), 1e-30))
             for a, b, p0 in zip(cpu.weights(), mlp.weights(), kaiming_model(5, dims))]
    print("final weights erro_rel vs f32", ["%.1e" % e for e in ew],
          "\n  |W_gpu - W_cpu| / |W_cpu - W_0|", ["%.2f" % m for m in moved])
    # Adam's per-element normalisation turns bf16 noise on near-zero gradients
    # into +-lr steps; 100 steps drift a few 1e-2 (the loss, above, is the
    # tracked quantity).  A wrong update rule would be far outside this.
    assert max(ew) < 0.1


def test_mixed_precision_mlp_full_size_step(gpu):
    # 8 x 4096 ReLU layers -> 1000 classes, batch 4096: the first step at full
    # size against the f32 oracle (~10 s on 16 threads), with the layer-local
    # checks and the float64 bf16 restatement on 1/8 of each dW's columns.
    dims = [4096] * 9 + [1000]
    t0 = time.time()
    losses, cpu, mlp = _mixed_step_check(gpu, dims, 4096, 1, 1e-3, 6, emu_bound=None, col_frac=0.125)
    d = [abs(a - b) / abs(a) for a, b in losses]
    print("full size loss", losses, "rel diff", ["%.1e" % x for x in d], f"{time.time() - t0:.0f}s")
    assert max(d) < 2e-2


SPIKE = (1, 2, 3)  # the loss spike of the 8 x 4096 -> 1000 trajectory (7.96 -> 26.0 -> 13.8 -> 7.3)


def _c5_fixture():
    import json
    import os
    from tests.golden import make_c5_trajectory as mk

    with open(os.path.join(os.path.dirname(mk.__file__), "c5_trajectory.json")) as f:
        fix = json.load(f)
    want_bits = [int(b) for b in fix["loss_bits"]]
    rest = [fix["bf16_restatement_f32_acc"], fix["bf16_restatement_f64_acc"]]
    assert len(want_bits) == mk.STEPS and all(len(r) == mk.STEPS for r in rest)
    return mk, want_bits, rest


def _f32(bits):
    return float(np.uint32(bits).view(np.float32))


def _spike_loss_gate(tag, s, plan, oracle, restated):
    """The loss of one spike step from a shared state.  The float64
    restatement of the bf16 pipeline from that state measures how far bf16
    storage alone moves the loss from f32 (in the spike the logits are large:
    2.6% at step 2).  The plan must be within 2e-2 of that restatement, and
    within max(2e-2, 2 x the restatement's own distance) of the f32 oracle."""
    d_re = abs(plan - restated) / abs(restated)
    inh = abs(restated - oracle) / abs(oracle)
    d_or = abs(plan - oracle) / abs(oracle)
    print(f"{tag} step {s}: oracle {oracle:.5f}, bf16 plan {plan:.5f}, float64 bf16 restatement {restated:.5f}; "
          f"plan vs restatement {d_re:.2e}, plan vs oracle {d_or:.2e} (restatement vs oracle {inh:.2e})",
          flush=True)
    assert d_re <= 2e-2, (tag, s, plan, restated)
    assert d_or <= max(2e-2, 2 * inh), (tag, s, plan, oracle, inh)
    return d_re, d_or, inh


def test_mixed_precision_mlp_full_size_teacher_forced_spike(gpu):
    """Steps 1-3 of the 8 x 4096 -> 1000 trajectory at batch 4096 (the loss
    spike), each started from the oracle's own state: before step s the
    oracle's f32 weights and Adam m, v, t after s updates are loaded into the
    bf16 plan (rt_mlp_set_weights, rt_mlp_set_optimizer_state), and the plan's
    step s on the same batch is checked against the oracle's step s:
    * the loss within 2e-2 of the float64 restatement of the bf16 pipeline
      from the same state, and within max(2e-2, 2 x that restatement's
      distance) of the oracle's (_spike_loss_gate);
    * every GEMM and rounding point of the step layer-locally against float64
      on the plan's own stored inputs;
    * the gradients against the oracle's, whole and scale-aware, within
      max(2e-2, 2 x the distance bf16 storage alone causes, from the float64
      restatement of the bf16 pipeline from the same state);
    * the update used the loaded state: m' = β1·m + (1 − β1)·g and
      v' = β2·v + (1 − β2)·g² in f32 on the plan's own g, to the bit, and t.
    With the state shared, the ~100x amplification of earlier differences that
    a free-running comparison meets in these steps (tests/gpu.rs:99-139
    compares free-running trajectories) is taken out.  The oracle's losses
    reproduce the committed fixture's bits."""
    mk, want_bits, _ = _c5_fixture()
    params = mk.initial_params()
    cpu = O.CpuMlp(params[0::2], params[1::2])
    cpu.set_optimizer("adam", mk.LR)
    mlp = G.GpuMlp.from_params(gpu, params, mk.BATCH, mk.LR, precision="bf16", loss_scale=1024.0)
    b1, b2 = np.float32(0.9), np.float32(0.999)
    t0 = time.time()
    x, lab = mk.batch(0)
    lc = cpu.step(x, lab)
    assert int(np.float32(lc).view(np.uint32)) == want_bits[0]
    for s in SPIKE:
        x, lab = mk.batch(s)
        w_s = cpu.weights()
        m_s, v_s, t_s = cpu.optimizer_state()
        assert t_s == s
        mlp.set_weights(w_s)
        mlp.set_optimizer_state(m_s, v_s, t_s)
        mlp.step(gpu.upload(x, G.BF16), G.upload_labels(gpu, lab))
        lg = mlp.last_loss()
        lc = cpu.step(x, lab)
        assert int(np.float32(lc).view(np.uint32)) == want_bits[s], (s, lc, _f32(want_bits[s]))
        _spike_loss_gate("teacher-forced", s, lg, lc, bf16_pipeline_loss(w_s, x, lab))
        assert not mlp.overflow()
        bf16_gates(mlp, cpu, w_s, x, lab)
        g = mlp.grads()
        m1, v1, t1 = mlp.optimizer_state()
        assert t1 == s + 1
        for i in range(len(g)):
            gi = g[i].astype(np.float32)
            want_m = (b1 * m_s[i] + (np.float32(1) - b1) * gi).astype(np.float32)
            want_v = (b2 * v_s[i] + (np.float32(1) - b2) * (gi * gi)).astype(np.float32)
            assert np.array_equal(m1[i], want_m), (s, i)
            assert np.array_equal(v1[i], want_v), (s, i)
        print(f"  step {s}: gates passed ({time.time() - t0:.0f} s)", flush=True)


def test_mixed_precision_mlp_full_size_100_step_trajectory(gpu):
    """tests/golden/c5_trajectory.json holds the oracle's f32 losses of 100
    Adam steps of the 8 x 4096 -> 1000 MLP at batch 4096 from bf16-rounded
    weights and inputs (written by make_c5_trajectory.py beside it).  The
    bf16 plan (f32 master weights, loss scale 1024) runs the same 100 steps
    free, as tests/gpu.rs:99-139 runs its trajectories, and every loss must
    stay within 2e-2 of the oracle's, except in the loss spike (steps 1-3).

    There the spike amplifies earlier differences ~100x: two independent
    numpy restatements of the bf16 plan (in the fixture) land up to 7.9% from
    the oracle at step 2, and the plan 11.7%.  Each spike step is checked
    from a shared state instead, from both sides:
    * from the oracle's state: test_..._teacher_forced_spike above;
    * from the plan's own state: before step s the plan's weights and Adam
      m, v, t are loaded into a second oracle, and the plan's step-s loss
      passes _spike_loss_gate against that oracle's loss and the float64
      bf16 restatement's from the same weights.
    So each spike loss is the right function of its state, and the
    free-running gap there is the difference of states, not of arithmetic."""
    import concurrent.futures as cf

    mk, want_bits, rest = _c5_fixture()
    want = [_f32(b) for b in want_bits]
    params = mk.initial_params()
    mlp = G.GpuMlp.from_params(gpu, params, mk.BATCH, mk.LR, precision="bf16", loss_scale=1024.0)
    rev = O.CpuMlp(params[0::2], params[1::2])  # the oracle run from the plan's state
    rev.set_optimizer("adam", mk.LR)
    t0 = time.time()
    got, rev_d = [], {}
    with cf.ThreadPoolExecutor(8) as ex:  # the Rng fills run in C, outside the GIL
        futs = [ex.submit(mk.batch, s) for s in range(mk.STEPS)]
        for s, fu in enumerate(futs):
            x, lab = fu.result()
            if s in SPIKE:
                m, v, t = mlp.optimizer_state()
                assert t == s
                w_s = mlp.weights()
                rev.set_weights(w_s)
                rev.set_optimizer_state(m, v, t)
                lr_ = rev.step(x, lab)
            mlp.step(gpu.upload(x, G.BF16), G.upload_labels(gpu, lab))
            got.append(mlp.last_loss())
            futs[s] = None
            if s in SPIKE:
                print(f"step {s}: oracle {want[s]:.5f} bf16 {got[-1]:.5f} (restatements {rest[0][s]:.5f}, "
                      f"{rest[1][s]:.5f}) ({time.time() - t0:.0f} s)", flush=True)
                rev_d[s] = _spike_loss_gate("from the plan's state", s, got[-1], lr_,
                                            bf16_pipeline_loss(w_s, x, lab))
            elif s < 6 or s % 10 == 0:
                print(f"step {s}: oracle {want[s]:.5f} bf16 {got[-1]:.5f} ({time.time() - t0:.0f} s)", flush=True)
    d = [abs(g - w) / abs(w) for g, w in zip(got, want)]
    off = [d[s] for s in range(mk.STEPS) if s not in SPIKE]
    print(f"100-step trajectory: outside the spike max rel diff {max(off):.2e}; spike free-running "
          f"{[round(d[s], 4) for s in SPIKE]}, from the plan's own state (vs restatement, vs oracle) "
          f"{[(f'{rev_d[s][0]:.1e}', f'{rev_d[s][1]:.1e}') for s in SPIKE]}; "
          f"final {want[-1]:.5f} vs {got[-1]:.5f}", flush=True)
    for s in range(mk.STEPS):
        if s not in SPIKE:
            assert d[s] <= 2e-2, (s, got[s], want[s])
    assert max(d[10:]) <= 1e-3  # past the spike every implementation sits near ln(1000)
    assert not mlp.overflow()


@pytest.mark.parametrize("dims,batch", [
    ([64, 64, 10], 32),      # register-staged GEMMs: the separate non-finite check
    ([128, 256, 128], 128),  # direct-to-LDS dW GEMMs: the flag comes from their epilogues alone
    ([128, 256, 100], 128),  # both: the 100-wide head is checked separately
])
def test_mixed_precision_overflow_skips_update(gpu, dims, batch):
    # A huge input makes the scaled gradient overflow: the step is skipped
    # (weights unchanged) and reported, and training continues afterwards.
    params = kaiming_model(8, dims)
    mlp = G.GpuMlp.from_params(gpu, params, batch, 1e-3, precision="bf16", loss_scale=1024.0)
    w0 = mlp.weights()
    x = np.full((batch, dims[0]), 3.0e38, np.float32)
    mlp.step(gpu.upload(x, G.BF16), G.upload_labels(gpu, np.zeros(batch, np.uint32)))
    assert mlp.overflow()
    for a, b in zip(w0, mlp.weights()):
        assert np.array_equal(a, b)
    x = normal_batch(1, batch, dims[0])
    mlp.step(gpu.upload(x, G.BF16), G.upload_labels(gpu, uniform_labels(2, batch, dims[-1])))
    assert not mlp.overflow()
    assert any(not np.array_equal(a, b) for a, b in zip(w0, mlp.weights()))


@pytest.mark.parametrize("dims,batch", [([256, 512, 512, 256, 64], 256), ([1024, 4096, 4096, 64], 4096),
                                        ([256, 96, 160, 64], 200)])
def test_mixed_plan_dx_equals_the_activation_masked_gemm(gpu, dims, batch):
    # The bf16 plan's dX GEMMs take the ReLU predicate as one bit per element,
    # written by the forward GEMM (64x64 tiles at the first shape, 256x256 at
    # the second); at the third (widths not a multiple of 64, ragged rows)
    # they read the activation itself.  Each δ_{l-1} must be, bit for bit, the
    # standalone NT GEMM masked by the stored bf16 activation A_{l-1}, on the
    # plan's own δ_l and the bf16 weights the step started from.
    params = kaiming_model(31, dims)
    x = normal_batch(32, batch, dims[0])
    lab = uniform_labels(33, batch, dims[-1])
    mlp = G.GpuMlp.from_params(gpu, params, batch, 1e-3, precision="bf16", loss_scale=1024.0)
    mlp.step(gpu.upload(x, G.BF16), G.upload_labels(gpu, lab))
    assert not mlp.overflow()
    zeros = 0
    for l in range(len(dims) - 2, 0, -1):
        act = mlp.activation(l - 1)
        zeros += int((act == 0).sum())
        d = gpu.upload(mlp.delta(l), G.BF16)
        w = gpu.upload(params[2 * l], G.BF16)
        out = gpu.zeros((batch, dims[l]), G.BF16)
        gpu.gemm(G.NT, d, w, out, G.EPI_RELU_MASK, gpu.upload(act, G.BF16))
        want = G.f32_to_bf16_bits(gpu.download_f32(out))
        got = G.f32_to_bf16_bits(mlp.delta(l - 1))
        assert np.array_equal(got, want), (l, int((got != want).sum()))
    assert zeros > 0  # the masks are not all ones


def test_linear4096_backward_bf16_full_size(gpu):
    """Linear 4096->4096 backward at batch 8192 (nn.rs:82-98 adjoints): X, dY
    ~N(0,1)/64 and Kaiming-uniform W in bf16; dX = dY·Wᵀ (bf16 out), dW = Xᵀ·dY
    (f32 out) with db = colsum(dY) fused.  Every output entry is checked
    against float64 GEMMs of the same bf16-rounded operands, with a bound per
    entry from |A|·|B|:
    * the products of two bf16 values are exact in f32, so the only error of
      an f32-accumulated entry is summation rounding; it is far below
      1e-5·Σ|a_k b_k| (its spread is ~4e-8 of that for these sums), while one
      dropped or doubled term moves the entry by ~1/K of Σ|a_k b_k|
      (1.2e-4 to 2.4e-4) and a wrong or zeroed tile by ~1/√K (1.1e-2 to
      1.6e-2);
    * dX is then rounded once to bf16 (round to nearest even): at most
      2⁻⁸·|dX| more.
    Then the whole outputs against the f32 inputs before rounding, within
    2e-2 (norm-wise and max-relative)."""
    B, D = 8192, 4096
    rng = np.random.default_rng(33)
    x32 = rng.standard_normal((B, D), dtype=np.float32) / np.float32(64)
    dy32 = rng.standard_normal((B, D), dtype=np.float32) / np.float32(64)
    lim = np.sqrt(6.0 / D)
    w32 = rng.uniform(-lim, lim, size=(D, D)).astype(np.float32)
    gx, gdy, gw = gpu.upload(x32, G.BF16), gpu.upload(dy32, G.BF16), gpu.upload(w32, G.BF16)
    dx, dw, db = gpu.zeros((B, D), G.BF16), gpu.zeros((D, D)), gpu.zeros((1, D))
    print(f"NT {B}x{D}x{D} then TN {D}x{D}x{B} with db", flush=True)
    gpu.gemm(G.NT, gdy, gw, dx)
    gpu.gemm(G.TN, gx, gdy, dw, colsum=db)
    got_dx, got_dw, got_db = gpu.download_f32(dx), gpu.download(dw), gpu.download(db)
    del gx, gdy, gw, dx, dw, db
    t0 = time.time()
    x, dy, w = (bf16_round(a).astype(np.float64) for a in (x32, dy32, w32))
    # db whole, against the exact column sums of the rounded dY
    ex_b = dy.sum(0, keepdims=True)
    assert np.all(np.abs(got_db - ex_b) <= 1e-5 * np.abs(dy).sum(0, keepdims=True))
    # dW whole: K = 8192
    ex = x.T @ dy
    ab = np.abs(x).T @ np.abs(dy)
    r_dw = np.abs(got_dw - ex) / ab
    print(f"dW [{D},{D}] whole: max |err|/Σ|ab| {r_dw.max():.2e}, mean {r_dw.mean():.2e} "
          f"({time.time() - t0:.0f} s)", flush=True)
    assert np.all(np.abs(got_dw - ex) <= 1e-5 * ab)
    del ex, ab, r_dw
    # dX whole: K = 4096, then one bf16 rounding
    ex = dy @ w.T
    ab = np.abs(dy) @ np.abs(w).T
    r_dx = np.abs(got_dx - ex) / (2.0 ** -8 * np.abs(ex) + 1e-5 * ab)
    print(f"dX [{B},{D}] whole: max |err|/bound {r_dx.max():.3f} ({time.time() - t0:.0f} s)", flush=True)
    assert np.all(np.abs(got_dx - ex) <= 2.0 ** -8 * np.abs(ex) + 1e-5 * ab)
    del ex, ab, r_dx, x, dy, w
    # Against the f32 inputs before rounding, whole, scale-aware (a zeroed or
    # wrong result scores ~1 on both measures).
    x, dy, w = (a.astype(np.float64) for a in (x32, dy32, w32))
    f_dx, f_dw, f_db = dy @ w.T, x.T @ dy, dy.sum(0, keepdims=True)
    rows = grad_gate("c3 vs the f32 inputs (dX, dW, db whole)", [f_dx, f_dw, f_db],
                     [got_dx, got_dw, got_db], 2e-2, 2e-2)
    print(f"vs f32 inputs: dX {rows[0][1]:.2e}, dW {rows[1][1]:.2e} max-relative ({time.time() - t0:.0f} s)",
          flush=True)
