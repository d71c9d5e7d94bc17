"""Device argmax / accuracy and checkpoint-resume of the training plan.

argmax and accuracy are integer / count results: bit-exact against the oracle
(tensor.rs:476-493, losses.rs:181-185), including ties and NaN columns.
Resume: a model that saves its state mid-run and a fresh model that loads it
must take bit-identical steps afterwards (same kernels, same state), for the
f32 plan and for the bf16 mixed-precision plan with its device-side Adam t.
"""
import numpy as np
import pytest

from oracle import oracle as O
from rgpu_amd import gpu as G
from tests.gpu_common import kaiming_model, normal_batch, uniform_labels

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gpu():
    g = G.Gpu(0)
    yield g
    g.close()


def logits_with_ties_and_nans(rows, cols, seed):
    rng = np.random.default_rng(seed)
    z = rng.integers(-3, 4, size=(rows, cols)).astype(np.float32)  # many ties
    z[rng.random(size=z.shape) < 0.02] = np.nan
    z[rng.random(size=z.shape) < 0.02] = -np.inf
    z[::17, 0] = np.nan
    return z


@pytest.mark.parametrize("rows,cols", [(1, 1), (7, 3), (2048, 10), (333, 1000), (64, 65)])
def test_argmax_matches_oracle_exactly(gpu, rows, cols):
    z = logits_with_ties_and_nans(rows, cols, rows + cols)
    out = gpu.zeros((rows,), G.U32)
    gpu.argmax_rows(gpu.upload(z), out)
    assert np.array_equal(gpu.download(out), O.argmax_rows(z))


def test_argmax_fixed_cases(gpu):
    nan, inf = np.nan, np.inf
    z = np.array([[nan, 1, 2], [1, nan, 3], [1, nan, 0], [-inf, -inf, -inf], [-0.0, 0.0, -inf],
                  [-inf, nan, -1], [inf, inf, 1]], np.float32)
    out = gpu.zeros((z.shape[0],), G.U32)
    gpu.argmax_rows(gpu.upload(z), out)
    assert gpu.download(out).tolist() == [0, 2, 0, 0, 0, 2, 0]


@pytest.mark.parametrize("rows,cols", [(2048, 10), (1000, 7)])
def test_accuracy_matches_oracle_exactly(gpu, rows, cols):
    z = logits_with_ties_and_nans(rows, cols, 5)
    lab = uniform_labels(6, rows, cols)
    got = gpu.accuracy(gpu.upload(z), G.upload_labels(gpu, lab))
    assert got == O.accuracy(z, lab)


def test_accuracy_shape_errors(gpu):
    z = gpu.upload(np.zeros((4, 3), np.float32))
    with pytest.raises(G.RtError):
        gpu.accuracy(z, G.upload_labels(gpu, np.zeros(5, np.uint32)))


@pytest.mark.parametrize("precision,optimizer", [("f32", "adam"), ("f32", "sgd"), ("bf16", "adam")])
def test_checkpoint_resume_is_bit_exact(gpu, tmp_path, precision, optimizer):
    dims, B = [64, 128, 96, 10], 256
    dt = G.BF16 if precision == "bf16" else G.F32
    lr = 1e-3 if optimizer == "adam" else 0.05
    kw = dict(optimizer=optimizer, precision=precision)
    if optimizer == "sgd":
        kw["momentum"] = 0.9
    if precision == "bf16":
        kw["loss_scale"] = 1024.0
    batches = [(gpu.upload(normal_batch(10 + i, B, dims[0]), dt), G.upload_labels(gpu, uniform_labels(20 + i, B, 10)))
               for i in range(8)]
    a = G.GpuMlp.from_params(gpu, kaiming_model(1, dims), B, lr, **kw)
    for x, y in batches[:4]:
        a.step(x, y)
    path = str(tmp_path / "ckpt.npz")
    a.save_checkpoint(path)
    st = a.state_dict()
    assert st["t"] == 4
    b = G.GpuMlp.from_params(gpu, kaiming_model(2, dims), B, lr, **kw)  # different start, then loaded
    b.load_checkpoint(path)
    for wa, wb in zip(a.weights(), b.weights()):
        assert np.array_equal(wa, wb)
    for x, y in batches[4:]:
        a.step(x, y)
        b.step(x, y)
        assert a.last_loss() == b.last_loss()
    for wa, wb in zip(a.weights(), b.weights()):
        assert np.array_equal(wa, wb)
    ma, va, ta = a.optimizer_state()
    mb, vb, tb = b.optimizer_state()
    assert ta == tb == 8
    for x1, x2 in zip(ma + va, mb + vb):
        assert np.array_equal(x1, x2)


def test_set_weights_round_trip_and_shape_check(gpu):
    dims, B = [32, 48, 10], 64
    m = G.GpuMlp.from_params(gpu, kaiming_model(3, dims), B, 1e-3)
    new = kaiming_model(4, dims)
    m.set_weights(new)
    for want, got in zip(new, m.weights()):
        assert np.array_equal(want.reshape(got.shape), got)
    with pytest.raises(ValueError):
        m.set_weights(new[:-1])


@pytest.mark.parametrize("optimizer", ["adam", "sgd"])
def test_optimizer_state_matches_oracle_and_resumes_from_it(gpu, optimizer):
    """The optimizer state GpuMlp keeps private (mod.rs:1291-1314, 1334)
    against the oracle's Optimizer (optim.rs:80-114, 162-198) on MLP
    512-1024-1024-10 at batch 2048: after 3 steps the exported m and v match
    within the f32 bar (erro_rel 1e-4; norm-wise and max-relative 1e-4 or
    three times a float32 numpy run's distance) and Adam's t exactly; then the ORACLE's weights, m, v and t loaded into a fresh plan
    follow the oracle's own continuation for 20 steps (loss within 2e-3, the
    gpu.rs:99-139 trajectory bar) and end with the same t."""
    from tests.gpu_common import grad_gate, numpy_f32_trajectory, oracle_threads

    O.set_threads(oracle_threads())
    dims, B = [512, 1024, 1024, 10], 2048
    lr = 1e-3 if optimizer == "adam" else 0.01
    kw = dict(optimizer=optimizer)
    if optimizer == "sgd":
        kw["momentum"] = 0.9
    params = kaiming_model(2, dims)
    batches = [(normal_batch(300 + s, B, dims[0]), uniform_labels(400 + s, B, 10)) for s in range(23)]
    cpu = O.CpuMlp(params[0::2], params[1::2])
    cpu.set_optimizer(optimizer, lr, 0.9 if optimizer == "sgd" else 0.0)
    mlp = G.GpuMlp.from_params(gpu, params, B, lr, **kw)
    for x, y in batches[:3]:
        cpu.step(x, y)
        mlp.step(gpu.upload(x), G.upload_labels(gpu, y))
    gm, gv, gt = mlp.optimizer_state()
    cm, cv, ct = cpu.optimizer_state()
    assert gt == 3
    if optimizer == "adam":
        assert ct == 3
    # At batch 2048 a few ReLU pre-activations lie within rounding of zero,
    # so the bounds are conditioned on a float32 numpy run of the same 3
    # steps (another summation order), as the step-1 gradient gate is.
    _, _, nm, nv = numpy_f32_trajectory(params, batches[:3], lr, optimizer=optimizer,
                                        momentum=0.9 if optimizer == "sgd" else 0.0, return_state=True)
    grad_gate("m", cm, gm, 1e-4, 1e-4, erro_bound=1e-4, ref=nm)
    if optimizer == "adam":
        grad_gate("v", cv, gv, 1e-4, 1e-4, erro_bound=1e-4, ref=nv)
    # resume from the oracle's state
    fresh = G.GpuMlp.from_params(gpu, kaiming_model(9, dims), B, lr, **kw)
    fresh.set_weights(cpu.weights())
    fresh.set_optimizer_state(cm, cv if optimizer == "adam" else [np.zeros_like(a) for a in cm], 3)
    worst = 0.0
    for x, y in batches[3:]:
        lc = cpu.step(x, y)
        fresh.step(gpu.upload(x), G.upload_labels(gpu, y))
        lg = fresh.last_loss()
        worst = max(worst, abs(lc - lg))
    print(f"{optimizer}: resumed from the oracle's state, max |loss diff| over 20 steps {worst:.2e}")
    assert worst < 2e-3
    assert fresh.optimizer_state()[2] == 23
    if optimizer == "adam":
        assert cpu.optimizer_state()[2] == 23
    O.set_threads(1)


def test_model_after_its_context_is_closed():
    """rt_close releases the models made on the context; the Python model
    then refuses calls instead of passing a dangling handle, and destroying
    it (explicitly or when collected) calls nothing on the released plan."""
    x = np.sin(np.arange(64 * 8, dtype=np.float32) * np.float32(0.37)).reshape(64, 8)
    lab = (np.arange(64) % 4).astype(np.uint32)
    g = G.Gpu(0)
    mlp = G.GpuMlp.from_params(g, kaiming_model(5, [8, 16, 4]), 64, 0.01)
    mlp.step(g.upload(x), G.upload_labels(g, lab))
    assert np.isfinite(mlp.last_loss())
    g.close()
    with pytest.raises(G.RtError):
        mlp.last_loss()
    with pytest.raises(G.RtError):
        mlp.weights()
    mlp.destroy()
    mlp.destroy()
    del mlp
    g2 = G.Gpu(0)  # the device is usable afterwards
    m2 = G.GpuMlp.from_params(g2, kaiming_model(5, [8, 16, 4]), 64, 0.01)
    m2.step(g2.upload(x), G.upload_labels(g2, lab))
    assert np.isfinite(m2.last_loss())
    g2.close()
    del m2
