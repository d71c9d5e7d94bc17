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
    a.save(path)
    st = a.state_dict()
    assert st["t"] == 4
    b = G.GpuMlp.from_params(gpu, kaiming_model(2, dims), B, lr, **kw)  # different start, then loaded
    b.load(path)
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
