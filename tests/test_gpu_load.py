"""Overlapped batch loading (rt_mlp_load / rt_mlp_step_loaded), the
asynchronous form of GpuMlp::carregar (mod.rs:1486-1495).

A loaded batch goes through pinned staging and a copy stream into one of
two device slots; a step on the loaded batch must take exactly the step the
same batch takes when uploaded and passed directly, for f32 and bf16 plans,
with the copy of batch i+1 issued while step i is still queued.
"""
import numpy as np
import pytest

from rgpu_amd import gpu as G
from tests.gpu_common import kaiming_model, normal_batch, uniform_labels

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gpu():
    g = G.Gpu(0)
    yield g
    g.close()


def bits_equal(a, b):
    return all(np.array_equal(np.asarray(x, np.float32).view(np.uint32), np.asarray(y, np.float32).view(np.uint32))
               for x, y in zip(a, b))


@pytest.mark.parametrize("precision", ["f32", "bf16"])
def test_loaded_steps_match_direct_steps(gpu, precision):
    dims, batch, steps = [64, 128, 96, 10], 256, 6
    params = kaiming_model(5, dims)
    kw = dict(precision=precision, loss_scale=256.0 if precision == "bf16" else 1.0)
    a = G.GpuMlp.from_params(gpu, params, batch, 1e-3, **kw)
    b = G.GpuMlp.from_params(gpu, params, batch, 1e-3, **kw)
    xs = [normal_batch(100 + i, batch, dims[0]) for i in range(steps)]
    ys = [uniform_labels(200 + i, batch, dims[-1]) for i in range(steps)]
    dt = G.BF16 if precision == "bf16" else G.F32
    la, lb = [], []
    a.carregar(xs[0], ys[0])
    for i in range(steps):
        a.step_loaded()
        if i + 1 < steps:
            a.carregar(xs[i + 1], ys[i + 1])  # copy overlaps step i
        la.append(a.last_loss() if i == steps - 1 else None)
        b.step(gpu.upload(xs[i], dt), G.upload_labels(gpu, ys[i]))
        lb.append(b.last_loss() if i == steps - 1 else None)
    assert la[-1] == lb[-1]
    assert bits_equal(a.weights(), b.weights())
    a.destroy()
    b.destroy()


def test_step_uses_the_latest_load(gpu):
    dims, batch = [32, 64, 10], 128
    params = kaiming_model(9, dims)
    a = G.GpuMlp.from_params(gpu, params, batch, 1e-3)
    b = G.GpuMlp.from_params(gpu, params, batch, 1e-3)
    x0, x1 = normal_batch(1, batch, dims[0]), normal_batch(2, batch, dims[0])
    y0, y1 = uniform_labels(3, batch, 10), uniform_labels(4, batch, 10)
    a.carregar(x0, y0)
    a.carregar(x1, y1)
    a.step_loaded()
    a.step_loaded()  # the same batch again
    b.step(gpu.upload(x1), G.upload_labels(gpu, y1))
    b.step(gpu.upload(x1), G.upload_labels(gpu, y1))
    assert bits_equal(a.weights(), b.weights())
    # many loads in a row reuse the pinned staging safely
    for i in range(5):
        a.carregar(normal_batch(10 + i, batch, dims[0]), uniform_labels(20 + i, batch, 10))
    a.step_loaded()
    b.step(gpu.upload(normal_batch(14, batch, dims[0])), G.upload_labels(gpu, uniform_labels(24, batch, 10)))
    assert bits_equal(a.weights(), b.weights())
    a.destroy()
    b.destroy()


def test_load_errors(gpu):
    dims, batch = [16, 32, 10], 64
    m = G.GpuMlp.from_params(gpu, kaiming_model(1, dims), batch, 1e-3)
    with pytest.raises(G.RtError) as e:
        m.step_loaded()
    assert e.value.status == "RT_ERR_INVALID"
    with pytest.raises(G.RtError) as e:
        m.carregar(np.zeros((batch + 1, dims[0]), np.float32), np.zeros(batch + 1))
    assert e.value.status == "RT_ERR_SHAPE"
    with pytest.raises(G.RtError) as e:
        m.carregar(np.zeros((batch, dims[0]), np.float32), np.zeros(batch - 1))
    assert e.value.status == "RT_ERR_SHAPE"
    m.destroy()
