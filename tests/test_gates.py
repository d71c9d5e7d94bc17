"""The scale-aware parity gate of the GPU tests (tests/gpu_common.grad_gate),
checked on the CPU with the oracle's own gradients: a mistake planted in a
copy of them (a zeroed tensor, a doubled one, a sign flip) must fail the gate,
where the reference's erro_rel alone (gpu.rs:53-60, an absolute error for
values far below 1) lets a zeroed small-magnitude tensor through."""
import numpy as np
import pytest

from oracle import oracle as O
from tests.gpu_common import grad_gate, kaiming_model, normal_batch, uniform_labels


@pytest.fixture(scope="module")
def grads():
    # MLP 512-1024-1024-10, batch 32: one step's gradients
    params = kaiming_model(1, [512, 1024, 1024, 10])
    cpu = O.CpuMlp(params[0::2], params[1::2])
    cpu.set_optimizer("none", 0.0)
    cpu.step(normal_batch(101, 32, 512), uniform_labels(102, 32, 10))
    return cpu.grads()


def test_gate_passes_rounding_noise(grads):
    rng = np.random.default_rng(0)
    got = [(g * (1 + 1e-6 * rng.standard_normal(g.shape))).astype(np.float32) for g in grads]
    grad_gate("noise", grads, got, 1e-4, 1e-4, erro_bound=1e-4)


@pytest.mark.parametrize("i", range(6))
@pytest.mark.parametrize("mistake", ["zero", "double", "negate"])
def test_gate_fails_a_planted_mistake(grads, i, mistake):
    got = [g.copy() for g in grads]
    got[i] = {"zero": 0 * got[i], "double": 2 * got[i], "negate": -got[i]}[mistake]
    with pytest.raises(AssertionError):
        grad_gate("planted", grads, got, 1e-4, 1e-4)
    # the bf16 bounds (at most twice the ~12% inherent distance) fail it too
    with pytest.raises(AssertionError):
        grad_gate("planted", grads, got, 0.25, 0.25)


@pytest.fixture(scope="module")
def batch2048():
    from tests.gpu_common import numpy_f32_grads

    params = kaiming_model(2, [512, 1024, 1024, 10])
    x, lab = normal_batch(10_000, 2048, 512), uniform_labels(20_000, 2048, 10)
    cpu = O.CpuMlp(params[0::2], params[1::2])
    cpu.set_optimizer("none", 0.0)
    cpu.step(x, lab)
    return cpu.grads(), numpy_f32_grads(params, x, lab)


@pytest.mark.parametrize("i", range(6))
def test_conditioned_gate_fails_a_zeroed_tensor_at_batch_2048(batch2048, i):
    # bounds widened to 3x an independent f32 implementation's distance
    # (at most ~5e-3 here) still fail a zeroed tensor
    g, ref = batch2048
    grad_gate("itself", g, [a.copy() for a in g], 1e-4, 1e-4, ref=ref)
    got = [a.copy() for a in g]
    got[i] = 0 * got[i]
    with pytest.raises(AssertionError):
        grad_gate("planted", g, got, 1e-4, 1e-4, ref=ref)


def test_erro_rel_alone_misses_a_zeroed_small_tensor():
    # At batch 2048 the hidden-layer gradients are far below 1: erro_rel of a
    # zeroed copy is about max|g|, under the bf16 bar of 2e-2, while the
    # scale-aware gate scores it 1.
    params = kaiming_model(2, [512, 1024, 1024, 10])
    cpu = O.CpuMlp(params[0::2], params[1::2])
    cpu.set_optimizer("none", 0.0)
    cpu.step(normal_batch(10_000, 2048, 512), uniform_labels(20_000, 2048, 10))
    g = cpu.grads()
    small = min(range(len(g)), key=lambda k: np.abs(g[k]).max())
    assert O.erro_rel(g[small], 0 * g[small]) < 2e-2
    with pytest.raises(AssertionError):
        grad_gate("zeroed", [g[small]], [0 * g[small]], 0.25, 0.25)
