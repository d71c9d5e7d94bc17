"""The op-level device backend (tensor ops + the device tape) against the
oracle's tape, and the reference's own autodiff tests (tests/autodiff.rs)
run on the device.

Bars:
* arithmetic that involves no transcendental and no reordered sum is
  bit-exact: +, −, ×, ÷ with broadcasting, scale/offset/neg/square/sqrt/relu/
  leaky_relu and every VJP built from them, and reduce_to onto any target
  with more than one element (each output sums its sources in increasing
  index order, as the reference does);
* exp / ln / sigmoid / tanh and softmax use the device's libm: within 4 ulp
  of the oracle's glibc values, their VJPs within erro_rel 1e-6;
* sum_all, the losses and matmul add in a different order: erro_rel <= 1e-5
  per op, gradients of whole models <= 1e-4 (the f32 parity bar), loss
  trajectories over 100 steps <= 1e-4.
"""
import numpy as np
import pytest

from oracle import oracle as O
from rgpu_amd import autograd as A
from rgpu_amd import gpu as G

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gpu():
    g = G.Gpu(0)
    yield g
    g.close()


def ulp_diff(a, b) -> int:
    a = np.ascontiguousarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.ascontiguousarray(b, np.float32).view(np.int32).astype(np.int64)
    a = np.where(a < 0, -(a & 0x7FFFFFFF), a)
    b = np.where(b < 0, -(b & 0x7FFFFFFF), b)
    return int(np.max(np.abs(a - b))) if a.size else 0


def bits_equal(a, b) -> bool:
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


# ---------------------------------------------------------------- autodiff.rs KATs
def test_matmul_known_answer(gpu):  # autodiff.rs:40-46
    t = A.Tape(gpu)
    a = t.constant(np.arange(1, 7, dtype=np.float32).reshape(2, 3))
    b = t.constant(np.arange(7, 13, dtype=np.float32).reshape(3, 2))
    c = a.matmul(b)
    assert c.shape == (2, 2)
    assert np.array_equal(c.numpy(), [[58, 64], [139, 154]])


def test_broadcast_add_known_answer(gpu):  # autodiff.rs:48-53
    t = A.Tape(gpu)
    x = t.constant(np.arange(1, 7, dtype=np.float32).reshape(2, 3))
    b = t.constant(np.array([[10, 20, 30]], np.float32))
    assert np.array_equal(x.add(b).numpy().ravel(), [11, 22, 33, 14, 25, 36])


def test_reduce_to_known_answer(gpu):  # autodiff.rs:55-60
    g = gpu.upload(np.arange(1, 7, dtype=np.float32).reshape(2, 3))
    r1, r2 = gpu.empty((1, 3)), gpu.empty((2, 1))
    gpu.reduce_to(g, r1)
    gpu.reduce_to(g, r2)
    assert np.array_equal(gpu.download(r1).ravel(), [5, 7, 9])
    assert np.array_equal(gpu.download(r2).ravel(), [6, 15])


def test_softmax_rows_normalise_and_stay_finite(gpu):  # autodiff.rs:62-72
    z = gpu.upload(np.array([[1, 2, 3], [100, 100, 100]], np.float32))
    s = gpu.empty((2, 3))
    gpu.softmax_rows(z, s)
    s = gpu.download(s)
    assert np.all(np.isfinite(s))
    assert np.all(np.abs(s.sum(axis=1) - 1) < 1e-5)


def test_gradient_accumulates_on_reused_variable(gpu):  # autodiff.rs:175-184
    w = A.Param(gpu, "w", np.array([[1.0, 2.0, 3.0]], np.float32))
    t = A.Tape(gpu)
    v = w.watch(t)
    g = v.mul(v).add(v).sum().backward()
    assert np.array_equal(gpu.download(g.of(w)).ravel(), [3.0, 5.0, 7.0])


def test_sgd_momentum_reduces_the_loss(gpu):  # autodiff.rs:214-231
    w = A.Param(gpu, "w", np.array([[4.0, -3.0]], np.float32))
    opt = A.Sgd.with_momentum(0.05, 0.9)

    def quad():
        return w.watch(A.Tape(gpu)).square().sum()

    first = quad().item()
    for _ in range(60):
        loss = quad()
        opt.step([w], loss.backward())
    last = quad().item()
    assert last < first * 1e-2

    # and the same 60 steps on the oracle land on the same weights bit for bit
    # (square, sum of two terms, SGD axpy: no reordering anywhere)
    wo = O.Param(np.array([[4.0, -3.0]], np.float32))
    oo = O.Optimizer("sgd", 0.05, 0.9)
    for _ in range(60):
        t = O.Tape()
        t.watch(wo).square().sum().backward()
        oo.step([wo], t)
    assert bits_equal(w.value(), wo.value())


def test_xor_converges(gpu):  # autodiff.rs:186-212
    rng = O.Rng(2024)
    model = A.Sequential([A.Dense(gpu, 2, 8, "tanh", rng), A.Dense(gpu, 8, 1, "sigmoid", rng)])
    x = np.array([[0, 0], [0, 1], [1, 0], [1, 1]], np.float32)
    y = np.array([[0], [1], [1], [0]], np.float32)
    xd, yd = gpu.upload(x), gpu.upload(y)
    opt = A.Adam(0.08)
    params = model.params()
    for _ in range(1500):
        t = A.Tape(gpu)
        loss = A.binary_cross_entropy(model.forward(t.constant(xd)), yd)
        opt.step(params, loss.backward())
    assert loss.item() < 0.05
    p = gpu.download(model.predict(xd))
    assert np.array_equal(p.ravel() > 0.5, y.ravel() > 0.5)


# ---------------------------------------------------------------- numeric gradients (autodiff.rs:5-35)
def check_gradients(gpu, params, grads, loss_fn):
    h = np.float32(1e-3)
    for p in params:
        g = gpu.download(grads.of(p)).ravel()
        base = p.value()
        flat = base.ravel()
        for i in range(flat.size):
            orig = flat[i]
            up_v = flat.copy()
            up_v[i] = orig + h
            p.set(up_v.reshape(base.shape))
            up = loss_fn()
            dn_v = flat.copy()
            dn_v[i] = orig - h
            p.set(dn_v.reshape(base.shape))
            down = loss_fn()
            p.set(base)
            num = (np.float32(up) - np.float32(down)) / (np.float32(2.0) * h)
            ana = g[i]
            tol = 2e-2 * (1.0 + max(abs(ana), abs(num)))
            assert abs(num - ana) < tol, (p.name, i, num, ana)


def test_mlp_mse_gradient_matches_numeric(gpu):  # autodiff.rs:81-101
    rng = O.Rng(11)
    model = A.Sequential([A.Dense(gpu, 3, 4, "tanh", rng), A.Dense(gpu, 4, 2, "linear", rng)])
    x = np.sin(np.arange(15, dtype=np.float32) * np.float32(0.37)).reshape(5, 3)
    y = np.cos(np.arange(10, dtype=np.float32) * np.float32(0.21)).reshape(5, 2)

    def fwd():
        return A.mse(model.forward(A.Tape(gpu).constant(x)), y).item()

    grads = A.mse(model.forward(A.Tape(gpu).constant(x)), y).backward()
    check_gradients(gpu, model.params(), grads, fwd)


def test_cross_entropy_gradient_matches_numeric(gpu):  # autodiff.rs:103-123
    rng = O.Rng(23)
    model = A.Sequential([A.Dense(gpu, 4, 6, "relu", rng), A.Dense(gpu, 6, 3, "linear", rng)])
    x = (np.cos(np.arange(32, dtype=np.float32) * np.float32(0.13)) * np.float32(1.5)).reshape(8, 4)
    y = A.one_hot([0, 1, 2, 1, 0, 2, 2, 0], 3)

    def fwd():
        return A.softmax_cross_entropy(model.forward(A.Tape(gpu).constant(x)), y).item()

    grads = A.softmax_cross_entropy(model.forward(A.Tape(gpu).constant(x)), y).backward()
    check_gradients(gpu, model.params(), grads, fwd)


def test_sigmoid_bce_gradient_matches_numeric(gpu):  # autodiff.rs:125-145
    rng = O.Rng(5)
    model = A.Sequential([A.Dense(gpu, 2, 5, "sigmoid", rng), A.Dense(gpu, 5, 1, "sigmoid", rng)])
    x = np.array([[0, 0], [0, 1], [1, 0], [1, 1]], np.float32)
    y = np.array([[0], [1], [1], [0]], np.float32)

    def fwd():
        return A.binary_cross_entropy(model.forward(A.Tape(gpu).constant(x)), y).item()

    grads = A.binary_cross_entropy(model.forward(A.Tape(gpu).constant(x)), y).backward()
    check_gradients(gpu, model.params(), grads, fwd)


def test_explicit_softmax_gradient_matches_numeric(gpu):  # autodiff.rs:147-173
    rng = O.Rng(31)
    model = A.Sequential([A.Dense(gpu, 3, 3, "linear", rng)])
    x = np.sin(np.arange(12, dtype=np.float32) * np.float32(0.29)).reshape(4, 3)
    y = A.one_hot([2, 0, 1, 2], 3)

    def graph():
        t = A.Tape(gpu)
        p = model.forward(t.constant(x)).softmax()
        return p.ln().mul(t.constant(y)).sum().scale(-0.25)

    check_gradients(gpu, model.params(), graph().backward(), lambda: graph().item())


# ---------------------------------------------------------------- per-op parity with the oracle tape
UNARY_CASES = [  # (op, k, input domain)
    ("scale", 1.7, "any"), ("offset", -0.3, "any"), ("neg", 0.0, "any"), ("square", 0.0, "any"),
    ("sqrt", 0.0, "pos"), ("relu", 0.0, "any"), ("leaky_relu", 0.05, "any"), ("ln", 0.0, "pos0"),
    ("exp", 0.0, "any"), ("sigmoid", 0.0, "wide"), ("tanh", 0.0, "wide"),
]
EXACT_UNARY = {"scale", "offset", "neg", "square", "sqrt", "relu", "leaky_relu"}


def unary_input(domain, shape, seed):
    r = np.random.default_rng(seed)
    x = r.standard_normal(shape).astype(np.float32)
    if domain == "pos":
        x = np.abs(x) + np.float32(1e-3)
    elif domain == "pos0":
        x = np.abs(x)
        x.ravel()[::7] = 0.0  # ln clamps at 1e-12
        x.ravel()[::11] = np.float32(1e-20)
    elif domain == "wide":
        x = x * np.float32(8.0)
    x.ravel()[::13] = 0.0
    return x


@pytest.mark.parametrize("op,k,domain", UNARY_CASES)
def test_unary_op_and_vjp_match_oracle(gpu, op, k, domain):
    shape = (37, 53)
    x = unary_input(domain, shape, hash(op) % 1000)
    gup = np.random.default_rng(7).standard_normal(shape).astype(np.float32)

    # device: value through the tape, VJP through rt_map_vjp
    xd = gpu.upload(x)
    y = gpu.empty(shape)
    gpu.map(op, xd, y, k)
    dx = gpu.empty(shape)
    gpu.map_vjp(op, gpu.upload(gup), xd, y, dx, k)
    y, dx = gpu.download(y), gpu.download(dx)

    # oracle: d/dx of sum(op(x) ⊙ G) is exactly the VJP of G
    p = O.Param(x)
    t = O.Tape()
    yo = getattr(t.watch(p), op)(k)
    yo.mul(t.constant(gup)).sum().backward()
    y_ref, dx_ref = yo.value(), t.grad(p)

    if op in EXACT_UNARY:
        assert bits_equal(y, y_ref), op
        assert bits_equal(dx, dx_ref), op
        return
    assert ulp_diff(y, y_ref) <= 4, (op, ulp_diff(y, y_ref))
    if op == "ln":  # the VJP g / x does not read the transcendental
        assert bits_equal(dx, dx_ref)
    else:
        assert O.erro_rel(dx, dx_ref) <= 1e-6, (op, O.erro_rel(dx, dx_ref))


BROADCAST_CASES = [
    ((3, 4), (3, 4)), ((3, 4), (1, 4)), ((3, 4), (4,)), ((3, 4), (3, 1)), ((1, 4), (3, 4)),
    ((2, 3, 4), (3, 1)), ((2, 1, 4), (1, 3, 1)), ((5,), (2, 1, 5)), ((64, 100), (1, 100)),
    ((2, 3, 4, 5), (3, 1, 5)), ((257, 129), (257, 1)),
]


@pytest.mark.parametrize("op", ["add", "sub", "mul", "div"])
@pytest.mark.parametrize("sa,sb", BROADCAST_CASES)
def test_binary_broadcast_value_and_grads_bit_exact(gpu, op, sa, sb):
    r = np.random.default_rng(len(sa) * 10 + len(sb))
    a = r.standard_normal(sa).astype(np.float32)
    b = r.standard_normal(sb).astype(np.float32)
    if op == "div":
        b = np.where(np.abs(b) < 0.1, np.float32(0.5), b).astype(np.float32)
    out_shape = A.broadcast_shapes(sa, sb)
    gup = r.standard_normal(out_shape).astype(np.float32)

    pa, pb = A.Param(gpu, "a", a), A.Param(gpu, "b", b)
    t = A.Tape(gpu)
    c = getattr(pa.watch(t), op)(pb.watch(t))
    grads = c.mul(t.constant(gup)).sum().backward()

    oa, ob = O.Param(a), O.Param(b)
    to = O.Tape()
    co = getattr(to.watch(oa), op)(to.watch(ob))
    co.mul(to.constant(gup)).sum().backward()

    assert c.shape == tuple(co.shape())
    assert bits_equal(c.numpy(), co.value())
    assert bits_equal(gpu.download(grads.of(pa)), to.grad(oa))
    assert bits_equal(gpu.download(grads.of(pb)), to.grad(ob))


@pytest.mark.parametrize("gshape,target", [
    ((6, 7), (1, 7)), ((6, 7), (6, 1)), ((6, 7), (7,)), ((2, 3, 4), (1, 3, 1)), ((2, 3, 4), (2, 1, 4)),
    ((2, 3, 4), (3, 4)), ((2, 3, 4, 5), (1, 3, 1, 5)), ((2048, 1000), (1, 1000)), ((1000, 300), (1000, 1)),
    ((4, 5), (4, 5)),
])
def test_reduce_to_bit_exact(gpu, gshape, target):
    g = np.random.default_rng(3).standard_normal(gshape).astype(np.float32)
    out = gpu.empty(target)
    gpu.reduce_to(gpu.upload(g), out)
    # the oracle's reduce_to for any rank, read off its tape: the VJP of
    # p + 0 (p of the target shape) for the upstream gradient g
    p = O.Param(np.zeros(target, np.float32))
    t = O.Tape()
    t.watch(p).add(t.constant(np.zeros(gshape, np.float32))).mul(t.constant(g)).sum().backward()
    want = t.grad(p)
    if len(target) == 2 and len(gshape) == 2:  # the oracle's direct reduce_to is rank 2
        assert bits_equal(want, O.reduce_to(g, target))
    assert bits_equal(gpu.download(out), want)


@pytest.mark.parametrize("n", [1, 5, 255, 256, 257, 65536, 65537, 1000003, 4 << 20])
def test_sum_all_and_scalar_reduce(gpu, n):
    x = np.random.default_rng(n).standard_normal(n).astype(np.float32)
    s = gpu.empty(())
    gpu.sum_all(gpu.upload(x), s, 1.0)
    exact = float(np.sum(x.astype(np.float64)))
    scale = float(np.sum(np.abs(x.astype(np.float64))))
    assert abs(float(gpu.download(s).ravel()[0]) - exact) <= 1e-6 * scale + 1e-30
    # reduce_to onto one element is sum_all (tensor.rs:406-409)
    r = gpu.empty((1, 1))
    gpu.reduce_to(gpu.upload(x.reshape(1, n)), r)
    assert gpu.download(r).ravel()[0] == gpu.download(s).ravel()[0]


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (5, 3, 2), (33, 17, 65), (128, 64, 96), (7, 300, 9)])
def test_matmul_value_and_grads(gpu, m, k, n):
    r = np.random.default_rng(m * k * n)
    a = r.standard_normal((m, k)).astype(np.float32)
    b = r.standard_normal((k, n)).astype(np.float32)
    gup = r.standard_normal((m, n)).astype(np.float32)
    pa, pb = A.Param(gpu, "a", a), A.Param(gpu, "b", b)
    t = A.Tape(gpu)
    c = pa.watch(t).matmul(pb.watch(t))
    grads = c.mul(t.constant(gup)).sum().backward()
    oa, ob = O.Param(a), O.Param(b)
    to = O.Tape()
    co = to.watch(oa).matmul(to.watch(ob))
    co.mul(to.constant(gup)).sum().backward()
    assert O.erro_rel(c.numpy(), co.value()) <= 1e-5
    assert O.erro_rel(gpu.download(grads.of(pa)), to.grad(oa)) <= 1e-5
    assert O.erro_rel(gpu.download(grads.of(pb)), to.grad(ob)) <= 1e-5


@pytest.mark.parametrize("red", ["sum", "mean", "softmax"])
def test_reductions_and_softmax_match_oracle(gpu, red):
    x = (np.random.default_rng(1).standard_normal((19, 23)) * 3).astype(np.float32)
    gup = np.random.default_rng(2).standard_normal((19, 23)).astype(np.float32)
    p = A.Param(gpu, "x", x)
    t = A.Tape(gpu)
    v = getattr(p.watch(t), red)()
    root = v.mul(t.constant(gup)).sum() if red == "softmax" else v.scale(1.5)
    grads = root.backward()
    po = O.Param(x)
    to = O.Tape()
    vo = getattr(to.watch(po), red)()
    (vo.mul(to.constant(gup)).sum() if red == "softmax" else vo.scale(1.5)).backward()
    assert O.erro_rel(v.numpy(), vo.value()) <= 1e-6
    assert O.erro_rel(gpu.download(grads.of(p)), to.grad(po)) <= 1e-6
    if red != "softmax":  # the VJP is Tensor::full(1.5 / n): exact
        assert bits_equal(gpu.download(grads.of(p)), to.grad(po))


def loss_f64(kind, pred, target):
    p, y = pred.astype(np.float64), target.astype(np.float64)
    if kind == "mse":
        return float(np.mean((p - y) ** 2))
    if kind == "mae":
        return float(np.mean(np.abs(p - y)))
    if kind == "binary_cross_entropy":
        c = np.clip(pred, np.float32(1e-7), np.float32(1.0) - np.float32(1e-7))
        omc = (np.float32(1.0) - c).astype(np.float64)
        return float(-np.mean(y * np.log(c.astype(np.float64)) + (1 - y) * np.log(omc)))
    z = p - p.max(axis=1, keepdims=True)
    sm = np.exp(z) / np.exp(z).sum(axis=1, keepdims=True)
    return float(-np.sum(y * np.log(np.maximum(sm, 1e-12))) / p.shape[0])


LOSSES = {"mse": A.mse, "mae": A.mae, "softmax_cross_entropy": A.softmax_cross_entropy,
          "binary_cross_entropy": A.binary_cross_entropy}


@pytest.mark.parametrize("kind", list(LOSSES))
@pytest.mark.parametrize("rows,cols", [(1, 1), (8, 3), (64, 10), (2048, 10), (100, 1)])
def test_loss_value_and_gradient_match_oracle(gpu, kind, rows, cols):
    r = np.random.default_rng(rows * 100 + cols)
    pred = r.standard_normal((rows, cols)).astype(np.float32)
    if kind == "binary_cross_entropy":
        pred = (1 / (1 + np.exp(-2 * pred))).astype(np.float32)
        pred.ravel()[::5] = 0.0  # clamped to 1e-7
        pred.ravel()[::9] = 1.0
        target = (r.random((rows, cols)) < 0.5).astype(np.float32)
    elif kind == "softmax_cross_entropy":
        target = A.one_hot(r.integers(0, cols, rows), cols)
    else:
        target = r.standard_normal((rows, cols)).astype(np.float32)
        if kind == "mae":
            target.ravel()[::4] = pred.ravel()[::4]  # sign(0) = +1
    p = A.Param(gpu, "p", pred)
    loss = LOSSES[kind](p.watch(A.Tape(gpu)), target)
    grads = loss.backward()
    po = O.Param(pred)
    to = O.Tape()
    lo = O.loss(kind, to.watch(po), target)
    lo.backward()
    # the value: within the f32 bar of the oracle's left-to-right sum, and
    # within 2e-6 of the float64 value of the same terms (the tree sum is
    # the more accurate of the two)
    assert O.erro_rel(loss.item(), lo.item()) <= 1e-4, (loss.item(), lo.item())
    exact = loss_f64(kind, pred, target)
    assert abs(loss.item() - exact) <= 2e-6 * max(1.0, abs(exact)), (loss.item(), exact, lo.item())
    g, g_ref = gpu.download(grads.of(p)), to.grad(po)
    if kind in ("mse", "mae"):
        assert bits_equal(g, g_ref)
    else:
        assert O.erro_rel(g, g_ref) <= 1e-6


# ---------------------------------------------------------------- model training parity
def build_pair(gpu, dims, acts, seed):
    """Device and oracle Sequential models with the same Glorot init."""
    ro, rd = O.Rng(seed), O.Rng(seed)
    dev = A.Sequential([A.Dense(gpu, dims[i], dims[i + 1], acts[i], rd) for i in range(len(acts))])
    ws = [(l.w.value(), l.b.value()) for l in dev.layers]
    # the oracle Dense draws from its own Rng(seed): same stream, same weights
    orc = [O.Dense(dims[i], dims[i + 1], "linear", ro) for i in range(len(acts))]
    for (w, b), l in zip(ws, orc):
        assert bits_equal(w, l.w.value())
    return dev, orc


def oracle_forward(t, layers, acts, x):
    for l, act in zip(layers, acts):
        x = x.matmul(t.watch(l.w)).add(t.watch(l.b))
        kind, slope = act if isinstance(act, tuple) else (act, 0.0)
        if kind != "linear":
            x = getattr(x, kind)(slope) if kind == "leaky_relu" else getattr(x, kind)()
    return x


TRAIN_CASES = [
    # dims, activations, loss, optimizer
    ((2, 16, 16, 1), ["tanh", "tanh", "sigmoid"], "binary_cross_entropy", ("adam", 0.01)),
    ((4, 32, 3), [("leaky_relu", 0.1), "linear"], "softmax_cross_entropy", ("sgd", 0.05, 0.9)),
    ((3, 24, 24, 2), ["sigmoid", "relu", "linear"], "mse", ("adam", 0.003)),
    ((5, 8, 4), ["tanh", "linear"], "mae", ("sgd", 0.02, 0.0)),
]


@pytest.mark.parametrize("case", TRAIN_CASES, ids=lambda c: c[2])
def test_training_trajectory_matches_oracle(gpu, case):
    dims, acts, kind, opt = case
    dev, orc = build_pair(gpu, dims, acts, seed=sum(dims))
    n = 64
    r = np.random.default_rng(dims[0])
    x = r.standard_normal((n, dims[0])).astype(np.float32)
    if kind == "softmax_cross_entropy":
        y = A.one_hot(r.integers(0, dims[-1], n), dims[-1])
    elif kind == "binary_cross_entropy":
        y = (x[:, :1] * x[:, 1:2] > 0).astype(np.float32)
    else:
        y = np.sin(x[:, : dims[-1]] * 2).astype(np.float32)
    xd, yd = gpu.upload(x), gpu.upload(y)

    if opt[0] == "adam":
        od, oo = A.Adam(opt[1]), O.Optimizer("adam", opt[1])
    else:
        od, oo = A.Sgd(opt[1], opt[2]), O.Optimizer("sgd", opt[1], opt[2])
    params_d = dev.params()
    params_o = [p for l in orc for p in (l.w, l.b)]
    loss_fn = LOSSES[kind]
    ld, lo = [], []
    for step in range(100):
        t = A.Tape(gpu)
        loss = loss_fn(dev.forward(t.constant(xd)), yd)
        grads = loss.backward()
        to = O.Tape()
        loss_o = O.loss(kind, oracle_forward(to, orc, acts, to.constant(x)), y)
        loss_o.backward()
        if step == 0:  # first-step gradients: the f32 parity bar
            for pd_, po_ in zip(params_d, params_o):
                assert O.erro_rel(gpu.download(grads.of(pd_)), to.grad(po_)) <= 1e-4
        od.step(params_d, grads)
        oo.step(params_o, to)
        ld.append(loss.value)  # read after the run: no sync per step
        lo.append(loss_o.item())
    ld = [float(gpu.download(v)) for v in ld]
    assert O.erro_rel(ld, lo) <= 1e-4, (ld[-1], lo[-1])
    assert ld[-1] < ld[0]
    for pd_, po_ in zip(params_d, params_o):
        assert O.erro_rel(pd_.value(), po_.value()) <= 1e-4


def test_predict_and_accuracy(gpu):
    rng = O.Rng(9)
    model = A.Sequential([A.Dense(gpu, 6, 12, "relu", rng), A.Dense(gpu, 12, 4, "linear", rng)])
    x = np.random.default_rng(0).standard_normal((300, 6)).astype(np.float32)
    labels = np.random.default_rng(1).integers(0, 4, 300)
    z = model.predict(x)
    zh = gpu.download(z)
    assert A.accuracy(z, labels) == O.accuracy(zh, labels)
    assert model.num_params() == 6 * 12 + 12 + 12 * 4 + 4
    assert "Dense(6 -> 12, relu)" in model.summary()


# ---------------------------------------------------------------- errors and the buffer cache
def test_shape_errors_are_reported(gpu):
    a, b = gpu.upload(np.ones((3, 4), np.float32)), gpu.upload(np.ones((2, 4), np.float32))
    with pytest.raises(G.RtError) as e:
        gpu.zip("add", a, b, gpu.empty((3, 4)))
    assert e.value.status == "RT_ERR_SHAPE"
    with pytest.raises(G.RtError):
        gpu.zip("add", a, gpu.upload(np.ones((1, 4), np.float32)), gpu.empty((4, 4)))
    with pytest.raises(G.RtError):
        gpu.reduce_to(a, gpu.empty((2, 4)))
    with pytest.raises(G.RtError):
        gpu.softmax_rows(gpu.upload(np.ones(5, np.float32)), gpu.empty((5,)))
    with pytest.raises(G.RtError):
        gpu.loss(G.LOSS_SOFTMAX_XENT, a, b, gpu.empty(()), None)
    with pytest.raises(ValueError):
        A.Tape(gpu).constant(np.ones((2, 2), np.float32)).backward()


def test_buffer_cache_reuse_keeps_results_correct(gpu):
    """Buffers freed while kernels that read them are still queued come back
    from the cache for later outputs; stream order keeps every result right."""
    r = np.random.default_rng(5)
    xs = [r.standard_normal((512, 257)).astype(np.float32) for _ in range(6)]
    want = []
    got = []
    for x in xs:
        a = gpu.upload(x)
        y = gpu.empty(x.shape)
        gpu.map("square", a, y)
        del a  # back to the cache while map may still run
        z = gpu.empty(x.shape)  # likely the same allocation as a
        gpu.map("neg", y, z)
        got.append(z)
        want.append(-(x * x))
    for g, w in zip(got, want):
        assert bits_equal(gpu.download(g), w)


@pytest.mark.parametrize("kind", ["adam", "sgd", "sgd_momentum"])
def test_multi_tensor_optimizer_matches_per_tensor(gpu, kind):
    """rt_adam_many / rt_sgd_many over a list (30 tensors: two launches) are
    bit-identical to one rt_adam / rt_sgd per tensor."""
    r = np.random.default_rng(11)
    shapes = [(int(r.integers(1, 300)), int(r.integers(1, 40))) for _ in range(30)]
    th = [r.standard_normal(s).astype(np.float32) for s in shapes]
    gs = [gpu.upload(r.standard_normal(s).astype(np.float32)) for s in shapes]
    a = [gpu.upload(t) for t in th]
    b = [gpu.upload(t) for t in th]
    ma, va = [gpu.zeros(s) for s in shapes], [gpu.zeros(s) for s in shapes]
    mb, vb = [gpu.zeros(s) for s in shapes], [gpu.zeros(s) for s in shapes]
    for t in (1, 2, 3):
        if kind == "adam":
            gpu.adam_many(a, ma, va, gs, 1e-2, t=t)
            for i in range(len(shapes)):
                gpu.adam(b[i], mb[i], vb[i], gs[i], 1e-2, t=t)
        elif kind == "sgd":
            gpu.sgd_many(a, gs, 0.1)
            for i in range(len(shapes)):
                gpu.sgd(b[i], gs[i], 0.1)
        else:
            gpu.sgd_many(a, gs, 0.1, 0.9, ma)
            for i in range(len(shapes)):
                gpu.sgd(b[i], gs[i], 0.1, 0.9, mb[i])
    for x, y in zip(a, b):
        assert bits_equal(gpu.download(x), gpu.download(y))


@pytest.mark.parametrize("kind", ["adam", "sgd_momentum"])
def test_multi_tensor_entry_point_orders_a_repeated_tensor(gpu, kind):
    """rt_adam_many / rt_sgd_many given the same tensor twice in one list
    update it twice, the second time from the first's result (a new launch
    starts at the repeat): bit-identical to two single-tensor calls."""
    r = np.random.default_rng(12)
    th, gr = r.standard_normal((70, 9)).astype(np.float32), r.standard_normal((70, 9)).astype(np.float32)
    other = r.standard_normal((5, 5)).astype(np.float32)
    a, b, g = gpu.upload(th), gpu.upload(th), gpu.upload(gr)
    o, go = gpu.upload(other), gpu.upload(other)
    ma, va, mb, vb = gpu.zeros(th.shape), gpu.zeros(th.shape), gpu.zeros(th.shape), gpu.zeros(th.shape)
    mo, vo = gpu.zeros(other.shape), gpu.zeros(other.shape)
    for t in (1, 2):
        if kind == "adam":
            gpu.adam_many([a, o, a], [ma, mo, ma], [va, vo, va], [g, go, g], 1e-2, t=t)
            gpu.adam(b, mb, vb, g, 1e-2, t=t)
            gpu.adam(b, mb, vb, g, 1e-2, t=t)
        else:
            gpu.sgd_many([a, o, a], [g, go, g], 0.1, 0.9, [ma, mo, ma])
            gpu.sgd(b, g, 0.1, 0.9, mb)
            gpu.sgd(b, g, 0.1, 0.9, mb)
    assert bits_equal(gpu.download(a), gpu.download(b))
    assert bits_equal(gpu.download(ma), gpu.download(mb))


def test_optimizer_updates_a_repeated_parameter_twice(gpu):
    """A parameter listed twice is stepped twice, one after the other, as in
    the reference's loop over params (optim.rs:167-197)."""
    w = A.Param(gpu, "w", np.array([[1.0, -2.0, 3.0]], np.float32))
    wo = O.Param(np.array([[1.0, -2.0, 3.0]], np.float32))
    opt, oo = A.Adam(0.1), O.Optimizer("adam", 0.1)
    for _ in range(3):
        opt.step([w, w], w.watch(A.Tape(gpu)).square().sum().backward())
        t = O.Tape()
        t.watch(wo).square().sum().backward()
        oo.step([wo, wo], t)
    assert bits_equal(w.value(), wo.value())


@pytest.mark.parametrize("act", ["relu", "linear"])
def test_fused_dense_node_matches_op_by_op(gpu, act):
    """dense_node (GEMM with bias/ReLU epilogue, colsum-fused db) against the
    reference's matmul -> add -> relu recording: same forward bits, same dX
    and dW bits (the same GEMM calls), db within rounding."""
    r = np.random.default_rng(21)
    x = r.standard_normal((96, 40)).astype(np.float32)
    w = r.standard_normal((40, 72)).astype(np.float32) * np.float32(0.2)
    b = r.standard_normal((1, 72)).astype(np.float32)
    gup = r.standard_normal((96, 72)).astype(np.float32)
    outs = []
    for fused in (True, False):
        layer = A.Dense(gpu, 40, 72, act, weights=w, bias=b, fused=fused)
        t = A.Tape(gpu)
        px = A.Param(gpu, "x", x)
        y = layer.forward(px.watch(t))
        grads = y.mul(t.constant(gup)).sum().backward()
        outs.append((y.numpy(), gpu.download(grads.of(px)), gpu.download(grads.of(layer.w)),
                     gpu.download(grads.of(layer.b)), len(t)))
    (yf, dxf, dwf, dbf, nf), (yu, dxu, dwu, dbu, nu) = outs
    assert nf < nu  # fewer tape nodes
    assert bits_equal(yf, yu)
    assert bits_equal(dxf, dxu)
    assert bits_equal(dwf, dwu)
    assert O.erro_rel(dbf, dbu) <= 1e-6


@pytest.mark.parametrize("rows,cols", [(1, 3), (256, 10), (257, 10), (3000, 33)])
def test_xent_from_logits_matches_probability_form(gpu, rows, cols):
    """RT_LOSS_SOFTMAX_XENT_LOGITS (one pass per row) against softmax_rows +
    RT_LOSS_SOFTMAX_XENT: the same P − Y bits, the value within rounding."""
    r = np.random.default_rng(rows + cols)
    z = (r.standard_normal((rows, cols)) * 4).astype(np.float32)
    y = A.one_hot(r.integers(0, cols, rows), cols)
    zd, yd = gpu.upload(z), gpu.upload(y)
    probs = gpu.empty((rows, cols))
    gpu.softmax_rows(zd, probs)
    v1, d1 = gpu.empty(()), gpu.empty((rows, cols))
    gpu.loss(G.LOSS_SOFTMAX_XENT, probs, yd, v1, d1)
    v2, d2 = gpu.empty(()), gpu.empty((rows, cols))
    gpu.loss(G.LOSS_SOFTMAX_XENT_LOGITS, zd, yd, v2, d2)
    assert bits_equal(gpu.download(d1), gpu.download(d2))
    a, b = float(gpu.download(v1)), float(gpu.download(v2))
    assert abs(a - b) <= 1e-6 * max(1.0, abs(a))


def test_softmax_xent_gradient_off_the_root(gpu):
    """The loss's VJP when its upstream is not the seed of ones (the loss is
    scaled, or added to itself, before backward): P − Y recomputed and
    scaled by ḡ / n, against the oracle's tape; the root case returns the
    gradient computed in the forward launch, and a second backward pass over
    the same tape gives the same bits (that buffer is never written through)."""
    r = np.random.default_rng(77)
    z = r.standard_normal((33, 7)).astype(np.float32)
    y = A.one_hot(r.integers(0, 7, 33), 7)
    for build in (lambda v: v.scale(3.0), lambda v: v.add(v), lambda v: v):
        p = A.Param(gpu, "z", z)
        total = build(A.softmax_cross_entropy(p.watch(A.Tape(gpu)), y))
        g1 = gpu.download(total.backward().of(p))
        g2 = gpu.download(total.backward().of(p))
        assert bits_equal(g1, g2)
        po = O.Param(z)
        to = O.Tape()
        build(O.loss("softmax_cross_entropy", to.watch(po), y)).backward()
        assert O.erro_rel(g1, to.grad(po)) <= 1e-6
