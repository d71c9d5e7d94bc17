"""rtensor's autodiff on the device: Tape, Var, Param, losses, optimizers and
Sequential/Dense, with every tensor in HBM and every op a HIP kernel.

The host side mirrors the reference's API (crates/rtensor/src/):

==========================  ==================================================
reference                   here
==========================  ==================================================
Tape, constant (tape.rs)    Tape(gpu), constant(tape, value) / tape.constant
Param (tape.rs:76-132)      Param(gpu, name, value); .watch(tape), .set, .value
Var ops (ops.rs:49-309)     Var.add/sub/mul/div/matmul/scale/offset/neg/square/
                            sqrt/exp/ln/relu/leaky_relu/sigmoid/tanh/sum/mean/
                            softmax
Var::backward (187-229)     Var.backward() -> Grads (.of(param), .of_var(var))
losses.rs                   mse, mae, softmax_cross_entropy,
                            binary_cross_entropy, one_hot, accuracy
optim.rs                    Sgd(lr, momentum), Adam(lr, beta1, beta2): .step
nn.rs                       Activation names, Dense, Sequential
==========================  ==================================================

Values are device tensors (``GpuTensor``); each op enqueues its kernels on the
context's stream and nothing waits for the device until a value is read
(``Var.numpy``, ``Var.item``, ``Param.value``).  Differences from the
reference, all of layout and not of arithmetic:

* A watched ``Param`` aliases its device buffer (the reference clones the
  tensor into the Var); an optimizer step therefore has to come after the
  backward pass that reads it, as it does in every training loop.
* A VJP that returns its upstream gradient unchanged (``offset``, and
  ``reduce_to`` onto the same shape) shares that buffer instead of copying it;
  the backward sweep accumulates into a shared gradient out of place, so no
  gradient is modified through an alias.

There is no CPU fallback: the ops call ``librtensor_hip.so`` and fail with
``RtError`` if it or the device is missing.
"""
from __future__ import annotations

import itertools
from typing import Callable, Dict, List, Optional, Sequence, Tuple, Union

import numpy as np

from .gpu import (EPI_BIAS, EPI_BIAS_RELU, LOSS_BCE, LOSS_MAE, LOSS_SOFTMAX_XENT_LOGITS,
                  LOSS_SOFTMAX_XENT_LOGITS_MEAN, NN, NT, TN, Gpu, GpuTensor, RtError, upload_labels)

Shape = Tuple[int, ...]

_next_param_id = itertools.count()


def broadcast_shapes(a: Sequence[int], b: Sequence[int]) -> Shape:
    """tensor.rs:575-592 (numpy rules; raises ValueError where it panics)."""
    r = max(len(a), len(b))
    out = []
    for i in range(r):
        da = 1 if i < r - len(a) else a[i - (r - len(a))]
        db = 1 if i < r - len(b) else b[i - (r - len(b))]
        if da == db or db == 1:
            out.append(da)
        elif da == 1:
            out.append(db)
        else:
            raise ValueError(f"shapes do not broadcast: {tuple(a)} and {tuple(b)}")
    return tuple(out)


def _numel(shape: Sequence[int]) -> int:
    n = 1
    for s in shape:
        n *= int(s)
    return n


def _as_device(gpu: Gpu, v) -> GpuTensor:
    if isinstance(v, GpuTensor):
        return v
    return gpu.upload(np.ascontiguousarray(v, dtype=np.float32))


def _ones(gpu: Gpu, shape) -> GpuTensor:
    """A device tensor of ones of this shape, uploaded once and kept on the
    Gpu object (the seed of backward; never written)."""
    cache = getattr(gpu, "_autograd_ones", None)
    if cache is None:
        cache = gpu._autograd_ones = {}
    key = tuple(int(d) for d in shape)
    t = cache.get(key)
    if t is None or not t.handle:
        t = cache[key] = gpu.upload(np.ones(key, np.float32))
    return t


# ------------------------------------------------------------------ tape
class Tape:
    """tape.rs:43-67: nodes in creation (topological) order."""

    def __init__(self, gpu: Gpu):
        self.gpu = gpu
        self.nodes: List[Tuple[Tuple[int, ...], Optional[Callable]]] = []
        self.param_nodes: Dict[int, int] = {}

    def _push(self, parents: Tuple[int, ...], backward: Optional[Callable]) -> int:
        self.nodes.append((parents, backward))
        return len(self.nodes) - 1

    def __len__(self) -> int:
        return len(self.nodes)

    def constant(self, value) -> "Var":
        return constant(self, value)

    def watch(self, p: "Param") -> "Var":
        return p.watch(self)


def constant(tape: Tape, value) -> "Var":
    """tape.rs:70-73: a leaf that takes part in the graph without a VJP."""
    return Var(tape, tape._push((), None), _as_device(tape.gpu, value))


class Param:
    """tape.rs:76-132: a trainable tensor, updated in place by optimizers."""

    def __init__(self, gpu: Gpu, name: str, value):
        self.gpu = gpu
        self.id = next(_next_param_id)
        self.name = name
        self.tensor = _as_device(gpu, value)

    @property
    def shape(self) -> Shape:
        return self.tensor.shape

    def value(self) -> np.ndarray:
        """The current value, downloaded (blocks)."""
        return self.gpu.download(self.tensor)

    def set(self, v) -> None:
        """Param::set (tape.rs:119-121); the shape may change, as there."""
        v = np.ascontiguousarray(v, dtype=np.float32)
        if v.shape == self.tensor.shape:
            self.gpu.write(self.tensor, v)
        else:
            self.tensor = self.gpu.upload(v)

    def watch(self, tape: Tape) -> "Var":
        """tape.rs:124-131: one leaf per parameter per tape."""
        idx = tape.param_nodes.get(self.id)
        if idx is None:
            idx = tape._push((), None)
            tape.param_nodes[self.id] = idx
        return Var(tape, idx, self.tensor)


# ------------------------------------------------------------------ vars and ops
class Var:
    """tape.rs:135-185: a node of the graph and its device value."""

    __slots__ = ("tape", "idx", "value")

    def __init__(self, tape: Tape, idx: int, value: GpuTensor):
        self.tape, self.idx, self.value = tape, idx, value

    @property
    def gpu(self) -> Gpu:
        return self.tape.gpu

    @property
    def shape(self) -> Shape:
        return self.value.shape

    def numpy(self) -> np.ndarray:
        return self.gpu.download(self.value)

    def item(self) -> float:
        if len(self.value) != 1:
            raise ValueError(f"item() needs a one-element tensor, shape {self.shape}")
        return float(self.numpy().reshape(-1)[0])

    # -------------------------------------------------------------- recording
    def _unary(self, value: GpuTensor, backward: Callable[[GpuTensor], GpuTensor]) -> "Var":
        idx = self.tape._push((self.idx,), lambda g: (backward(g),))
        return Var(self.tape, idx, value)

    def _binary(self, other: "Var", value: GpuTensor,
                backward: Callable[[GpuTensor], Tuple[GpuTensor, GpuTensor]]) -> "Var":
        if other.tape is not self.tape:
            raise ValueError("operands belong to different tapes")  # tape.rs:163-166
        idx = self.tape._push((self.idx, other.idx), backward)
        return Var(self.tape, idx, value)

    def _empty(self, shape) -> GpuTensor:
        return self.gpu.empty(shape)

    def _map(self, op: str, k: float = 0.0) -> GpuTensor:
        y = self._empty(self.shape)
        self.gpu.map(op, self.value, y, k)
        return y

    # -------------------------------------------------------------- binary ops
    def _zip(self, op: str, other: "Var") -> GpuTensor:
        out = self._empty(broadcast_shapes(self.shape, other.shape))
        self.gpu.zip(op, self.value, other.value, out)
        return out

    def add(self, other: "Var") -> "Var":
        """ops.rs:49-53: (reduce(ḡ), reduce(ḡ))."""
        sa, sb = self.shape, other.shape
        gpu = self.gpu
        return self._binary(other, self._zip("add", other),
                            lambda g: (_reduce_to(gpu, g, sa), _reduce_to(gpu, g, sb)))

    def sub(self, other: "Var") -> "Var":
        """ops.rs:61-65: (reduce(ḡ), reduce(−ḡ))."""
        sa, sb = self.shape, other.shape
        gpu = self.gpu
        return self._binary(other, self._zip("sub", other),
                            lambda g: (_reduce_to(gpu, g, sa), _reduce_to(gpu, _map(gpu, "neg", g), sb)))

    def mul(self, other: "Var") -> "Var":
        """ops.rs:76-83: (reduce(ḡ ⊙ B), reduce(ḡ ⊙ A))."""
        a, b = self.value, other.value
        gpu = self.gpu
        return self._binary(other, self._zip("mul", other),
                            lambda g: (_reduce_to(gpu, _zip(gpu, "mul", g, b), a.shape),
                                       _reduce_to(gpu, _zip(gpu, "mul", g, a), b.shape)))

    def div(self, other: "Var") -> "Var":
        """ops.rs:93-102: (reduce(ḡ ⊘ B), reduce(−(ḡ ⊙ A) ⊘ (B ⊙ B)))."""
        a, b = self.value, other.value
        gpu = self.gpu

        def bw(g):
            da = _reduce_to(gpu, _zip(gpu, "div", g, b), a.shape)
            q = _zip(gpu, "div", _zip(gpu, "mul", g, a), _zip(gpu, "mul", b, b))
            return da, _reduce_to(gpu, _map(gpu, "neg", q), b.shape)

        return self._binary(other, self._zip("div", other), bw)

    def matmul(self, other: "Var") -> "Var":
        """ops.rs:125-129 with rt_gemm: C = A·B; Ā = ḡ·Bᵀ (NT), B̄ = Aᵀ·ḡ (TN)."""
        a, b = self.value, other.value
        if len(a.shape) != 2 or len(b.shape) != 2:
            raise ValueError(f"matmul needs rank 2, got {a.shape} and {b.shape}")
        (m, k), (k2, n) = a.shape, b.shape
        if k != k2:
            raise ValueError(f"incompatible shapes: {a.shape} x {b.shape}")
        gpu = self.gpu
        c = self._empty((m, n))
        gpu.gemm(NN, a, b, c)

        def bw(g):
            ga = gpu.empty((m, k))
            gb = gpu.empty((k, n))
            gpu.gemm(NT, g, b, ga)
            gpu.gemm(TN, a, g, gb)
            return ga, gb

        return self._binary(other, c, bw)

    # -------------------------------------------------------------- unary ops
    def _pointwise(self, op: str, k: float = 0.0) -> "Var":
        x = self.value
        y = self._map(op, k)
        gpu = self.gpu

        def bw(g):
            dx = gpu.empty(x.shape)
            gpu.map_vjp(op, g, x, y, dx, k)
            return dx

        return self._unary(y, bw)

    def scale(self, k: float) -> "Var":
        return self._pointwise("scale", k)

    def offset(self, k: float) -> "Var":
        return self._unary(self._map("offset", k), lambda g: g)

    def neg(self) -> "Var":
        return self._pointwise("neg")

    def square(self) -> "Var":
        return self._pointwise("square")

    def sqrt(self) -> "Var":
        return self._pointwise("sqrt")

    def exp(self) -> "Var":
        return self._pointwise("exp")

    def ln(self) -> "Var":
        return self._pointwise("ln")

    def relu(self) -> "Var":
        return self._pointwise("relu")

    def leaky_relu(self, slope: float) -> "Var":
        return self._pointwise("leaky_relu", slope)

    def sigmoid(self) -> "Var":
        return self._pointwise("sigmoid")

    def tanh(self) -> "Var":
        return self._pointwise("tanh")

    def sum(self) -> "Var":
        """ops.rs:239-243: scalar Σx; VJP full(shape, ḡ)."""
        return self._reduce_all(1.0)

    def mean(self) -> "Var":
        """ops.rs:250-255: scalar Σx / n; VJP full(shape, ḡ / n)."""
        return self._reduce_all(float(np.float32(len(self.value))))

    def _reduce_all(self, div: float) -> "Var":
        gpu, shape = self.gpu, self.shape
        out = gpu.empty(())
        gpu.sum_all(self.value, out, div)

        def bw(g):
            dx = gpu.empty(shape)
            gpu.fill_scaled(g, dx, div)
            return dx

        return self._unary(out, bw)

    def softmax(self) -> "Var":
        """ops.rs:288-309: row softmax; VJP s ⊙ (ḡ − rowsum(ḡ ⊙ s))."""
        gpu = self.gpu
        if len(self.shape) != 2:
            raise ValueError("softmax needs rank 2")
        s = gpu.empty(self.shape)
        gpu.softmax_rows(self.value, s)

        def bw(g):
            dx = gpu.empty(s.shape)
            gpu.softmax_rows_vjp(s, g, dx)
            return dx

        return self._unary(s, bw)

    # -------------------------------------------------------------- backward
    def backward(self) -> "Grads":
        """tape.rs:187-229: seed ones, sweep nodes in reverse, accumulate."""
        if len(self.value) != 1:
            raise ValueError(f"backward() must start at a scalar, shape {self.shape}")
        gpu = self.gpu
        nodes = self.tape.nodes
        grads: List[Optional[GpuTensor]] = [None] * len(nodes)
        shared = [False] * len(nodes)
        grads[self.idx] = _ones(gpu, self.shape)  # shared: accumulated into out of place
        shared[self.idx] = True
        for i in range(len(nodes) - 1, -1, -1):
            parents, backward = nodes[i]
            g = grads[i]
            if backward is None or g is None:
                continue
            for p, gp in zip(parents, backward(g)):
                acc = grads[p]
                if acc is None:
                    grads[p] = gp
                    shared[p] = gp is g or getattr(gp, "vjp_shared", False)
                elif acc.shape == gp.shape and not shared[p]:
                    gpu.zip("add", acc, gp, acc)  # v̄_j += Jᵀ v̄_i in place
                else:
                    s = gpu.empty(broadcast_shapes(acc.shape, gp.shape))
                    gpu.zip("add", acc, gp, s)
                    grads[p] = s
                    shared[p] = False
        return Grads(grads, dict(self.tape.param_nodes))


class Grads:
    """tape.rs:232-252."""

    def __init__(self, grads: List[Optional[GpuTensor]], param_nodes: Dict[int, int]):
        self.grads = grads
        self.param_nodes = param_nodes

    def of(self, p: Param) -> Optional[GpuTensor]:
        idx = self.param_nodes.get(p.id)
        return None if idx is None else self.grads[idx]

    def of_var(self, v: Var) -> Optional[GpuTensor]:
        return self.grads[v.idx]


def _map(gpu: Gpu, op: str, x: GpuTensor, k: float = 0.0) -> GpuTensor:
    y = gpu.empty(x.shape)
    gpu.map(op, x, y, k)
    return y


def _zip(gpu: Gpu, op: str, a: GpuTensor, b: GpuTensor) -> GpuTensor:
    out = gpu.empty(broadcast_shapes(a.shape, b.shape))
    gpu.zip(op, a, b, out)
    return out


def _reduce_to(gpu: Gpu, g: GpuTensor, shape: Shape) -> GpuTensor:
    """tensor.rs:399-438; the same shape returns g itself (shared, see Var.backward)."""
    if tuple(g.shape) == tuple(shape):
        return g
    out = gpu.empty(shape)
    gpu.reduce_to(g, out)
    return out


# ------------------------------------------------------------------ losses
def mse(pred: Var, target) -> Var:
    """losses.rs:31-34: sub → square → mean."""
    return pred.sub(constant(pred.tape, target)).square().mean()


def mae(pred: Var, target) -> Var:
    """losses.rs:46-53: mean |d|, VJP sign(d) · ḡ / n (sign(0) = +1)."""
    d = pred.sub(constant(pred.tape, target))
    gpu = pred.gpu
    value, sign = gpu.empty(()), gpu.empty(d.shape)
    gpu.loss(LOSS_MAE, d.value, None, value, sign)
    n = float(np.float32(len(d.value)))

    def bw(g):
        dx = gpu.empty(sign.shape)
        gpu.fill_scaled(g, dx, n, sign)
        return dx

    return d._unary(value, bw)


def softmax_cross_entropy(logits: Var, targets) -> Var:
    """losses.rs:99-115: −(1/n) Σ y ln max(p, 1e-12); VJP (P − Y) · ḡ / n."""
    gpu = logits.gpu
    y = _as_device(gpu, targets)
    if tuple(y.shape) != tuple(logits.shape):
        raise ValueError("logits and targets differ in shape")
    # Softmax, loss and the gradient for ḡ = 1, (P − Y)·(1/n), in one launch:
    # the VJP of a loss that is the root of backward() (its upstream is the
    # seed of ones) is then that buffer, shared (never written through).
    value, dmean = gpu.empty(()), gpu.empty(logits.shape)
    gpu.loss(LOSS_SOFTMAX_XENT_LOGITS_MEAN, logits.value, y, value, dmean)
    dmean.vjp_shared = True
    batch = float(np.float32(logits.shape[0]))
    z = logits.value

    def bw(g):
        if g is _ones(gpu, ()):
            return dmean
        dirn, scratch = gpu.empty(z.shape), gpu.empty(())
        gpu.loss(LOSS_SOFTMAX_XENT_LOGITS, z, y, scratch, dirn)  # P − Y again
        dx = gpu.empty(dirn.shape)
        gpu.fill_scaled(g, dx, batch, dirn)
        return dx

    return logits._unary(value, bw)


def binary_cross_entropy(probs: Var, targets) -> Var:
    """losses.rs:143-162 with clamp(p, 1e-7, 1 − 1e-7)."""
    gpu = probs.gpu
    y = _as_device(gpu, targets)
    if len(y) != len(probs.value):
        raise ValueError("probabilities and targets differ in size")
    value, dirn = gpu.empty(()), gpu.empty(probs.shape)
    gpu.loss(LOSS_BCE, probs.value, y, value, dirn)
    n = float(np.float32(len(probs.value)))

    def bw(g):
        dx = gpu.empty(dirn.shape)
        gpu.fill_scaled(g, dx, n, dirn)
        return dx

    return probs._unary(value, bw)


def one_hot(labels, classes: int) -> np.ndarray:
    """losses.rs:169-175 (host); a label >= classes raises (a panic there)."""
    lab = np.asarray(labels, dtype=np.int64).reshape(-1)
    if lab.size and (lab.min() < 0 or lab.max() >= classes):
        raise IndexError("label out of range")
    out = np.zeros((lab.size, classes), np.float32)
    out[np.arange(lab.size), lab] = 1.0
    return out


def accuracy(logits: Union[Var, GpuTensor], labels) -> float:
    """losses.rs:181-185 on the device (rt_accuracy)."""
    z = logits.value if isinstance(logits, Var) else logits
    lab = labels if isinstance(labels, GpuTensor) else upload_labels(z.gpu, labels)
    return z.gpu.accuracy(z, lab)


# ------------------------------------------------------------------ optimizers
def _live_groups(params: Sequence[Param], grads: Grads):
    """The parameters that have a gradient, in order, cut into runs without a
    repeated parameter: the reference updates a parameter listed twice twice,
    one after the other, and one launch cannot."""
    groups, cur, seen = [], [], set()
    for p in params:
        g = grads.of(p)
        if g is None:
            continue
        if p.id in seen:
            groups.append(cur)
            cur, seen = [], set()
        cur.append((p, g))
        seen.add(p.id)
    if cur:
        groups.append(cur)
    return groups


class Sgd:
    """optim.rs:64-114: θ −= α g, or v = μ v + α g; θ −= v."""

    def __init__(self, lr: float, momentum: float = 0.0):
        self.lr, self.momentum = lr, momentum
        self.velocity: Dict[int, GpuTensor] = {}

    @classmethod
    def with_momentum(cls, lr: float, momentum: float) -> "Sgd":
        return cls(lr, momentum)

    def step(self, params: Sequence[Param], grads: Grads) -> None:
        for live in _live_groups(params, grads):
            gpu = live[0][0].gpu
            thetas, gs = [p.tensor for p, _ in live], [g for _, g in live]
            if self.momentum == 0.0:
                gpu.sgd_many(thetas, gs, self.lr)
                continue
            vel = []
            for p, _ in live:
                v = self.velocity.get(p.id)
                if v is None:
                    v = self.velocity[p.id] = p.gpu.zeros(p.shape)
                vel.append(v)
            gpu.sgd_many(thetas, gs, self.lr, self.momentum, vel)


class Adam:
    """optim.rs:136-198: bias-corrected moments; t counts step() calls."""

    def __init__(self, lr: float, beta1: float = 0.9, beta2: float = 0.999, eps: float = 1e-8):
        self.lr, self.beta1, self.beta2, self.eps = lr, beta1, beta2, eps
        self.t = 0
        self.m: Dict[int, GpuTensor] = {}
        self.v: Dict[int, GpuTensor] = {}

    @classmethod
    def with_betas(cls, lr: float, beta1: float, beta2: float) -> "Adam":
        return cls(lr, beta1, beta2)

    def step(self, params: Sequence[Param], grads: Grads) -> None:
        self.t += 1
        for live in _live_groups(params, grads):
            for p, _ in live:
                if p.id not in self.m:
                    self.m[p.id] = p.gpu.zeros(p.shape)
                    self.v[p.id] = p.gpu.zeros(p.shape)
            live[0][0].gpu.adam_many([p.tensor for p, _ in live], [self.m[p.id] for p, _ in live],
                                     [self.v[p.id] for p, _ in live], [g for _, g in live], self.lr,
                                     (self.beta1, self.beta2), self.t, self.eps)


# ------------------------------------------------------------------ layers
def _activation(name) -> Tuple[str, float]:
    if isinstance(name, tuple):
        return name[0], float(name[1])
    return name, 0.0


def apply_activation(z: Var, activation) -> Var:
    """nn.rs:52-60: linear, relu, (leaky_relu, slope), sigmoid, tanh."""
    kind, slope = _activation(activation)
    if kind == "linear":
        return z
    if kind == "relu":
        return z.relu()
    if kind == "leaky_relu":
        return z.leaky_relu(slope)
    if kind == "sigmoid":
        return z.sigmoid()
    if kind == "tanh":
        return z.tanh()
    raise ValueError(f"unknown activation {activation!r}")


def dense_node(x: Var, w: Var, b: Var, relu: bool) -> Var:
    """A = φ(X W + 1ₙ b) for φ = relu or linear as ONE tape node: the GEMM
    applies the bias (and ReLU) in its epilogue, whose arithmetic is the
    reference's matmul, add and relu in sequence (acc + b, then max(·, 0)),
    so the values are the same bits.  Backward: δ = ḡ ⊙ 1[A > 0] (A > 0
    exactly where Z > 0), dW = Xᵀδ with db = 1ᵀδ summed in the same launch,
    dX = δ Wᵀ — the ReLU VJP and one paired GEMM launch where the node-per-op
    tape takes four, and one forward launch instead of three.  db is summed in the GEMM's order, not
    reduce_to's row order: equal within rounding, not bit for bit."""
    gpu = x.gpu
    xv, wv, bv = x.value, w.value, b.value
    (m, k), (k2, n) = xv.shape, wv.shape
    if k != k2 or bv.shape not in ((1, n), (n,)):
        raise ValueError(f"dense: {xv.shape} x {wv.shape} + {bv.shape}")
    a = gpu.empty((m, n))
    gpu.gemm(NN, xv, wv, a, EPI_BIAS_RELU if relu else EPI_BIAS, bv)

    def bw(g):
        if relu:
            d = gpu.empty((m, n))
            gpu.map_vjp("relu", g, a, None, d)
        else:
            d = g
        dx, dw, db = gpu.empty((m, k)), gpu.empty((k, n)), gpu.empty(bv.shape)
        gpu.linear_backward(xv, d, wv, dx, dw, db)  # TN + colsum and NT, one launch where it can
        return dx, dw, db

    if x.tape is not w.tape or w.tape is not b.tape:
        raise ValueError("operands belong to different tapes")
    idx = x.tape._push((x.idx, w.idx, b.idx), bw)
    return Var(x.tape, idx, a)


class Dense:
    """nn.rs:108-159: A = φ(X W + 1ₙ b), W [inputs, units], b [1, units].

    The Glorot-uniform draw (nn.rs:122-130) takes its numbers from ``rng``,
    any object with ``range(lo, hi)`` (or a vectorised ``ranges(n, lo, hi)``)
    that follows rtensor's Rng; or pass ``weights`` / ``bias`` directly.
    With ``fused`` (the default) a ReLU or linear layer is one tape node
    (``dense_node``); ``fused=False`` records matmul, add and the activation
    as the reference does."""

    def __init__(self, gpu: Gpu, inputs: int, units: int, activation="linear", rng=None,
                 weights=None, bias=None, fused: bool = True):
        self.fused = fused
        if weights is None:
            if rng is None:
                raise ValueError("Dense needs an rng or explicit weights")
            limit = float(np.sqrt(np.float32(6.0) / np.float32(inputs + units), dtype=np.float32))
            n = inputs * units
            if hasattr(rng, "ranges"):
                w = np.asarray(rng.ranges(n, -limit, limit), np.float32)
            else:
                w = np.array([rng.range(-limit, limit) for _ in range(n)], np.float32)
            weights = w.reshape(inputs, units)
        if bias is None:
            bias = np.zeros((1, units), np.float32)
        self.w = Param(gpu, "W", np.asarray(weights, np.float32).reshape(inputs, units))
        self.b = Param(gpu, "b", np.asarray(bias, np.float32).reshape(1, units))
        self.activation = activation

    def weights(self) -> Param:
        return self.w

    def bias(self) -> Param:
        return self.b

    def forward(self, x: Var) -> Var:
        t = x.tape
        w, b = self.w.watch(t), self.b.watch(t)
        kind, _ = _activation(self.activation)
        if self.fused and kind in ("relu", "linear") and len(x.shape) == 2:
            return dense_node(x, w, b, kind == "relu")
        z = x.matmul(w).add(b)
        return apply_activation(z, self.activation)

    def params(self) -> List[Param]:
        return [self.w, self.b]

    def describe(self) -> str:
        kind, slope = _activation(self.activation)
        act = f"leaky_relu({slope})" if kind == "leaky_relu" else kind
        return f"Dense({self.w.shape[0]} -> {self.w.shape[1]}, {act})"


class Sequential:
    """nn.rs:161-215."""

    def __init__(self, layers: Sequence = ()):
        self.layers = list(layers)

    def add(self, layer) -> "Sequential":
        self.layers.append(layer)
        return self

    def forward(self, x: Var) -> Var:
        for layer in self.layers:
            x = layer.forward(x)
        return x

    def predict(self, x) -> GpuTensor:
        """Forward without keeping a tape for backward (nn.rs:184-188)."""
        gpu = self.layers[0].w.gpu
        return self.forward(constant(Tape(gpu), x)).value

    def params(self) -> List[Param]:
        return [p for layer in self.layers for p in layer.params()]

    def num_params(self) -> int:
        return sum(_numel(p.shape) for p in self.params())

    def summary(self) -> str:
        lines = ["Sequential"] + [f"  {layer.describe()}" for layer in self.layers]
        lines.append(f"  params: {self.num_params()}")
        return "\n".join(lines)


__all__ = ["Tape", "constant", "Param", "Var", "Grads", "mse", "mae", "softmax_cross_entropy",
           "binary_cross_entropy", "one_hot", "accuracy", "Sgd", "Adam", "Dense", "Sequential",
           "apply_activation", "broadcast_shapes", "RtError"]
