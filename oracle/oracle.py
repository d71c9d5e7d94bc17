"""CPU oracle for the rtensor training step -- TEST INFRASTRUCTURE ONLY.

This module wraps ``librtensor_cpu.so`` (built from ``rtensor_cpu.cpp`` by
the Makefile beside it), a C++ restatement of rtensor's single-threaded CPU
path.  It is the oracle the HIP backend in ``rgpu_amd`` is tested against, and the CPU
baseline that ``bench.py`` times.  Only ``tests/``, ``__graft_entry__.smoke``
and ``bench.py``'s ``cpu_baseline`` leg may import it; the product path never
does.

Parity status of each restated function (what pins it, all in tests/):

===========================  ==========================================================
function (reference file)    pinned by
===========================  ==========================================================
Rng (src/rng.rs:3-49)        golden u64/f32 streams computed with Python integer
                             arithmetic (tests/golden/make_rng_vectors.py); Box-Muller
                             checked against a float64 restatement to 1 ulp-ish and by
                             moments; below() exact
matmul (tensor.rs:318-373)   autodiff.rs:40-46 KAT; float64 brute force on the 7 gpu.rs
                             shapes; bit-identity of row-parallel vs 1 thread;
                             exact results on integer-valued inputs
t (tensor.rs:132-155)        involution KAT (autodiff.rs:74-79); numpy transpose
zip/add (tensor.rs:183-246)  broadcast KAT (autodiff.rs:48-53)
reduce_to (399-438)          KATs [5,7,9] and [6,15] (autodiff.rs:55-60)
softmax_rows (455-472)       rows sum to 1, finite at logits 100 (autodiff.rs:62-72);
                             float64 softmax within 2 ulp
argmax_rows (476-493)        first-max tie rule on hand-built rows
tape + VJPs (tape.rs, ops.rs) central-difference gradient checks of autodiff.rs:81-173;
                             fan-out accumulation KAT [3,5,7] (autodiff.rs:175-184)
div VJP (ops.rs:93-102)      float64 closed form (A/B: g/B, -g·A/B²) over 5 broadcast
                             shape pairs incl. reduction axes; central differences
offset, sqrt, exp VJPs       float64 derivative (1, 1/(2√x), eˣ) times a random
(ops.rs:139-142, 158-170)    upstream, within 1e-6; central differences of the forward
leaky_relu VJP (197-203)     float64 derivative; x = ±0 takes the slope; the slope
                             argument is honoured (two slopes, exact)
mae (losses.rs:46-53)        value vs float64; gradient exactly sign(d)·(ḡ/N) with
                             sign(0) = +1 and ḡ = 3; central differences off the kink
softmax_cross_entropy        numeric gradient check; delta rows sum to 0;
(losses.rs:99-115)           delta[r, y_r] in [-1/B, 0]; loss = mean(-ln p_y) in float64
Sgd (optim.rs:80-114)        exact axpy; momentum convergence (autodiff.rs:214-231)
Adam (optim.rs:162-198)      t=1 closed form (step = -lr*g/(|g|+eps)); powi against
                             exact float64 power rounded; XOR convergence (186-212)
Dense init (nn.rs:122-130)   Glorot bound and draw order against Rng golden stream
===========================  ==========================================================

The bit-level behaviour of glibc ``expf``/``logf``/``cosf`` against the Rust
reference's calls into the same libm is assumed, not pinned: the Rust
reference cannot be compiled here (no rustc/cargo).  The tolerance tests do
not depend on it.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import List, Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "librtensor_cpu.so")
_lib: Optional[C.CDLL] = None

F32P = C.POINTER(C.c_float)
U32P = C.POINTER(C.c_uint32)
SZP = C.POINTER(C.c_size_t)
I64P = C.POINTER(C.c_int64)


def _p(a: np.ndarray, t=F32P):
    return a.ctypes.data_as(t)


def lib() -> C.CDLL:
    """Load the oracle library (build it with ``make -C oracle``)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        raise RuntimeError(f"oracle library missing: {_LIB_PATH} (run `make -C oracle`)")
    L = C.CDLL(_LIB_PATH)
    sig = {
        "ocpu_last_error": (C.c_char_p, []),
        "ocpu_set_threads": (None, [C.c_int]),
        "ocpu_get_threads": (C.c_int, []),
        "ocpu_rng_new": (C.c_void_p, [C.c_uint64]),
        "ocpu_rng_free": (None, [C.c_void_p]),
        "ocpu_rng_next_u64": (C.c_uint64, [C.c_void_p]),
        "ocpu_rng_uniform": (C.c_float, [C.c_void_p]),
        "ocpu_rng_range": (C.c_float, [C.c_void_p, C.c_float, C.c_float]),
        "ocpu_rng_normal": (C.c_float, [C.c_void_p]),
        "ocpu_rng_below": (C.c_uint64, [C.c_void_p, C.c_uint64]),
        "ocpu_rng_fill_normal": (None, [C.c_void_p, F32P, C.c_size_t]),
        "ocpu_rng_fill_range": (None, [C.c_void_p, F32P, C.c_size_t, C.c_float, C.c_float]),
        "ocpu_rng_fill_below": (None, [C.c_void_p, U32P, C.c_size_t, C.c_uint64]),
        "ocpu_powi": (C.c_float, [C.c_float, C.c_int]),
        "ocpu_matmul": (C.c_int, [F32P, F32P, F32P, C.c_size_t, C.c_size_t, C.c_size_t]),
        "ocpu_transpose": (C.c_int, [F32P, F32P, C.c_size_t, C.c_size_t]),
        "ocpu_softmax_rows": (C.c_int, [F32P, F32P, C.c_size_t, C.c_size_t]),
        "ocpu_reduce_to": (C.c_int, [F32P, C.c_size_t, C.c_size_t, C.c_size_t, C.c_size_t, F32P]),
        "ocpu_argmax_rows": (C.c_int, [F32P, C.c_size_t, C.c_size_t, U32P]),
        "ocpu_accuracy": (C.c_float, [F32P, C.c_size_t, C.c_size_t, U32P]),
        "ocpu_one_hot": (C.c_int, [U32P, C.c_size_t, C.c_size_t, F32P]),
        "ocpu_param_new": (C.c_int64, [SZP, C.c_int, F32P]),
        "ocpu_param_get": (C.c_int, [C.c_int64, F32P]),
        "ocpu_param_set": (C.c_int, [C.c_int64, F32P]),
        "ocpu_param_len": (C.c_int64, [C.c_int64]),
        "ocpu_param_free": (None, [C.c_int64]),
        "ocpu_dense_new": (C.c_int, [C.c_size_t, C.c_size_t, C.c_void_p, I64P, I64P]),
        "ocpu_tape_new": (C.c_void_p, []),
        "ocpu_tape_free": (None, [C.c_void_p]),
        "ocpu_var_constant": (C.c_int64, [C.c_void_p, SZP, C.c_int, F32P]),
        "ocpu_var_watch": (C.c_int64, [C.c_void_p, C.c_int64]),
        "ocpu_var_unary": (C.c_int64, [C.c_void_p, C.c_int, C.c_int64, C.c_float]),
        "ocpu_var_binary": (C.c_int64, [C.c_void_p, C.c_int, C.c_int64, C.c_int64]),
        "ocpu_var_loss": (C.c_int64, [C.c_void_p, C.c_int, C.c_int64, SZP, C.c_int, F32P]),
        "ocpu_var_shape": (C.c_int, [C.c_void_p, C.c_int64, SZP, C.POINTER(C.c_int)]),
        "ocpu_var_value": (C.c_int, [C.c_void_p, C.c_int64, F32P]),
        "ocpu_backward": (C.c_int, [C.c_void_p, C.c_int64]),
        "ocpu_grad_of_param": (C.c_int, [C.c_void_p, C.c_int64, F32P]),
        "ocpu_opt_new": (C.c_void_p, [C.c_int, C.c_float, C.c_float, C.c_float]),
        "ocpu_opt_free": (None, [C.c_void_p]),
        "ocpu_opt_step": (C.c_int, [C.c_void_p, C.c_void_p, I64P, C.c_size_t]),
        "ocpu_mlp_new": (C.c_void_p, [C.c_int, SZP, C.POINTER(C.c_int), C.POINTER(F32P), C.POINTER(F32P)]),
        "ocpu_mlp_free": (None, [C.c_void_p]),
        "ocpu_mlp_set_optimizer": (C.c_int, [C.c_void_p, C.c_int, C.c_float, C.c_float, C.c_float]),
        "ocpu_mlp_step": (C.c_int, [C.c_void_p, F32P, C.c_size_t, U32P, F32P]),
        "ocpu_mlp_forward": (C.c_int, [C.c_void_p, F32P, C.c_size_t, F32P]),
        "ocpu_mlp_get": (C.c_int, [C.c_void_p, C.c_int, C.c_int, F32P]),
        "ocpu_mlp_logits": (C.c_int, [C.c_void_p, F32P]),
        "ocpu_mlp_set": (C.c_int, [C.c_void_p, C.c_int, C.c_int, F32P]),
        "ocpu_mlp_get_t": (C.c_int, [C.c_void_p]),
        "ocpu_mlp_set_t": (None, [C.c_void_p, C.c_int]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _check(rc: int) -> None:
    if rc < 0:
        raise RuntimeError("oracle: " + lib().ocpu_last_error().decode())


def set_threads(n: int) -> None:
    """Row-parallel matmul threads; results are bit-identical for any count."""
    lib().ocpu_set_threads(int(n))


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


# ------------------------------------------------------------------ Rng
class Rng:
    """rtensor ``Rng`` (src/rng.rs:3-49)."""

    def __init__(self, seed: int):
        self._h = lib().ocpu_rng_new(C.c_uint64(seed))

    def __del__(self):
        if getattr(self, "_h", None) and _lib is not None:
            _lib.ocpu_rng_free(self._h)
            self._h = None

    def next_u64(self) -> int:
        return lib().ocpu_rng_next_u64(self._h)

    def uniform(self) -> float:
        return lib().ocpu_rng_uniform(self._h)

    def range(self, lo: float, hi: float) -> float:
        return lib().ocpu_rng_range(self._h, lo, hi)

    def normal(self) -> float:
        return lib().ocpu_rng_normal(self._h)

    def below(self, n: int) -> int:
        return lib().ocpu_rng_below(self._h, n)

    def normals(self, n: int) -> np.ndarray:
        out = np.empty(n, np.float32)
        lib().ocpu_rng_fill_normal(self._h, _p(out), n)
        return out

    def ranges(self, n: int, lo: float, hi: float) -> np.ndarray:
        out = np.empty(n, np.float32)
        lib().ocpu_rng_fill_range(self._h, _p(out), n, lo, hi)
        return out

    def belows(self, n: int, c: int) -> np.ndarray:
        out = np.empty(n, np.uint32)
        lib().ocpu_rng_fill_below(self._h, _p(out, U32P), n, c)
        return out


def powi(a: float, b: int) -> float:
    return lib().ocpu_powi(a, b)


# ------------------------------------------------------------------ tensor kernels
def matmul(a, b) -> np.ndarray:
    """``Tensor::matmul`` (tensor.rs:318-373), bit-faithful summation order."""
    a, b = f32(a), f32(b)
    m, k = a.shape
    k2, n = b.shape
    assert k == k2
    out = np.empty((m, n), np.float32)
    _check(lib().ocpu_matmul(_p(a), _p(b), _p(out), m, k, n))
    return out


def transpose(a) -> np.ndarray:
    a = f32(a)
    r, c = a.shape
    out = np.empty((c, r), np.float32)
    _check(lib().ocpu_transpose(_p(a), _p(out), r, c))
    return out


def softmax_rows(z) -> np.ndarray:
    z = f32(z)
    out = np.empty_like(z)
    _check(lib().ocpu_softmax_rows(_p(z), _p(out), z.shape[0], z.shape[1]))
    return out


def reduce_to(g, target) -> np.ndarray:
    g = f32(g)
    t0, t1 = target
    out = np.empty(t0 * t1, np.float32)
    _check(lib().ocpu_reduce_to(_p(g), g.shape[0], g.shape[1], t0, t1, _p(out)))
    return out.reshape(t0, t1)


def argmax_rows(z) -> np.ndarray:
    z = f32(z)
    out = np.empty(z.shape[0], np.uint32)
    _check(lib().ocpu_argmax_rows(_p(z), z.shape[0], z.shape[1], _p(out, U32P)))
    return out


def accuracy(z, labels) -> float:
    z = f32(z)
    lab = np.ascontiguousarray(labels, dtype=np.uint32)
    return lib().ocpu_accuracy(_p(z), z.shape[0], z.shape[1], _p(lab, U32P))


def one_hot(labels, classes: int) -> np.ndarray:
    lab = np.ascontiguousarray(labels, dtype=np.uint32)
    out = np.empty((lab.size, classes), np.float32)
    _check(lib().ocpu_one_hot(_p(lab, U32P), lab.size, classes, _p(out)))
    return out


# ------------------------------------------------------------------ params, tape
class Param:
    """rtensor ``Param`` (tape.rs:76-132): shared, updated in place by optimizers."""

    def __init__(self, value=None, _pid: Optional[int] = None, shape=None):
        if _pid is None:
            v = f32(value)
            shp = (C.c_size_t * max(v.ndim, 1))(*v.shape)
            _pid = lib().ocpu_param_new(shp, v.ndim, _p(v))
            _check(_pid)
            shape = v.shape
        self.pid = _pid
        self.shape = tuple(shape)

    def value(self) -> np.ndarray:
        out = np.empty(self.shape, np.float32)
        _check(lib().ocpu_param_get(self.pid, _p(out)))
        return out

    def set(self, v) -> None:
        v = f32(v).reshape(self.shape)
        _check(lib().ocpu_param_set(self.pid, _p(v)))


UNARY = {"scale": 0, "offset": 1, "neg": 2, "square": 3, "sqrt": 4, "exp": 5, "ln": 6, "relu": 7,
         "leaky_relu": 8, "sigmoid": 9, "tanh": 10, "sum": 11, "mean": 12, "softmax": 13}
BINARY = {"add": 0, "sub": 1, "mul": 2, "div": 3, "matmul": 4}
LOSS = {"mse": 0, "mae": 1, "softmax_cross_entropy": 2, "binary_cross_entropy": 3}
ACT = {"linear": 0, "relu": 1, "leaky_relu": 2, "sigmoid": 3, "tanh": 4}


class Tape:
    """rtensor ``Tape`` (tape.rs:43-229) driven op by op."""

    def __init__(self):
        self._h = lib().ocpu_tape_new()

    def __del__(self):
        if getattr(self, "_h", None) and _lib is not None:
            _lib.ocpu_tape_free(self._h)
            self._h = None

    def constant(self, v) -> "Var":
        v = f32(v)
        shp = (C.c_size_t * max(v.ndim, 1))(*v.shape)
        idx = lib().ocpu_var_constant(self._h, shp, v.ndim, _p(v))
        _check(idx)
        return Var(self, idx)

    def watch(self, p: Param) -> "Var":
        idx = lib().ocpu_var_watch(self._h, p.pid)
        _check(idx)
        return Var(self, idx)

    def grad(self, p: Param) -> Optional[np.ndarray]:
        out = np.empty(p.shape, np.float32)
        rc = lib().ocpu_grad_of_param(self._h, p.pid, _p(out))
        _check(rc)
        return out if rc == 1 else None


class Var:
    def __init__(self, tape: Tape, idx: int):
        self.tape, self.idx = tape, idx

    def shape(self):
        shp = (C.c_size_t * 8)()
        r = C.c_int()
        _check(lib().ocpu_var_shape(self.tape._h, self.idx, shp, C.byref(r)))
        return tuple(shp[i] for i in range(r.value))

    def value(self) -> np.ndarray:
        out = np.empty(self.shape(), np.float32)
        _check(lib().ocpu_var_value(self.tape._h, self.idx, _p(out)))
        return out

    def item(self) -> float:
        return float(self.value().reshape(-1)[0])

    def _u(self, op: str, k: float = 0.0) -> "Var":
        idx = lib().ocpu_var_unary(self.tape._h, UNARY[op], self.idx, k)
        _check(idx)
        return Var(self.tape, idx)

    def _b(self, op: str, other: "Var") -> "Var":
        idx = lib().ocpu_var_binary(self.tape._h, BINARY[op], self.idx, other.idx)
        _check(idx)
        return Var(self.tape, idx)

    def __getattr__(self, name):
        if name in UNARY:
            return lambda k=0.0: self._u(name, k)
        if name in BINARY:
            return lambda other: self._b(name, other)
        raise AttributeError(name)

    def backward(self) -> None:
        _check(lib().ocpu_backward(self.tape._h, self.idx))


def loss(kind: str, pred: Var, target) -> Var:
    t = f32(target)
    shp = (C.c_size_t * max(t.ndim, 1))(*t.shape)
    idx = lib().ocpu_var_loss(pred.tape._h, LOSS[kind], pred.idx, shp, t.ndim, _p(t))
    _check(idx)
    return Var(pred.tape, idx)


class Optimizer:
    """``Sgd`` (kind 1: lr, momentum) or ``Adam`` (kind 2: lr, β1, β2) from optim.rs."""

    def __init__(self, kind: str, lr: float, a: float = 0.0, b: float = 0.0):
        k = {"sgd": 1, "adam": 2}[kind]
        if kind == "adam" and a == 0.0:
            a, b = 0.9, 0.999
        self._h = lib().ocpu_opt_new(k, lr, a, b)

    def __del__(self):
        if getattr(self, "_h", None) and _lib is not None:
            _lib.ocpu_opt_free(self._h)
            self._h = None

    def step(self, params: Sequence[Param], tape: Tape) -> None:
        ids = np.array([p.pid for p in params], np.int64)
        _check(lib().ocpu_opt_step(self._h, tape._h, _p(ids, I64P), len(ids)))


class Dense:
    """``Dense`` (nn.rs:108-159) with Glorot init drawn from an ``Rng``."""

    def __init__(self, inputs: int, units: int, activation: str, rng: Rng):
        w, b = C.c_int64(), C.c_int64()
        _check(lib().ocpu_dense_new(inputs, units, rng._h, C.byref(w), C.byref(b)))
        self.w = Param(_pid=w.value, shape=(inputs, units))
        self.b = Param(_pid=b.value, shape=(1, units))
        self.activation = activation

    def forward(self, x: Var) -> Var:
        t = x.tape
        z = x.matmul(t.watch(self.w)).add(t.watch(self.b))
        a = self.activation
        return z if a == "linear" else getattr(z, a)()

    def params(self) -> List[Param]:
        return [self.w, self.b]


class Sequential:
    def __init__(self, layers: Sequence[Dense]):
        self.layers = list(layers)

    def forward(self, x: Var) -> Var:
        for l in self.layers:
            x = l.forward(x)
        return x

    def params(self) -> List[Param]:
        return [p for l in self.layers for p in l.params()]

    def predict(self, x) -> np.ndarray:
        t = Tape()
        return self.forward(t.constant(x)).value()


# ------------------------------------------------------------------ MLP step
class CpuMlp:
    """A Sequential of Dense layers trained with softmax cross-entropy.

    ``step`` is one CPU training step exactly as tests/gpu.rs:116-121 runs it:
    tape forward, ``softmax_cross_entropy`` on one-hot labels, backward,
    ``Optimizer::step``.
    """

    def __init__(self, weights: Sequence[np.ndarray], biases: Sequence[np.ndarray],
                 activations: Optional[Sequence[str]] = None):
        n = len(weights)
        dims = [weights[0].shape[0]] + [w.shape[1] for w in weights]
        if activations is None:
            activations = ["relu"] * (n - 1) + ["linear"]
        self.dims = dims
        self._w = [f32(w) for w in weights]
        self._b = [f32(b).reshape(1, -1) for b in biases]
        wp = (F32P * n)(*[_p(w) for w in self._w])
        bp = (F32P * n)(*[_p(b) for b in self._b])
        d = (C.c_size_t * (n + 1))(*dims)
        a = (C.c_int * n)(*[ACT[x] for x in activations])
        self._h = lib().ocpu_mlp_new(n, d, a, wp, bp)
        if not self._h:
            _check(-1)
        self.n_layers = n

    def __del__(self):
        if getattr(self, "_h", None) and _lib is not None:
            _lib.ocpu_mlp_free(self._h)
            self._h = None

    def set_optimizer(self, kind: str, lr: float, a: float = 0.0, b: float = 0.0) -> None:
        k = {"none": 0, "sgd": 1, "adam": 2}[kind]
        if kind == "adam" and a == 0.0:
            a, b = 0.9, 0.999
        lib().ocpu_mlp_set_optimizer(self._h, k, lr, a, b)

    def step(self, x, labels) -> float:
        x = f32(x)
        lab = np.ascontiguousarray(labels, dtype=np.uint32)
        out = C.c_float()
        _check(lib().ocpu_mlp_step(self._h, _p(x), x.shape[0], _p(lab, U32P), C.byref(out)))
        return out.value

    def forward(self, x) -> np.ndarray:
        x = f32(x)
        out = np.empty((x.shape[0], self.dims[-1]), np.float32)
        _check(lib().ocpu_mlp_forward(self._h, _p(x), x.shape[0], _p(out)))
        return out

    def _shape(self, idx: int):
        l = idx // 2
        return (self.dims[l], self.dims[l + 1]) if idx % 2 == 0 else (1, self.dims[l + 1])

    def weights(self) -> List[np.ndarray]:
        out = []
        for i in range(2 * self.n_layers):
            a = np.empty(self._shape(i), np.float32)
            _check(lib().ocpu_mlp_get(self._h, 0, i, _p(a)))
            out.append(a)
        return out

    def grads(self) -> List[np.ndarray]:
        return self._get_all(1)

    def _get_all(self, which: int) -> List[np.ndarray]:
        out = []
        for i in range(2 * self.n_layers):
            a = np.empty(self._shape(i), np.float32)
            _check(lib().ocpu_mlp_get(self._h, which, i, _p(a)))
            out.append(a)
        return out

    def _set_all(self, which: int, arrays) -> None:
        assert len(arrays) == 2 * self.n_layers
        for i, a in enumerate(arrays):
            a = f32(a).reshape(self._shape(i))
            _check(lib().ocpu_mlp_set(self._h, which, i, _p(a)))

    def set_weights(self, arrays) -> None:
        """``Param::set`` (tape.rs:119-121) on every parameter, [W1, b1, ...]."""
        self._set_all(0, arrays)

    def optimizer_state(self):
        """The optimizer's state after the steps so far: (m, v, t) for Adam
        (optim.rs:143-149, 163), (velocity, [], 0) for Sgd.  Parameters not
        updated yet read as zeros."""
        return self._get_all(2), self._get_all(3), int(lib().ocpu_mlp_get_t(self._h))

    def set_optimizer_state(self, m, v, t: int) -> None:
        self._set_all(2, m)
        if v is not None:
            self._set_all(3, v)
        lib().ocpu_mlp_set_t(self._h, int(t))


# ------------------------------------------------------------------ data helpers
def erro_rel(a, b) -> float:
    """tests/gpu.rs:53-60: max |x-y| / (1 + max(|x|,|y|)), the parity metric."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    assert a.shape == b.shape, (a.shape, b.shape)
    if a.size == 0:
        return 0.0
    return float(np.max(np.abs(a - b) / (1.0 + np.maximum(np.abs(a), np.abs(b)))))


def kaiming_uniform(rng: Rng, fan_in: int, fan_out: int) -> np.ndarray:
    """Kaiming-uniform W [fan_in, fan_out]: U(-√(6/fan_in), √(6/fan_in)) drawn
    row-major with ``Rng::range``."""
    bound = float(np.sqrt(np.float32(6.0) / np.float32(fan_in), dtype=np.float32))
    return rng.ranges(fan_in * fan_out, -bound, bound).reshape(fan_in, fan_out)
