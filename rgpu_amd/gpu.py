"""Host-side mirror of ``rtensor::gpu`` over the C ABI of librtensor_hip.so.

Names follow the reference API (crates/rtensor/src/gpu/mod.rs):

=======================  =============================================  ===============
rtensor::gpu             here                                           mod.rs
=======================  =============================================  ===============
Gpu::new                 Gpu()                                          263-277
Gpu::info                Gpu.info()                                     412
Gpu::zeros / upload      Gpu.zeros(shape) / Gpu.upload(array)           501-517
Gpu::download            Gpu.download(t) -> numpy (blocking)            530-544
Gpu::sync                Gpu.sync()                                     564-566
op_matmul(_at_b/_a_bt)   Gpu.matmul / matmul_at_b / matmul_a_bt         685-700
op_matmul_bias           Gpu.matmul_bias(a, w, c, bias, relu)           722-749
op_matmul_f16            Gpu.matmul(...) on bf16/f16 tensors            1191-1229
ops_split_k              Gpu.split_k(a, b, c, partials, slices, trans)  1095-1146
fatias_sugeridas         Gpu.fatias_sugeridas(m, n, k)                  1079-1088
ops_colsum               Gpu.colsum(src, dst)                           838-855
op_bias_add / relu(_bwd) Gpu.bias_add / relu / relu_bwd                 752-788
op_softmax_xent          Gpu.softmax_xent(logits, labels, delta, loss)  791-808
op_adam (+atualizar)     Gpu.adam(theta, m, v, g, lr, betas, t)         859-907
upload_labels            upload_labels(gpu, labels)                     1672-1675
GpuMlp                   GpuMlp.from_params(gpu, params, lote, lr, ...)  1322-1562
=======================  =============================================  ===============

Misuse that panics in the reference raises ``RtError`` here, carrying the
rt_status code.  There is no CPU fallback: if librtensor_hip.so is missing or
no gfx950 device is present, construction fails loudly.
"""
from __future__ import annotations

import ctypes as C
import math
import os
from typing import List, Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "librtensor_hip.so")

F32, BF16, F16, U32 = 0, 1, 2, 3
NN, TN, NT = 0, 1, 2
EPI_NONE, EPI_BIAS, EPI_BIAS_RELU, EPI_RELU_MASK = 0, 1, 2, 3
OPT_ADAM, OPT_SGD = 0, 1
PREC_F32, PREC_BF16 = 0, 1
# rt_unary_op, rt_binary_op, rt_loss_kind
UNARY = {"scale": 0, "offset": 1, "neg": 2, "square": 3, "sqrt": 4, "exp": 5, "ln": 6, "relu": 7,
         "leaky_relu": 8, "sigmoid": 9, "tanh": 10}
BINARY = {"add": 0, "sub": 1, "mul": 2, "div": 3}
LOSS_MAE, LOSS_SOFTMAX_XENT, LOSS_BCE, LOSS_SOFTMAX_XENT_LOGITS, LOSS_SOFTMAX_XENT_LOGITS_MEAN = 1, 2, 3, 4, 5

STATUS = {0: "RT_OK", 1: "RT_ERR_NO_DEVICE", 2: "RT_ERR_INVALID", 3: "RT_ERR_SHAPE", 4: "RT_ERR_DTYPE",
          5: "RT_ERR_OOM", 6: "RT_ERR_LABEL", 7: "RT_ERR_HIP", 8: "RT_ERR_OVERFLOW"}

# Every symbol include/rtensor_hip.h declares, with its ctypes signature.
_VP = C.c_void_p
_SZP = C.POINTER(C.c_size_t)
SIGNATURES = {
    "rt_open": (C.c_int, [C.c_int, C.POINTER(_VP)]),
    "rt_close": (C.c_int, [_VP]),
    "rt_last_error": (C.c_char_p, [_VP]),
    "rt_info": (C.c_int, [_VP, C.c_char_p, C.c_size_t]),
    "rt_sync": (C.c_int, [_VP]),
    "rt_zeros": (C.c_int, [_VP, C.c_int, _SZP, C.c_int, C.POINTER(_VP)]),
    "rt_upload": (C.c_int, [_VP, C.c_int, _SZP, C.c_int, _VP, C.POINTER(_VP)]),
    "rt_download": (C.c_int, [_VP, _VP, _VP, C.c_size_t]),
    "rt_write": (C.c_int, [_VP, _VP, _VP, C.c_size_t]),
    "rt_free": (C.c_int, [_VP, _VP]),
    "rt_buf_info": (C.c_int, [_VP, C.POINTER(C.c_int), _SZP, C.POINTER(C.c_int)]),
    "rt_upload_labels": (C.c_int, [_VP, C.POINTER(C.c_uint64), C.c_size_t, C.POINTER(_VP)]),
    "rt_convert": (C.c_int, [_VP, _VP, _VP]),
    "rt_gemm": (C.c_int, [_VP, C.c_int, _VP, _VP, _VP, C.c_int, _VP, _VP]),
    "rt_gemm_splitk": (C.c_int, [_VP, C.c_int, _VP, _VP, _VP, _VP, C.c_size_t, _VP]),
    "rt_gemm_splitk_static": (C.c_int, [_VP, C.c_int, _VP, _VP, _VP, C.c_size_t, _VP]),
    "rt_splitk_slices": (C.c_size_t, [C.c_size_t, C.c_size_t, C.c_size_t]),
    "rt_colsum": (C.c_int, [_VP, _VP, _VP]),
    "rt_bias_add": (C.c_int, [_VP, _VP, _VP]),
    "rt_relu": (C.c_int, [_VP, _VP, _VP]),
    "rt_relu_bwd": (C.c_int, [_VP, _VP, _VP]),
    "rt_softmax_xent": (C.c_int, [_VP, _VP, _VP, _VP, _VP, C.c_float]),
    "rt_adam": (C.c_int, [_VP, _VP, _VP, _VP, _VP, C.c_float, C.c_float, C.c_float, C.c_float, C.c_int]),
    "rt_sgd": (C.c_int, [_VP, _VP, _VP, _VP, C.c_float, C.c_float]),
    "rt_mlp_create": (C.c_int, [_VP, C.c_int, _SZP, C.POINTER(C.POINTER(C.c_float)),
                                C.POINTER(C.POINTER(C.c_float)), C.c_size_t, _VP, C.POINTER(_VP)]),
    "rt_mlp_destroy": (C.c_int, [_VP]),
    "rt_mlp_step": (C.c_int, [_VP, _VP, _VP]),
    "rt_mlp_forward": (C.c_int, [_VP, _VP]),
    "rt_mlp_logits": (C.c_int, [_VP, C.POINTER(C.c_float), C.c_size_t]),
    "rt_mlp_activation": (C.c_int, [_VP, C.c_int, C.POINTER(C.c_float), C.c_size_t]),
    "rt_mlp_delta": (C.c_int, [_VP, C.c_int, C.POINTER(C.c_float), C.c_size_t]),
    "rt_mlp_last_loss": (C.c_int, [_VP, C.POINTER(C.c_float)]),
    "rt_mlp_weights": (C.c_int, [_VP, C.POINTER(C.POINTER(C.c_float)), C.c_int]),
    "rt_mlp_grads": (C.c_int, [_VP, C.POINTER(C.POINTER(C.c_float)), C.c_int]),
    "rt_mlp_dispatches": (C.c_int, [_VP, C.POINTER(C.c_int)]),
    "rt_mlp_overflow": (C.c_int, [_VP, C.POINTER(C.c_int)]),
    "rt_profile_enable": (C.c_int, [_VP, C.c_int]),
    "rt_profile_reset": (C.c_int, [_VP]),
    "rt_profile_report": (C.c_int, [_VP, C.c_char_p, C.c_size_t, C.POINTER(C.c_int), C.POINTER(C.c_double),
                                    C.c_int, C.POINTER(C.c_int)]),
    "rt_timer_begin": (C.c_int, [_VP]),
    "rt_timer_end": (C.c_int, [_VP, C.POINTER(C.c_float)]),
    "rt_mlp_set_weights": (C.c_int, [_VP, C.POINTER(C.POINTER(C.c_float)), C.c_int]),
    "rt_mlp_get_optimizer_state": (C.c_int, [_VP, C.POINTER(C.POINTER(C.c_float)), C.POINTER(C.POINTER(C.c_float)),
                                             C.c_int, C.POINTER(C.c_int)]),
    "rt_mlp_set_optimizer_state": (C.c_int, [_VP, C.POINTER(C.POINTER(C.c_float)), C.POINTER(C.POINTER(C.c_float)),
                                             C.c_int, C.c_int]),
    "rt_argmax_rows": (C.c_int, [_VP, _VP, _VP]),
    "rt_accuracy": (C.c_int, [_VP, _VP, _VP, C.POINTER(C.c_float)]),
    "rt_map": (C.c_int, [_VP, C.c_int, C.c_float, _VP, _VP]),
    "rt_map_vjp": (C.c_int, [_VP, C.c_int, C.c_float, _VP, _VP, _VP, _VP]),
    "rt_zip": (C.c_int, [_VP, C.c_int, _VP, _VP, _VP]),
    "rt_reduce_to": (C.c_int, [_VP, _VP, _VP]),
    "rt_sum_all": (C.c_int, [_VP, _VP, C.c_float, _VP]),
    "rt_fill_scaled": (C.c_int, [_VP, _VP, C.c_float, _VP, _VP]),
    "rt_softmax_rows": (C.c_int, [_VP, _VP, _VP]),
    "rt_softmax_rows_vjp": (C.c_int, [_VP, _VP, _VP, _VP]),
    "rt_loss": (C.c_int, [_VP, C.c_int, _VP, _VP, _VP, _VP]),
    "rt_empty": (C.c_int, [_VP, C.c_int, _SZP, C.c_int, C.POINTER(_VP)]),
    "rt_adam_many": (C.c_int, [_VP, C.c_int, C.POINTER(_VP), C.POINTER(_VP), C.POINTER(_VP), C.POINTER(_VP),
                               C.c_float, C.c_float, C.c_float, C.c_float, C.c_int]),
    "rt_linear_backward": (C.c_int, [_VP, _VP, _VP, _VP, _VP, _VP, _VP]),
    "rt_mlp_load": (C.c_int, [_VP, _VP, C.c_size_t, C.POINTER(C.c_uint64), C.c_size_t]),
    "rt_mlp_step_loaded": (C.c_int, [_VP]),
    "rt_sgd_many": (C.c_int, [_VP, C.c_int, C.POINTER(_VP), C.POINTER(_VP), C.POINTER(_VP), C.c_float, C.c_float]),
}


class RtMlpConfig(C.Structure):
    """``rt_mlp_config`` from include/rtensor_hip.h."""
    _fields_ = [("optimizer", C.c_int), ("lr", C.c_float), ("beta1", C.c_float), ("beta2", C.c_float),
                ("eps", C.c_float), ("momentum", C.c_float), ("precision", C.c_int), ("loss_scale", C.c_float)]


_lib: Optional[C.CDLL] = None


def lib() -> C.CDLL:
    """Load librtensor_hip.so; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m rgpu_amd.build`")
    L = C.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


class RtError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{STATUS.get(code, code)}: {msg}")
        self.code = code
        self.status = STATUS.get(code, str(code))


def _np_dtype(dt: int):
    return {F32: np.float32, BF16: np.uint16, F16: np.float16, U32: np.uint32}[dt]


_ITEMSIZE = {F32: 4, BF16: 2, F16: 2, U32: 4}


def _shape(shape) -> tuple:
    """A shape as a tuple of Python ints (the common case passes through)."""
    if type(shape) is tuple and all(type(d) is int for d in shape):
        return shape
    return tuple(int(d) for d in shape)


def f32_to_bf16_bits(a) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16, returned as uint16 bit patterns."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(b) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


class GpuTensor:
    """``GpuTensor`` (mod.rs:190-208): owns one device buffer."""

    def __init__(self, gpu: "Gpu", handle: int, shape, dtype: int):
        self.gpu = gpu
        self.handle = handle
        self.shape = _shape(shape)
        self.dtype = dtype

    def __len__(self):
        return math.prod(self.shape)

    @property
    def len(self) -> int:
        return len(self)

    def free(self):
        if self.handle and self.gpu._h and not self.gpu._keep(self):
            self.gpu._call("rt_free", self.gpu._h, self.handle)
        self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Gpu:
    """``rtensor::gpu::Gpu`` (mod.rs:224-1237): one device, one HIP stream."""

    def __init__(self, device: int = 0):
        L = lib()
        h = C.c_void_p()
        rc = L.rt_open(device, C.byref(h))
        if rc != 0:
            raise RtError(rc, L.rt_last_error(None).decode())
        self._h = h.value
        # Freed buffers kept for the next ``empty`` of the same shape and dtype
        # (an op-level tape allocates and drops the same shapes every step):
        # no call into the library either way.  Reuse is safe for the same
        # reason as the library's own cache: the context's work runs in order
        # on its one stream.
        self._spare = {}

    _SPARE_PER_SHAPE = 8
    _SPARE_MAX_BYTES = 64 << 20

    def _keep(self, t: "GpuTensor") -> bool:
        if len(t) * _ITEMSIZE[t.dtype] > self._SPARE_MAX_BYTES:
            return False
        lst = self._spare.setdefault((t.shape, t.dtype), [])
        if len(lst) >= self._SPARE_PER_SHAPE:
            return False
        lst.append(t.handle)
        return True

    def close(self):
        if self._h:
            self._spare = {}  # the context frees every buffer it still owns
            lib().rt_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _call(self, name: str, *args) -> int:
        rc = getattr(lib(), name)(*args)
        if rc != 0:
            raise RtError(rc, lib().rt_last_error(self._h).decode())
        return rc

    # --------------------------------------------------------------- device
    def info(self) -> str:
        buf = C.create_string_buffer(256)
        self._call("rt_info", self._h, buf, 256)
        return buf.value.decode()

    def sync(self) -> None:
        self._call("rt_sync", self._h)

    # --------------------------------------------------------------- buffers
    def zeros(self, shape, dtype: int = F32) -> GpuTensor:
        shape = _shape(shape)
        arr = (C.c_size_t * max(len(shape), 1))(*shape)
        h = C.c_void_p()
        self._call("rt_zeros", self._h, dtype, arr, len(shape), C.byref(h))
        return GpuTensor(self, h.value, shape, dtype)

    def empty(self, shape, dtype: int = F32) -> GpuTensor:
        """A buffer whose contents are undefined, for outputs written whole."""
        shape = _shape(shape)
        lst = self._spare.get((shape, dtype))
        if lst:
            return GpuTensor(self, lst.pop(), shape, dtype)
        arr = (C.c_size_t * max(len(shape), 1))(*shape)
        h = C.c_void_p()
        self._call("rt_empty", self._h, dtype, arr, len(shape), C.byref(h))
        return GpuTensor(self, h.value, shape, dtype)

    def upload(self, a, dtype: Optional[int] = None) -> GpuTensor:
        """Upload a host array.  dtype BF16 takes f32 values (rounded to
        nearest even) or uint16 bit patterns; F16 takes anything numpy can
        cast to float16."""
        a = np.asarray(a)
        if dtype is None:
            dtype = {np.dtype(np.float32): F32, np.dtype(np.float16): F16, np.dtype(np.uint32): U32}.get(a.dtype, F32)
        if dtype == BF16:
            host = a if a.dtype == np.uint16 else f32_to_bf16_bits(a)
        else:
            host = a.astype(_np_dtype(dtype), copy=False)
        host = np.ascontiguousarray(host)
        shape = host.shape
        arr = (C.c_size_t * max(len(shape), 1))(*shape)
        h = C.c_void_p()
        self._call("rt_upload", self._h, dtype, arr, len(shape), host.ctypes.data_as(C.c_void_p), C.byref(h))
        return GpuTensor(self, h.value, shape, dtype)

    def download(self, t: GpuTensor) -> np.ndarray:
        out = np.empty(t.shape, _np_dtype(t.dtype))
        self._call("rt_download", self._h, t.handle, out.ctypes.data_as(C.c_void_p), out.nbytes)
        return out

    def download_f32(self, t: GpuTensor) -> np.ndarray:
        a = self.download(t)
        if t.dtype == BF16:
            return bf16_bits_to_f32(a)
        return a.astype(np.float32)

    def write(self, t: GpuTensor, a) -> None:
        host = np.ascontiguousarray(a, dtype=_np_dtype(t.dtype))
        self._call("rt_write", self._h, t.handle, host.ctypes.data_as(C.c_void_p), host.nbytes)

    def convert(self, src: GpuTensor, dst: GpuTensor) -> None:
        self._call("rt_convert", self._h, src.handle, dst.handle)

    # --------------------------------------------------------------- ops
    def gemm(self, layout: int, a: GpuTensor, b: GpuTensor, c: GpuTensor, epi: int = EPI_NONE,
             aux: Optional[GpuTensor] = None, colsum: Optional[GpuTensor] = None) -> None:
        self._call("rt_gemm", self._h, layout, a.handle, b.handle, c.handle, epi,
                   aux.handle if aux else None, colsum.handle if colsum else None)

    def matmul(self, a, b, c):
        """C = A·B (op_matmul, mod.rs:685-688)."""
        self.gemm(NN, a, b, c)

    def matmul_at_b(self, a, b, c, colsum: Optional[GpuTensor] = None):
        """C = Aᵀ·B with A stored [k, m] (op_matmul_at_b, mod.rs:691-694)."""
        self.gemm(TN, a, b, c, colsum=colsum)

    def matmul_a_bt(self, a, b, c, relu_mask_from: Optional[GpuTensor] = None):
        """C = A·Bᵀ with B stored [n, k] (op_matmul_a_bt, mod.rs:697-700),
        optionally masked by 1[mask > 0] (fused op_relu_bwd)."""
        if relu_mask_from is None:
            self.gemm(NT, a, b, c)
        else:
            self.gemm(NT, a, b, c, EPI_RELU_MASK, relu_mask_from)

    def matmul_bias(self, a, w, c, bias, relu: bool):
        """C = X·W + 1ₙb, ReLU optional (op_matmul_bias, mod.rs:722-749)."""
        self.gemm(NN, a, w, c, EPI_BIAS_RELU if relu else EPI_BIAS, bias)

    @staticmethod
    def fatias_sugeridas(m: int, n: int, k: int) -> int:
        return int(lib().rt_splitk_slices(m, n, k))

    def split_k(self, a, b, c, partials, slices: int, transposta: bool, colsum: Optional[GpuTensor] = None):
        """ops_split_k (mod.rs:1095-1146)."""
        self._call("rt_gemm_splitk", self._h, TN if transposta else NN, a.handle, b.handle, c.handle,
                   partials.handle, slices, colsum.handle if colsum else None)

    def split_k_static(self, a, b, c, slices: int, transposta: bool, colsum: Optional[GpuTensor] = None):
        """split_k with its partial planes in the library's static device
        array: allocates nothing (rt_gemm_splitk_static)."""
        self._call("rt_gemm_splitk_static", self._h, TN if transposta else NN, a.handle, b.handle, c.handle, slices,
                   colsum.handle if colsum else None)

    def linear_backward(self, x, delta, w, dx, dw, db=None):
        """dW = Xᵀδ, db = 1ᵀδ, dX = δWᵀ of a Linear layer (one launch when the
        paired kernel takes the shapes)."""
        self._call("rt_linear_backward", self._h, x.handle, delta.handle, w.handle,
                   dx.handle if dx is not None else None, dw.handle, db.handle if db is not None else None)

    def colsum(self, src, dst):
        self._call("rt_colsum", self._h, src.handle, dst.handle)

    def bias_add(self, z, b):
        self._call("rt_bias_add", self._h, z.handle, b.handle)

    def relu(self, x, y):
        self._call("rt_relu", self._h, x.handle, y.handle)

    def relu_bwd(self, a, delta):
        self._call("rt_relu_bwd", self._h, a.handle, delta.handle)

    def softmax_xent(self, logits, labels, delta, loss_rows, scale: float = 1.0):
        self._call("rt_softmax_xent", self._h, logits.handle, labels.handle, delta.handle, loss_rows.handle, scale)

    def adam(self, theta, m, v, g, lr: float, betas=(0.9, 0.999), t: int = 1, eps: float = 1e-8):
        self._call("rt_adam", self._h, theta.handle, m.handle, v.handle, g.handle, lr, betas[0], betas[1], eps, t)

    def sgd(self, theta, g, lr: float, momentum: float = 0.0, velocity: Optional[GpuTensor] = None):
        self._call("rt_sgd", self._h, theta.handle, velocity.handle if velocity else None, g.handle, lr, momentum)

    @staticmethod
    def _handles(ts):
        return (C.c_void_p * max(len(ts), 1))(*[t.handle if t is not None else None for t in ts])

    def adam_many(self, thetas, ms, vs, gs, lr: float, betas=(0.9, 0.999), t: int = 1, eps: float = 1e-8):
        """Adam::step over a parameter list (optim.rs:162-198) in one launch per 24 tensors."""
        self._call("rt_adam_many", self._h, len(thetas), self._handles(thetas), self._handles(ms),
                   self._handles(vs), self._handles(gs), lr, betas[0], betas[1], eps, t)

    def sgd_many(self, thetas, gs, lr: float, momentum: float = 0.0, velocities=None):
        """Sgd::step over a parameter list (optim.rs:80-114)."""
        self._call("rt_sgd_many", self._h, len(thetas), self._handles(thetas),
                   self._handles(velocities) if velocities is not None else None, self._handles(gs), lr, momentum)

    def argmax_rows(self, logits, out):
        """Tensor::argmax_rows (tensor.rs:476-493) into a u32 [B] device buffer."""
        self._call("rt_argmax_rows", self._h, logits.handle, out.handle)

    def accuracy(self, logits, labels) -> float:
        """losses::accuracy (losses.rs:181-185) of device logits against u32 labels."""
        v = C.c_float()
        self._call("rt_accuracy", self._h, logits.handle, labels.handle, C.byref(v))
        return v.value

    # --------------------------------------------------------------- tensor ops
    def map(self, op: str, x, y, k: float = 0.0):
        """Tensor::map with the forward closure of ops.rs's ``op`` (y = f(x))."""
        self._call("rt_map", self._h, UNARY[op], k, x.handle, y.handle)

    def map_vjp(self, op: str, g, x, y, dx, k: float = 0.0):
        """The VJP closure of ``op`` (ops.rs:132-227); x / y may be None when unused."""
        self._call("rt_map_vjp", self._h, UNARY[op], k, g.handle, x.handle if x is not None else None,
                   y.handle if y is not None else None, dx.handle)

    def zip(self, op: str, a, b, out):
        """Tensor::zip (tensor.rs:183-246) with broadcasting; op in add/sub/mul/div."""
        self._call("rt_zip", self._h, BINARY[op], a.handle, b.handle, out.handle)

    def reduce_to(self, g, out):
        """Tensor::reduce_to (tensor.rs:399-438) onto out's shape."""
        self._call("rt_reduce_to", self._h, g.handle, out.handle)

    def sum_all(self, x, out, div: float = 1.0):
        """out[0] = sum_all(x) / div (tensor.rs:279-286)."""
        self._call("rt_sum_all", self._h, x.handle, div, out.handle)

    def fill_scaled(self, s, out, div: float = 1.0, x=None):
        """out = x * (s / div), or Tensor::full(s / div) when x is None."""
        self._call("rt_fill_scaled", self._h, s.handle, div, x.handle if x is not None else None, out.handle)

    def softmax_rows(self, z, y):
        """Tensor::softmax_rows (tensor.rs:455-472)."""
        self._call("rt_softmax_rows", self._h, z.handle, y.handle)

    def softmax_rows_vjp(self, s, g, dx):
        """softmax's VJP (ops.rs:291-309): dx = s * (g - rowsum(g * s))."""
        self._call("rt_softmax_rows_vjp", self._h, s.handle, g.handle, dx.handle)

    def loss(self, kind: int, p, y, value, dir_=None):
        """Loss value (total / batch) and unscaled gradient direction (losses.rs)."""
        self._call("rt_loss", self._h, kind, p.handle, y.handle if y is not None else None, value.handle,
                   dir_.handle if dir_ is not None else None)

    # --------------------------------------------------------------- profiling
    def profile(self, on: bool) -> None:
        self._call("rt_profile_enable", self._h, 1 if on else 0)

    def profile_reset(self) -> None:
        self._call("rt_profile_reset", self._h)

    def timer_begin(self) -> None:
        """Start a region timer: a HIP event on the library stream."""
        self._call("rt_timer_begin", self._h)

    def timer_end(self) -> float:
        """Device milliseconds since timer_begin (blocks)."""
        ms = C.c_float()
        self._call("rt_timer_end", self._h, C.byref(ms))
        return ms.value

    def perfilar(self) -> List[tuple]:
        """Per-label (name, launches, device ms) since the last reset (Gpu::perfilar, mod.rs:1245-1286)."""
        cap, nl = 256, 64
        names = C.create_string_buffer(cap * nl)
        counts = (C.c_int * cap)()
        ms = (C.c_double * cap)()
        n = C.c_int()
        self._call("rt_profile_report", self._h, names, nl, counts, ms, cap, C.byref(n))
        out = []
        for i in range(n.value):
            nm = names.raw[i * nl:(i + 1) * nl].split(b"\0", 1)[0].decode()
            out.append((nm, counts[i], ms[i]))
        return out


def upload_labels(gpu: Gpu, labels) -> GpuTensor:
    """upload_labels (mod.rs:1672-1675): integer labels -> u32 device buffer."""
    lab = np.ascontiguousarray(np.asarray(labels).astype(np.uint64))
    h = C.c_void_p()
    gpu._call("rt_upload_labels", gpu._h, lab.ctypes.data_as(C.POINTER(C.c_uint64)), lab.size, C.byref(h))
    return GpuTensor(gpu, h.value, (lab.size,), U32)


class GpuMlp:
    """``GpuMlp`` (mod.rs:1322-1562): ReLU hidden layers, linear output,
    softmax cross-entropy, trained entirely on the device."""

    def __init__(self, gpu: Gpu, handle: int, dims: Sequence[int], batch: int, precision: str = "f32"):
        self.gpu = gpu
        self._h = handle
        self.dims = list(dims)
        self.lote = batch
        self.precision = precision

    @classmethod
    def from_params(cls, gpu: Gpu, params: Sequence[np.ndarray], lote: int, lr: float, optimizer: str = "adam",
                    betas=(0.9, 0.999), eps: float = 1e-8, momentum: float = 0.0, precision: str = "f32",
                    loss_scale: float = 1.0) -> "GpuMlp":
        """Build from host parameters in ``[W1, b1, W2, b2, ...]`` order (mod.rs:1341)."""
        if len(params) % 2 != 0 or not params:
            raise ValueError("expected (W, b) pairs")
        ws = [np.ascontiguousarray(params[i], dtype=np.float32) for i in range(0, len(params), 2)]
        bs = [np.ascontiguousarray(params[i], dtype=np.float32).reshape(-1) for i in range(1, len(params), 2)]
        n = len(ws)
        dims = [ws[0].shape[0]] + [w.shape[1] for w in ws]
        cfg = RtMlpConfig(OPT_ADAM if optimizer == "adam" else OPT_SGD, lr, betas[0], betas[1], eps, momentum,
                          PREC_BF16 if precision == "bf16" else PREC_F32, loss_scale)
        wp = (C.POINTER(C.c_float) * n)(*[w.ctypes.data_as(C.POINTER(C.c_float)) for w in ws])
        bp = (C.POINTER(C.c_float) * n)(*[b.ctypes.data_as(C.POINTER(C.c_float)) for b in bs])
        d = (C.c_size_t * (n + 1))(*dims)
        h = C.c_void_p()
        gpu._call("rt_mlp_create", gpu._h, n, d, wp, bp, lote, C.byref(cfg), C.byref(h))
        return cls(gpu, h.value, dims, lote, precision)

    def destroy(self):
        # A closed Gpu already released its models.
        if self._h and self.gpu._h:
            lib().rt_mlp_destroy(self._h)
        self._h = None

    def _live(self):
        """The plan's handle; raises once the plan or its Gpu is gone (a
        closed context releases its models, so the handle would dangle)."""
        if not self._h or not self.gpu._h:
            raise RtError(2, "the model was destroyed or its Gpu was closed")
        return self._h

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass

    def step(self, x: GpuTensor, labels: GpuTensor) -> None:
        self.gpu._call("rt_mlp_step", self._live(), x.handle, labels.handle)

    def carregar(self, x, labels) -> None:
        """GpuMlp::carregar (mod.rs:1486-1495), overlapped: stage a host batch
        (f32, or bf16 bits / f32 values for a bf16 plan) and its labels; the
        host-to-device copy runs while earlier steps compute."""
        x = np.asarray(x)
        if self.precision == "bf16":
            host = x if x.dtype == np.uint16 else f32_to_bf16_bits(x)
        else:
            host = x.astype(np.float32, copy=False)
        host = np.ascontiguousarray(host)
        lab = np.ascontiguousarray(np.asarray(labels).astype(np.uint64))
        self.gpu._call("rt_mlp_load", self._live(), host.ctypes.data_as(C.c_void_p), host.nbytes,
                       lab.ctypes.data_as(C.POINTER(C.c_uint64)), lab.size)

    load = carregar  # the batch loader, rt_mlp_load (checkpoints: save_checkpoint / load_checkpoint)

    def step_loaded(self) -> None:
        """rt_mlp_step on the most recently loaded batch."""
        self.gpu._call("rt_mlp_step_loaded", self._live())

    def forward_only(self, x: GpuTensor) -> None:
        self.gpu._call("rt_mlp_forward", self._live(), x.handle)

    def activation(self, layer: int) -> np.ndarray:
        """The stored activation of ``layer`` (ReLU output of a hidden layer,
        logits of the last), f32 [batch, width]."""
        out = np.empty((self.lote, self.dims[layer + 1]), np.float32)
        self.gpu._call("rt_mlp_activation", self._live(), int(layer), out.ctypes.data_as(C.POINTER(C.c_float)),
                       out.size)
        return out

    def delta(self, layer: int) -> np.ndarray:
        """δ = ∂L/∂Z of ``layer`` as the backward GEMMs read it (under bf16,
        the bf16 values times the loss scale), f32 [batch, width]."""
        out = np.empty((self.lote, self.dims[layer + 1]), np.float32)
        self.gpu._call("rt_mlp_delta", self._live(), int(layer), out.ctypes.data_as(C.POINTER(C.c_float)), out.size)
        return out

    def logits(self) -> np.ndarray:
        out = np.empty((self.lote, self.dims[-1]), np.float32)
        self.gpu._call("rt_mlp_logits", self._live(), out.ctypes.data_as(C.POINTER(C.c_float)), out.size)
        return out

    def last_loss(self) -> float:
        v = C.c_float()
        self.gpu._call("rt_mlp_last_loss", self._live(), C.byref(v))
        return v.value

    def _shapes(self):
        out = []
        for l in range(len(self.dims) - 1):
            out += [(self.dims[l], self.dims[l + 1]), (1, self.dims[l + 1])]
        return out

    def _fetch(self, fn: str) -> List[np.ndarray]:
        arrs = [np.empty(s, np.float32) for s in self._shapes()]
        ptrs = (C.POINTER(C.c_float) * len(arrs))(*[a.ctypes.data_as(C.POINTER(C.c_float)) for a in arrs])
        self.gpu._call(fn, self._live(), ptrs, len(arrs))
        return arrs

    def weights(self) -> List[np.ndarray]:
        return self._fetch("rt_mlp_weights")

    @staticmethod
    def _ptrs(arrs):
        return (C.POINTER(C.c_float) * len(arrs))(*[a.ctypes.data_as(C.POINTER(C.c_float)) for a in arrs])

    def _checked(self, arrs) -> List[np.ndarray]:
        shapes = self._shapes()
        if len(arrs) != len(shapes):
            raise ValueError(f"need {len(shapes)} arrays, got {len(arrs)}")
        out = []
        for a, shp in zip(arrs, shapes):
            a = np.ascontiguousarray(a, dtype=np.float32)
            if a.size != int(np.prod(shp)):
                raise ValueError(f"array of {a.size} elements for a parameter of shape {shp}")
            out.append(a)
        return out

    def set_weights(self, arrs) -> None:
        """Param::set (tape.rs:119-121) for every parameter, in parameter order."""
        arrs = self._checked(arrs)
        self.gpu._call("rt_mlp_set_weights", self._live(), self._ptrs(arrs), len(arrs))

    def optimizer_state(self):
        """(m, v, t): the optimizer's moments per parameter and the applied-update count."""
        m = [np.empty(s, np.float32) for s in self._shapes()]
        v = [np.empty(s, np.float32) for s in self._shapes()]
        t = C.c_int()
        self.gpu._call("rt_mlp_get_optimizer_state", self._live(), self._ptrs(m), self._ptrs(v), len(m), C.byref(t))
        return m, v, t.value

    def set_optimizer_state(self, m, v, t: int) -> None:
        m, v = self._checked(m), self._checked(v)
        self.gpu._call("rt_mlp_set_optimizer_state", self._live(), self._ptrs(m), self._ptrs(v), len(m), int(t))

    def state_dict(self) -> dict:
        """Everything a resumed run needs: weights, optimizer moments and t."""
        m, v, t = self.optimizer_state()
        return {"weights": self.weights(), "m": m, "v": v, "t": t}

    def load_state_dict(self, state: dict) -> None:
        self.set_weights(state["weights"])
        self.set_optimizer_state(state["m"], state["v"], state["t"])

    def save_checkpoint(self, path: str) -> None:
        """Checkpoint to an .npz file (plain arrays, no pickled objects)."""
        st = self.state_dict()
        arrays = {"t": np.array([st["t"]], np.int64)}
        for key in ("weights", "m", "v"):
            for i, a in enumerate(st[key]):
                arrays[f"{key}_{i}"] = a
        np.savez(path, **arrays)

    def load_checkpoint(self, path: str) -> None:
        n = len(self._shapes())
        with np.load(path, allow_pickle=False) as z:
            st = {key: [z[f"{key}_{i}"] for i in range(n)] for key in ("weights", "m", "v")}
            st["t"] = int(z["t"][0])
        self.load_state_dict(st)

    def grads(self) -> List[np.ndarray]:
        return self._fetch("rt_mlp_grads")

    def dispatches_por_passo(self) -> int:
        v = C.c_int()
        self.gpu._call("rt_mlp_dispatches", self._live(), C.byref(v))
        return v.value

    def overflow(self) -> bool:
        v = C.c_int()
        self.gpu._call("rt_mlp_overflow", self._live(), C.byref(v))
        return bool(v.value)
