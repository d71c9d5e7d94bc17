"""C ABI checks that need no GPU: the library loads and exports exactly what
include/rtensor_hip.h declares; opening a device without one fails cleanly."""
import ctypes as C
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "rtensor_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rt_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    syms = declared_symbols()
    for must in ("rt_open", "rt_gemm", "rt_gemm_splitk", "rt_colsum", "rt_softmax_xent", "rt_adam", "rt_sgd",
                 "rt_mlp_create", "rt_mlp_step", "rt_mlp_last_loss", "rt_mlp_weights", "rt_mlp_grads"):
        assert must in syms


def test_library_exports_every_declared_symbol():
    from rgpu_amd import gpu as G

    L = G.lib()
    for s in declared_symbols():
        assert hasattr(L, s), s
    # and the ctypes mirror covers the same set
    assert sorted(G.SIGNATURES) == declared_symbols()
    out = subprocess.run(["nm", "-D", "--defined-only", G.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (rt_[a-z0-9_]+)\b", out))
    assert set(declared_symbols()) <= exported


def test_open_without_device_reports_no_device():
    from rgpu_amd import gpu as G

    L = G.lib()
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU is present")
    h = C.c_void_p()
    rc = L.rt_open(0, C.byref(h))
    assert rc == 1 and not h.value  # RT_ERR_NO_DEVICE
    assert L.rt_last_error(None).decode()
    with pytest.raises(G.RtError) as e:
        G.Gpu(0)
    assert e.value.status == "RT_ERR_NO_DEVICE"


def test_null_handles_are_rejected():
    from rgpu_amd import gpu as G

    L = G.lib()
    assert L.rt_sync(None) == 2
    assert L.rt_mlp_step(None, None, None) == 2
    assert L.rt_gemm(None, 0, None, None, None, 0, None, None) == 2


def test_splitk_slice_rule():
    # fatias_sugeridas' contract (tests/gpu.rs:432-441), re-derived for 256 CUs
    from rgpu_amd.gpu import Gpu

    assert Gpu.fatias_sugeridas(64, 64, 8192) > 1
    assert Gpu.fatias_sugeridas(4096, 4096, 4096) == 1
    assert Gpu.fatias_sugeridas(64, 64, 64) == 1
    assert Gpu.fatias_sugeridas(1024, 10, 2048) > 1


def test_bf16_rounding_helper():
    import numpy as np

    from rgpu_amd.gpu import bf16_bits_to_f32, f32_to_bf16_bits

    x = np.array([1.0, 1.00390625, 1.01171875, -2.5, 3.4e38, 1e-40], np.float32)
    b = f32_to_bf16_bits(x)
    # 1 + 2^-8 is a tie -> even (1.0); 1 + 3·2^-8 is a tie -> even (1 + 2^-6)
    assert bf16_bits_to_f32(b).tolist()[:4] == [1.0, 1.0, 1.015625, -2.5]
    y = np.random.default_rng(0).normal(size=1000).astype(np.float32)
    assert np.max(np.abs(bf16_bits_to_f32(f32_to_bf16_bits(y)) - y) / np.abs(y)) <= 2.0 ** -8
