"""Half-precision conversion on the device (rt_convert) against IEEE 754.

The reference packs f32 into f16 on the GPU (EMPACOTA, gpu/mista.rs:326-341,
through upload_f16, gpu/mod.rs:1151-1185) and decodes halves back to f32; its
notes record a hand-written f16 decoder that halved every subnormal
(RESULTADOS-NEGATIVOS.md:737-747: 0x0001 must decode to 2^-24).  Here:

* half -> f32 is exhaustive: all 65536 f16 and all 65536 bf16 bit patterns,
  bit-exact against numpy's float16 widening and the bf16 bit shift;
* f32 -> f16 and f32 -> bf16 are checked at every representable half value,
  at every midpoint between neighbours (ties go to the even neighbour) and
  one f32 ulp either side of it, across subnormals, the normal range and the
  overflow boundary, against numpy (f16) and a nearest-value search in
  float64 (bf16) that shares no code with the kernel;
* NaN stays NaN, signed zeros keep their sign, odd lengths convert whole.
"""
import numpy as np
import pytest

from rgpu_amd import gpu as G

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gpu():
    g = G.Gpu(0)
    yield g
    g.close()


def to_f32(gpu, bits: np.ndarray, dtype: int) -> np.ndarray:
    src = gpu.upload(bits.view(np.float16) if dtype == G.F16 else bits, dtype)
    dst = gpu.zeros(bits.shape, G.F32)
    gpu.convert(src, dst)
    return gpu.download(dst)


def from_f32(gpu, x: np.ndarray, dtype: int) -> np.ndarray:
    src = gpu.upload(np.ascontiguousarray(x, np.float32))
    dst = gpu.zeros(x.shape, dtype)
    gpu.convert(src, dst)
    return gpu.download(dst).view(np.uint16)


def test_f16_to_f32_exhaustive(gpu):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = to_f32(gpu, bits, G.F16)
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    # the subnormals the reference's hand-written decoder got wrong
    assert got[0x0001] == np.float32(2.0 ** -24)
    assert got[0x03FF] == np.float32(1023 * 2.0 ** -24)
    assert got[0x8001] == np.float32(-(2.0 ** -24))
    assert got[0x0400] == np.float32(2.0 ** -14)  # smallest normal


def test_bf16_to_f32_exhaustive(gpu):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = to_f32(gpu, bits, G.BF16)
    want = (bits.astype(np.uint32) << 16).view(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def boundary_inputs(values: np.ndarray) -> np.ndarray:
    """Each finite half value, the midpoints to its upper neighbour, and one
    f32 ulp either side of each midpoint (all as f32)."""
    v = values.astype(np.float64)
    lo, hi = v[:-1], v[1:]
    mid = ((lo + hi) / 2).astype(np.float32)  # exact in f32 for f16 and bf16 neighbours
    below = np.nextafter(mid, np.float32(-np.inf))
    above = np.nextafter(mid, np.float32(np.inf))
    return np.concatenate([values.astype(np.float32), mid, below, above])


def test_f32_to_f16_rounds_to_nearest_even(gpu):
    pos = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16)  # +0 .. 65504
    x = boundary_inputs(pos.astype(np.float32))
    x = np.concatenate([x, -x, np.float32([65519.996, 65520.0, 1e6, np.inf, -np.inf, 2.0 ** -25, 2.0 ** -26])])
    got = from_f32(gpu, x, G.F16)
    with np.errstate(over="ignore"):  # values past 65520 overflow to inf, as intended
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    # spot checks: ties to even in the subnormal range, the overflow boundary
    f = lambda v: int(from_f32(gpu, np.float32([v]), G.F16)[0])  # noqa: E731
    assert f(2.0 ** -25) == 0x0000      # half of the smallest subnormal: tie to even 0
    assert f(3 * 2.0 ** -25) == 0x0002  # 1.5 ulp: tie to even 2
    assert f(65504.0) == 0x7BFF
    assert f(65520.0) == 0x7C00         # tie above the largest finite rounds to inf
    assert f(-0.0) == 0x8000


def nearest_bf16(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even onto bf16 by searching the two bf16 neighbours
    in float64 (no bit tricks shared with the kernel); finite inputs only."""
    u = x.view(np.uint32)
    lo_bits = (u >> 16).astype(np.uint32)  # truncation toward zero (sign-magnitude)
    hi_bits = lo_bits + 1
    lo = (lo_bits << 16).view(np.float32).astype(np.float64)
    hi = (hi_bits << 16).view(np.float32).astype(np.float64)
    xv = x.astype(np.float64)
    dlo, dhi = np.abs(xv - lo), np.abs(hi - xv)
    pick_hi = (dhi < dlo) | ((dhi == dlo) & (lo_bits & 1 == 1))
    return np.where(pick_hi, hi_bits, lo_bits).astype(np.uint16)


def test_f32_to_bf16_rounds_to_nearest_even(gpu):
    # every positive finite bf16 below the largest, its midpoints and neighbours
    pos_bits = np.arange(0, 0x7F7F, dtype=np.uint32)
    pos = (pos_bits << 16).view(np.float32)
    x = boundary_inputs(pos)
    x = np.concatenate([x, -x])
    got = from_f32(gpu, x, G.BF16)
    assert np.array_equal(got, nearest_bf16(x))
    # overflow to inf past the largest finite bf16, NaN stays NaN
    big = np.float32([3.3961776e38, np.inf, -np.inf, np.nan])
    g = from_f32(gpu, big, G.BF16)
    assert g[0] == 0x7F80 and g[1] == 0x7F80 and g[2] == 0xFF80
    assert (g[3] & 0x7F80) == 0x7F80 and (g[3] & 0x007F) != 0


def test_nan_and_signed_zero_round_trip(gpu):
    x = np.float32([np.nan, -np.nan, 0.0, -0.0, 1.0, -2.5])
    for dt in (G.F16, G.BF16):
        h = gpu.upload(x)
        d = gpu.zeros(x.shape, dt)
        gpu.convert(h, d)
        back = gpu.zeros(x.shape, G.F32)
        gpu.convert(d, back)
        b = gpu.download(back)
        assert np.isnan(b[0]) and np.isnan(b[1])
        assert b[2:].tobytes() == x[2:].tobytes()  # signs of the zeros kept


@pytest.mark.parametrize("n", [1, 3, 1001, 65537])
def test_odd_lengths_convert_every_element(gpu, n):
    # EMPACOTA pads the last packed word of an odd length with zero; a
    # per-element layout has no padding: every element converts.
    x = np.random.default_rng(n).standard_normal(n).astype(np.float32) * np.float32(1e-5)
    got = from_f32(gpu, x, G.F16)
    assert np.array_equal(got, x.astype(np.float16).view(np.uint16))
