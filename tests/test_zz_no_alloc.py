"""rt_gemm_splitk_static, the split-K GEMM that allocates nothing (its partial
planes live in the library's static device array), against rt_gemm_splitk with
a caller's workspace: the same kernels, so the same bits.  Two calls in a row,
the second on a smaller input (the array keeps the first call's contents), and
the capacity limit."""
import numpy as np
import pytest

from rgpu_amd import gpu as G
from tests.gpu_common import normal_batch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gpu():
    g = G.Gpu(0)
    yield g
    g.close()


def _operands(gpu, dtype, K, M, N, seed):
    # A stored [K, M] (TN) and B [K, N], N(0,1)/16 as the split-K dW config
    a = normal_batch(seed, K, M) / np.float32(16)
    b = normal_batch(seed + 1, K, N) / np.float32(16)
    return gpu.upload(a, dtype), gpu.upload(b, dtype)


def _both(gpu, dtype, K, M, N, slices, colsum, seed):
    print(f"static split-K: dtype {dtype} K={K} M={M} N={N} slices={slices} colsum={colsum}", flush=True)
    ga, gb = _operands(gpu, dtype, K, M, N, seed)
    ref_c, got_c = gpu.zeros((M, N)), gpu.zeros((M, N))
    ref_b = gpu.zeros((1, N)) if colsum else None
    got_b = gpu.zeros((1, N)) if colsum else None
    part = gpu.zeros((slices * (M * N + N),))
    gpu.split_k(ga, gb, ref_c, part, slices, True, colsum=ref_b)
    gpu.split_k_static(ga, gb, got_c, slices, True, colsum=got_b)
    assert np.array_equal(gpu.download(got_c), gpu.download(ref_c))
    if colsum:
        assert np.array_equal(gpu.download(got_b), gpu.download(ref_b))
    return gpu.download(got_c)


def test_static_split_k_matches_the_workspace_version_on_two_calls(gpu):
    # the K = 262144 f16 weight gradient with db at 32 slices (33.6 MB of
    # planes), then a smaller bf16 one whose planes overlap the first's
    big = _both(gpu, G.F16, 262144, 512, 512, 32, True, 31)
    small = _both(gpu, G.BF16, 8192, 256, 384, 8, True, 41)
    assert big.shape == (512, 512) and small.shape == (256, 384)
    # f32 operands, no column sums, a ragged shape; and one slice (no planes)
    _both(gpu, G.F32, 5000, 130, 70, 16, False, 51)
    _both(gpu, G.F32, 777, 64, 64, 1, True, 61)


def test_static_split_k_rejects_more_than_its_array(gpu):
    # 64 slices of a 512 x 512 product with column sums: 64·(512·512 + 512)
    # floats plus the shares exceed 64 MiB
    ga, gb = _operands(gpu, G.F16, 64 * 512, 512, 512, 71)
    c, b = gpu.zeros((512, 512)), gpu.zeros((1, 512))
    with pytest.raises(G.RtError) as e:
        gpu.split_k_static(ga, gb, c, 64, True, colsum=b)
    assert e.value.status == "RT_ERR_SHAPE"
    assert not gpu.download(c).any()  # nothing ran
    gpu.split_k_static(ga, gb, c, 16, True, colsum=b)  # and the context still works
    assert gpu.download(c).any()
