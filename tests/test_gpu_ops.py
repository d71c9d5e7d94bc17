"""Op-level parity of the HIP kernels against the CPU oracle
(crates/rtensor/tests/gpu.rs:215-503 and closed forms)."""
import numpy as np
import pytest

from oracle import oracle as O
from rgpu_amd import gpu as G

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gpu():
    g = G.Gpu(0)
    print("device:", g.info(), flush=True)
    yield g
    g.close()


def assert_near_exact(got, exact, cpu, floor=1e-5, what=""):
    """got must be as close to the float64 result as max(floor, 3x the CPU
    path's own f32 error) -- long sums of N(0,1) data make the sequential
    CPU sum itself ~1e-5 off exact."""
    e_cpu = O.erro_rel(cpu, exact)
    e = O.erro_rel(got, exact)
    print(f"{what}: vs exact {e:.2e} (CPU path {e_cpu:.2e})")
    assert e < max(floor, 3 * e_cpu), (what, e, e_cpu)


def sincos(m, k, n, fa=0.013, fb=0.007):
    a = np.sin(np.arange(m * k, dtype=np.float32) * np.float32(fa)).astype(np.float32).reshape(m, k)
    b = np.cos(np.arange(k * n, dtype=np.float32) * np.float32(fb)).astype(np.float32).reshape(k, n)
    return a, b


def test_upload_download_roundtrip_is_exact(gpu):  # gpu.rs:215-221
    t = (np.arange(15, dtype=np.float32) * 0.5 - 3.0).reshape(3, 5)
    assert np.array_equal(gpu.download(gpu.upload(t)), t)
    u = np.arange(1000, dtype=np.uint32) * 7919
    assert np.array_equal(gpu.download(gpu.upload(u)), u)
    h = np.random.default_rng(0).normal(size=(33, 7)).astype(np.float16)
    assert np.array_equal(gpu.download(gpu.upload(h)), h)
    lab = gpu.download(G.upload_labels(gpu, np.array([0, 9, 3, 4294967295], np.uint64)))
    assert lab.tolist() == [0, 9, 3, 4294967295]


def test_matmul_37x19x23(gpu):  # gpu.rs:223-240
    a = np.sin(np.arange(37 * 23, dtype=np.float32) * np.float32(0.11)).reshape(37, 23)
    b = np.cos(np.arange(23 * 19, dtype=np.float32) * np.float32(0.07)).reshape(23, 19)
    c = gpu.zeros((37, 19))
    gpu.matmul(gpu.upload(a), gpu.upload(b), c)
    assert O.erro_rel(O.matmul(a, b), gpu.download(c)) < 1e-5


# The seven shapes of gpu.rs:250-258 (K <= 128) keep the reference's 1e-5
# bound against the CPU result.  For long K the CPU result itself sits ~2e-5
# from the exact product on this data, so those shapes are judged against the
# float64 product with a bound of 3x the CPU path's own error (the rule
# gpu.rs:418-426 applies to split-K).
REF_SHAPES = [(1, 1, 1), (17, 33, 65), (64, 64, 64), (65, 64, 63), (130, 96, 80), (199, 130, 71), (256, 512, 128)]
LONG_K = [(300, 1030, 257), (2048, 10, 1024), (1024, 10, 2048), (2048, 1024, 1024)]


def _three_layouts(gpu, a, b):
    m, n = a.shape[0], b.shape[1]
    ga, gb = gpu.upload(a), gpu.upload(b)
    gat, gbt = gpu.upload(a.T.copy()), gpu.upload(b.T.copy())
    c1, c2, c3 = gpu.zeros((m, n)), gpu.zeros((m, n)), gpu.zeros((m, n))
    gpu.matmul(ga, gb, c1)
    gpu.matmul_at_b(gat, gb, c2)
    gpu.matmul_a_bt(ga, gbt, c3)
    return (("mm", gpu.download(c1)), ("mm_atb", gpu.download(c2)), ("mm_abt", gpu.download(c3)))


@pytest.mark.parametrize("m,n,k", REF_SHAPES)
def test_gemm_three_layouts(gpu, m, n, k):  # gpu.rs:244-295
    a, b = sincos(m, k, n)
    want = O.matmul(a, b)
    for name, got in _three_layouts(gpu, a, b):
        e = O.erro_rel(want, got)
        print(f"{name} {m}x{n}x{k}: erro_rel {e:.2e}")
        assert e < 1e-5, (name, m, n, k, e)


@pytest.mark.parametrize("m,n,k", LONG_K)
def test_gemm_three_layouts_long_k(gpu, m, n, k):
    a, b = sincos(m, k, n)
    exact = a.astype(np.float64) @ b.astype(np.float64)
    e_cpu = O.erro_rel(O.matmul(a, b), exact)
    for name, got in _three_layouts(gpu, a, b):
        e = O.erro_rel(exact, got)
        print(f"{name} {m}x{n}x{k}: vs exact {e:.2e} (CPU path {e_cpu:.2e})")
        assert e < max(3 * e_cpu, 2e-5), (name, m, n, k, e, e_cpu)


def test_gemm_large_tile_path(gpu):
    # 2048 x 2048 output takes the 128x128 tile kernel
    m, n, k = 2048, 2048, 96
    rng = np.random.default_rng(1)
    a = rng.normal(size=(m, k)).astype(np.float32)
    b = rng.normal(size=(k, n)).astype(np.float32)
    want = O.matmul(a, b)
    for layout, A, B in ((G.NN, a, b), (G.TN, a.T.copy(), b), (G.NT, a, b.T.copy())):
        c = gpu.zeros((m, n))
        gpu.gemm(layout, gpu.upload(A), gpu.upload(B), c)
        assert O.erro_rel(want, gpu.download(c)) < 1e-5, layout


# (130, 200, 77) takes the register-staged kernel; (128, 192, 96) is made of
# whole 64x64 tiles and takes the direct-to-LDS one.
@pytest.mark.parametrize("m,n,k", [(130, 200, 77), (128, 192, 96)])
def test_gemm_epilogues(gpu, m, n, k):
    rng = np.random.default_rng(2)
    a = rng.normal(size=(m, k)).astype(np.float32)
    w = rng.normal(size=(k, n)).astype(np.float32)
    bias = rng.normal(size=(1, n)).astype(np.float32)
    z = O.matmul(a, w) + bias
    ga, gw, gbias = gpu.upload(a), gpu.upload(w), gpu.upload(bias)
    c = gpu.zeros((m, n))
    gpu.matmul_bias(ga, gw, c, gbias, relu=False)
    assert O.erro_rel(z, gpu.download(c)) < 1e-5
    gpu.matmul_bias(ga, gw, c, gbias, relu=True)
    got = gpu.download(c)
    assert O.erro_rel(np.maximum(z, 0), got) < 1e-5 and (got >= 0).all()
    # δ_prev = (δ·Wᵀ) ⊙ 1[A > 0]: mask from a post-ReLU activation
    d = rng.normal(size=(m, n)).astype(np.float32)
    act = np.maximum(rng.normal(size=(m, k)).astype(np.float32), 0)
    want = O.matmul(d, w.T.copy()) * (act > 0)
    out = gpu.zeros((m, k))
    gpu.matmul_a_bt(gpu.upload(d), gw, out, relu_mask_from=gpu.upload(act))
    got = gpu.download(out)
    assert O.erro_rel(want, got) < 1e-5
    assert np.all(got[act <= 0] == 0)



# Products of at most 64 rows with 16-column and 16-k blocks (K >= 128) run on
# the skinny kernel: 8 waves of a block split K and their partial tiles are
# added in LDS.  Row counts below, at and above a 16-row block, K runs of one
# to several load chunks per wave.
@pytest.mark.parametrize("m,n,k", [(1, 16, 128), (17, 48, 144), (32, 1024, 512), (33, 64, 1040), (64, 512, 1024),
                                   (64, 16, 4096)])
def test_skinny_products_with_epilogues(gpu, m, n, k):
    rng = np.random.default_rng(m * 7 + n + k)
    a = rng.normal(size=(m, k)).astype(np.float32)
    w = rng.normal(size=(k, n)).astype(np.float32)
    bias = rng.normal(size=(1, n)).astype(np.float32)
    ga, gw, gbias = gpu.upload(a), gpu.upload(w), gpu.upload(bias)
    exact = a.astype(np.float64) @ w.astype(np.float64) + bias
    cpu = O.matmul(a, w) + bias
    c = gpu.zeros((m, n))
    gpu.matmul_bias(ga, gw, c, gbias, relu=False)
    assert_near_exact(gpu.download(c), exact, cpu, floor=2e-5, what=f"NN+bias {m}x{n}x{k}")
    gpu.matmul_bias(ga, gw, c, gbias, relu=True)
    got = gpu.download(c)
    assert_near_exact(got, np.maximum(exact, 0), np.maximum(cpu, 0), floor=2e-5, what=f"NN+bias+relu {m}x{n}x{k}")
    assert (got >= 0).all()
    # NT with the ReLU mask: out [m, n] = d [m, k] · v [n, k]ᵀ, zero where act <= 0
    d = rng.normal(size=(m, k)).astype(np.float32)
    v = rng.normal(size=(n, k)).astype(np.float32)
    act = np.maximum(rng.normal(size=(m, n)).astype(np.float32), 0)
    exact = (d.astype(np.float64) @ v.astype(np.float64).T) * (act > 0)
    cpu = O.matmul(d, v.T.copy()) * (act > 0)
    out = gpu.zeros((m, n))
    gpu.matmul_a_bt(gpu.upload(d), gpu.upload(v), out, relu_mask_from=gpu.upload(act))
    got = gpu.download(out)
    assert_near_exact(got, exact, cpu, floor=2e-5, what=f"NT+mask {m}x{n}x{k}")
    assert np.all(got[act <= 0] == 0)

# NT products with K <= 16 (the dX of a narrow output layer) run on the
# rank-K block: ragged M and N (edges of the 64x64 blocks, N not a multiple of
# 4 for the scalar stores), K from 1 to 16, every epilogue.
@pytest.mark.parametrize("m,n,k", [(1, 4, 1), (65, 130, 10), (100, 33, 7), (256, 1024, 16), (2048, 1024, 10)])
def test_rank_k_nt_products_with_epilogues(gpu, m, n, k):
    rng = np.random.default_rng(m + 3 * n + k)
    d = rng.normal(size=(m, k)).astype(np.float32)
    v = rng.normal(size=(n, k)).astype(np.float32)
    gd, gv = gpu.upload(d), gpu.upload(v)
    exact = d.astype(np.float64) @ v.astype(np.float64).T
    cpu = O.matmul(d, v.T.copy())
    out = gpu.zeros((m, n))
    gpu.matmul_a_bt(gd, gv, out)
    assert_near_exact(gpu.download(out), exact, cpu, floor=2e-5, what=f"NT {m}x{n}x{k}")
    act = np.maximum(rng.normal(size=(m, n)).astype(np.float32), 0)
    gpu.matmul_a_bt(gd, gv, out, relu_mask_from=gpu.upload(act))
    got = gpu.download(out)
    assert_near_exact(got, exact * (act > 0), cpu * (act > 0), floor=2e-5, what=f"NT+mask {m}x{n}x{k}")
    assert np.all(got[act <= 0] == 0)
    # integer operands: every order of the K products gives the exact sum
    di = rng.integers(-4, 5, size=(m, k)).astype(np.float32)
    vi = rng.integers(-4, 5, size=(n, k)).astype(np.float32)
    gpu.matmul_a_bt(gpu.upload(di), gpu.upload(vi), out)
    assert np.array_equal(gpu.download(out), (di.astype(np.float64) @ vi.T).astype(np.float32))


@pytest.mark.parametrize("k,m,n", [(2048, 1024, 10), (64, 130, 96), (513, 64, 1024), (256, 128, 192)])
def test_tn_gemm_fused_colsum(gpu, k, m, n):
    rng = np.random.default_rng(3)
    x = rng.normal(size=(k, m)).astype(np.float32)
    d = rng.normal(size=(k, n)).astype(np.float32)
    c, cs = gpu.zeros((m, n)), gpu.zeros((1, n))
    gpu.matmul_at_b(gpu.upload(x), gpu.upload(d), c, colsum=cs)
    assert_near_exact(gpu.download(c), x.T.astype(np.float64) @ d, O.matmul(x.T.copy(), d), what="dW")
    assert_near_exact(gpu.download(cs), d.astype(np.float64).sum(0, keepdims=True), O.reduce_to(d, (1, n)),
                      what="db")
    # integer-valued δ: every order gives the exact sum
    di = rng.integers(-8, 9, size=(k, n)).astype(np.float32)
    gpu.matmul_at_b(gpu.upload(x), gpu.upload(di), c, colsum=cs)
    assert np.array_equal(gpu.download(cs).reshape(-1), di.sum(0, dtype=np.float64).astype(np.float32))


# N = 10 and 7: the reduction's scalar path (rows not a multiple of four
# floats); slices 1..16 take the eight-plane loop and the tail.
@pytest.mark.parametrize("m,n,k", [(64, 64, 4096), (32, 96, 2048), (128, 64, 1024), (50, 10, 2048), (33, 7, 1024)])
def test_split_k_against_whole_gemm(gpu, m, n, k):  # gpu.rs:383-430
    a, b = sincos(m, k, n)
    want = O.matmul(a, b)
    ga, gat, gb = gpu.upload(a), gpu.upload(a.T.copy()), gpu.upload(b)
    whole = gpu.zeros((m, n))
    gpu.matmul(ga, gb, whole)
    e_whole = O.erro_rel(want, gpu.download(whole))
    whole_t = gpu.zeros((m, n))
    gpu.matmul_at_b(gat, gb, whole_t)
    for slices in (1, 2, 4, 8, 16):
        for trans, inp, ref in ((False, ga, whole), (True, gat, whole_t)):
            c = gpu.zeros((m, n))
            part = gpu.zeros((slices * m + slices, n))
            gpu.split_k(inp, gb, c, part, slices, trans)
            got = gpu.download(c)
            e = O.erro_rel(want, got)
            assert e < max(3 * e_whole, 2e-5), (slices, trans, e, e_whole)
            if slices == 1:
                assert np.array_equal(got, gpu.download(ref))
            c2 = gpu.zeros((m, n))
            gpu.split_k(inp, gb, c2, part, slices, trans)
            assert np.array_equal(got, gpu.download(c2))  # deterministic


def test_split_k_fused_colsum(gpu):  # dW and db of a K-dominant layer in one split launch
    rng = np.random.default_rng(4)
    k, m, n, s = 4096, 100, 12, 8
    x = rng.normal(size=(k, m)).astype(np.float32)
    d = rng.normal(size=(k, n)).astype(np.float32)
    c, cs = gpu.zeros((m, n)), gpu.zeros((1, n))
    part = gpu.zeros((s * m * n + s * n,))
    gpu.split_k(gpu.upload(x), gpu.upload(d), c, part, s, True, colsum=cs)
    assert_near_exact(gpu.download(c), x.T.astype(np.float64) @ d, O.matmul(x.T.copy(), d), what="dW")
    assert_near_exact(gpu.download(cs), d.astype(np.float64).sum(0, keepdims=True), O.reduce_to(d, (1, n)),
                      what="db")


@pytest.mark.parametrize("rows,cols,dt", [(2048, 1024, G.F32), (33, 7, G.F32), (5000, 300, G.BF16),
                                          (4096, 512, G.F16), (1, 1, G.F32)])
def test_colsum(gpu, rows, cols, dt):
    rng = np.random.default_rng(5)
    x = rng.normal(size=(rows, cols)).astype(np.float32)
    if dt == G.BF16:
        x = G.bf16_bits_to_f32(G.f32_to_bf16_bits(x))
    elif dt == G.F16:
        x = x.astype(np.float16).astype(np.float32)
    out = gpu.zeros((1, cols))
    gpu.colsum(gpu.upload(x, dt), out)
    assert_near_exact(gpu.download(out), x.astype(np.float64).sum(0, keepdims=True), O.reduce_to(x, (1, cols)),
                      what=f"colsum {rows}x{cols}")
    xi = np.random.default_rng(6).integers(-4, 5, size=(rows, cols)).astype(np.float32)
    gpu.colsum(gpu.upload(xi, dt), out)  # integers: exact in every order
    assert np.array_equal(gpu.download(out).reshape(-1), xi.sum(0, dtype=np.float64).astype(np.float32))


def test_softmax_xent_matches_cpu_and_flags_bad_labels(gpu):
    rng = np.random.default_rng(6)
    B, C = 300, 10
    z = (rng.normal(size=(B, C)) * 4).astype(np.float32)
    lab = rng.integers(0, C, size=B).astype(np.uint32)
    p = O.softmax_rows(z)
    want_delta = ((p - O.one_hot(lab, C)) * np.float32(1.0 / B)).astype(np.float32)
    want_loss = -np.log(np.maximum(p[np.arange(B), lab], np.float32(1e-12)))
    gz, gl = gpu.upload(z), G.upload_labels(gpu, lab)
    d, lr = gpu.zeros((B, C)), gpu.zeros((B,))
    gpu.softmax_xent(gz, gl, d, lr)
    assert O.erro_rel(want_delta, gpu.download(d)) < 1e-6
    assert np.max(np.abs(want_loss - gpu.download(lr))) < 1e-5
    gpu.sync()
    lab[7] = C  # out of range: reported at the next blocking call, nothing read out of bounds
    gpu.softmax_xent(gz, G.upload_labels(gpu, lab), d, lr)
    with pytest.raises(G.RtError) as e:
        gpu.sync()
    assert e.value.status == "RT_ERR_LABEL"
    gpu.sync()  # flag cleared once reported


def test_relu_bias_add_relu_bwd(gpu):
    rng = np.random.default_rng(7)
    z = rng.normal(size=(77, 33)).astype(np.float32)
    b = rng.normal(size=(1, 33)).astype(np.float32)
    gz = gpu.upload(z)
    gpu.bias_add(gz, gpu.upload(b))
    assert np.array_equal(gpu.download(gz), (z + b).astype(np.float32))
    y = gpu.zeros((77, 33))
    gpu.relu(gz, y)
    assert np.array_equal(gpu.download(y), np.maximum(z + b, 0))
    d = rng.normal(size=(77, 33)).astype(np.float32)
    gd = gpu.upload(d)
    gpu.relu_bwd(y, gd)
    assert np.array_equal(gpu.download(gd), np.where(np.maximum(z + b, 0) > 0, d, 0).astype(np.float32))


def test_adam_and_sgd_are_bit_exact_with_cpu_arithmetic(gpu):
    # Same inputs -> same bits as optim.rs's expression order.
    rng = np.random.default_rng(8)
    n = 10_001
    theta = rng.normal(size=(1, n)).astype(np.float32)
    p = O.Param(theta)
    opt = O.Optimizer("adam", 1e-3)
    gt, gm, gv = gpu.upload(theta), gpu.zeros((1, n)), gpu.zeros((1, n))
    for t in range(1, 6):
        g = rng.normal(size=(1, n)).astype(np.float32) * np.float32(10.0 ** -t)
        tp = O.Tape()
        tp.watch(p).mul(tp.constant(g)).sum().backward()
        opt.step([p], tp)
        gpu.adam(gt, gm, gv, gpu.upload(g), 1e-3, (0.9, 0.999), t)
        assert np.array_equal(gpu.download(gt), p.value()), t
    p2 = O.Param(theta)
    sgd = O.Optimizer("sgd", 0.01, 0.9)
    gt2, vel = gpu.upload(theta), gpu.zeros((1, n))
    for _ in range(3):
        g = rng.normal(size=(1, n)).astype(np.float32)
        tp = O.Tape()
        tp.watch(p2).mul(tp.constant(g)).sum().backward()
        sgd.step([p2], tp)
        gpu.sgd(gt2, gpu.upload(g), 0.01, 0.9, vel)
    assert np.array_equal(gpu.download(gt2), p2.value())


def test_adam_launch_larger_than_the_cache_gives_the_same_bits(gpu):
    # An optimizer launch that moves more than the 256 MB last-level cache
    # reads and writes its streams non-temporally; the same update as two
    # launches of half the size each does not.  Same arithmetic, same bits,
    # the ragged tail (n not a multiple of 4) included.
    n, h = 10_000_003, 5_000_000  # 28 B per Adam parameter: ~280 MB, ~140 MB
    rng = np.random.default_rng(21)
    theta = rng.normal(size=(1, n)).astype(np.float32)
    whole = [gpu.upload(theta), gpu.zeros((1, n)), gpu.zeros((1, n))]
    parts = [[gpu.upload(np.ascontiguousarray(theta[:, s])), gpu.zeros((1, w)), gpu.zeros((1, w))]
             for s, w in ((slice(0, h), h), (slice(h, n), n - h))]
    for t in (1, 2, 3):
        g = (rng.normal(size=(1, n)) * 10.0 ** -t).astype(np.float32)
        gpu.adam(*whole, gpu.upload(g), 1e-3, (0.9, 0.999), t)
        for (th, m, v), s in zip(parts, (slice(0, h), slice(h, n))):
            gpu.adam(th, m, v, gpu.upload(np.ascontiguousarray(g[:, s])), 1e-3, (0.9, 0.999), t)
    for i in range(3):  # theta, m, v
        want = np.concatenate([gpu.download(parts[0][i]), gpu.download(parts[1][i])], axis=1)
        assert np.array_equal(gpu.download(whole[i]), want), i


@pytest.mark.parametrize("m,n,k", [(64, 64, 64), (256, 128, 512), (512, 512, 256), (130, 70, 200)])
@pytest.mark.parametrize("dt", [G.F16, G.BF16])
def test_half_gemm_three_layouts(gpu, m, n, k, dt):  # gpu.rs:445-503
    a = np.sin(np.arange(m * k, dtype=np.float32) * np.float32(0.019)).astype(np.float32).reshape(m, k)
    b = np.cos(np.arange(k * n, dtype=np.float32) * np.float32(0.013)).astype(np.float32).reshape(k, n)
    want = O.matmul(a, b)
    if dt == G.F16:
        ar, br = a.astype(np.float16).astype(np.float32), b.astype(np.float16).astype(np.float32)
        bound = 10 * np.sqrt(k) * 2.0 ** -11
    else:
        ar, br = G.bf16_bits_to_f32(G.f32_to_bf16_bits(a)), G.bf16_bits_to_f32(G.f32_to_bf16_bits(b))
        bound = 10 * np.sqrt(k) * 2.0 ** -8
    exact_inputs = O.matmul(ar, br)  # same rounded operands, f32 accumulate
    for layout, A, B in ((G.NN, a, b), (G.TN, a.T.copy(), b), (G.NT, a, b.T.copy())):
        c = gpu.zeros((m, n))
        gpu.gemm(layout, gpu.upload(A, dt), gpu.upload(B, dt), c)
        got = gpu.download(c)
        assert O.erro_rel(want, got) < bound, (layout, O.erro_rel(want, got), bound)
        assert O.erro_rel(exact_inputs, got) < 1e-5, (layout, O.erro_rel(exact_inputs, got))


def test_half_gemm_bf16_output_and_epilogue(gpu):
    rng = np.random.default_rng(9)
    m, n, k = 256, 384, 192
    a = G.bf16_bits_to_f32(G.f32_to_bf16_bits(rng.normal(size=(m, k)).astype(np.float32)))
    w = G.bf16_bits_to_f32(G.f32_to_bf16_bits(rng.normal(size=(k, n)).astype(np.float32)))
    bias = rng.normal(size=(1, n)).astype(np.float32)
    want = np.maximum(O.matmul(a, w) + bias, 0)
    c = gpu.zeros((m, n), G.BF16)
    gpu.gemm(G.NN, gpu.upload(a, G.BF16), gpu.upload(w, G.BF16), c, G.EPI_BIAS_RELU, gpu.upload(bias))
    got = G.bf16_bits_to_f32(gpu.download(c))
    assert np.max(np.abs(got - want) / (1 + np.abs(want))) < 2.0 ** -8


def test_convert_round_trip(gpu):
    x = np.random.default_rng(10).normal(size=(1000,)).astype(np.float32)
    x[:4] = [1.00390625, 1.01171875, 6.0e-8, -65504.0]
    src = gpu.upload(x)
    hb, hf = gpu.zeros((1000,), G.BF16), gpu.zeros((1000,), G.F16)
    gpu.convert(src, hb)
    gpu.convert(src, hf)
    assert np.array_equal(gpu.download(hb), G.f32_to_bf16_bits(x))
    assert np.array_equal(gpu.download(hf), x.astype(np.float16))  # RNE, subnormals kept


def test_shape_errors_are_reported(gpu):
    a, b, c = gpu.zeros((4, 5)), gpu.zeros((6, 7)), gpu.zeros((4, 7))
    with pytest.raises(G.RtError) as e:
        gpu.matmul(a, b, c)
    assert e.value.status == "RT_ERR_SHAPE"
    with pytest.raises(G.RtError) as e:
        gpu.matmul(gpu.zeros((4, 6)), b, gpu.zeros((4, 8)))
    assert e.value.status == "RT_ERR_SHAPE"


def test_row_counts_past_int32_are_refused(gpu):
    # The row kernels take int row and column counts and add block extents to
    # them: counts above 2^30 are refused on the host, before any launch
    # (8 GiB buffers of 2^31 rows, never initialised or read).
    rows = 2 ** 31
    z = gpu.empty((rows, 1))
    lab = gpu.empty((rows,), G.U32)
    calls = (lambda: gpu.colsum(z, gpu.zeros((1, 1))),
             lambda: gpu.bias_add(z, gpu.zeros((1,))),
             lambda: gpu.softmax_xent(z, lab, z, z))
    for call in calls:
        with pytest.raises(G.RtError) as e:
            call()
        assert e.value.status == "RT_ERR_SHAPE" and "large" in str(e.value)
    del z, lab


@pytest.mark.parametrize("m,n,k", [(4096, 4096, 256), (4100, 4000, 96)])
@pytest.mark.parametrize("dt", [G.BF16, G.F16])
def test_half_gemm_large_tiles(gpu, m, n, k, dt):
    # Shapes big enough for the 256x256 block configuration, including ragged
    # edge tiles; against the float64 product of the same rounded operands.
    rng = np.random.default_rng(11)
    a = rng.standard_normal((m, k), dtype=np.float32)
    b = rng.standard_normal((k, n), dtype=np.float32)
    if dt == G.F16:
        ar, br = a.astype(np.float16).astype(np.float64), b.astype(np.float16).astype(np.float64)
    else:
        ar = G.bf16_bits_to_f32(G.f32_to_bf16_bits(a)).astype(np.float64)
        br = G.bf16_bits_to_f32(G.f32_to_bf16_bits(b)).astype(np.float64)
    exact = ar @ br
    bias = rng.standard_normal((1, n), dtype=np.float32)
    for layout, A, B in ((G.NN, a, b), (G.TN, a.T.copy(), b), (G.NT, a, b.T.copy())):
        ga, gb = gpu.upload(A, dt), gpu.upload(B, dt)
        c = gpu.zeros((m, n))
        gpu.gemm(layout, ga, gb, c)
        e = O.erro_rel(exact, gpu.download(c))
        print(f"layout {layout} {m}x{n}x{k}: erro_rel vs exact {e:.2e}")
        assert e < 2e-6 * np.sqrt(k), (layout, e)
    # bf16 output with the bias+ReLU epilogue, and TN with the fused colsum
    cb = gpu.zeros((m, n), G.BF16)
    gpu.gemm(G.NN, gpu.upload(a, dt), gpu.upload(b, dt), cb, G.EPI_BIAS_RELU, gpu.upload(bias))
    want = np.maximum(exact + bias, 0)
    got = G.bf16_bits_to_f32(gpu.download(cb))
    assert np.max(np.abs(got - want) / (1 + np.abs(want))) < 2.0 ** -8
    cs = gpu.zeros((1, n))
    gpu.gemm(G.TN, gpu.upload(a.T.copy(), dt), gpu.upload(b, dt), c, colsum=cs)
    assert O.erro_rel(br.sum(0, keepdims=True), gpu.download(cs)) < 1e-5


@pytest.mark.gpu
def test_region_timer(gpu):
    a = gpu.upload(np.ones((256, 256), np.float32))
    c = gpu.zeros((256, 256))
    gpu.timer_begin()
    for _ in range(3):
        gpu.gemm(G.NN, a, a, c)
    ms = gpu.timer_end()
    assert 0.0 < ms < 1000.0
    assert np.all(gpu.download(c) == 256.0)
    with pytest.raises(G.RtError):
        gpu.timer_end()  # no region open


@pytest.mark.parametrize("m,k,n,dt", [(256, 128, 512, G.F32), (256, 512, 10, G.F32), (200, 96, 72, G.F32),
                                      (256, 256, 128, G.BF16)])
def test_linear_backward_matches_separate_gemms(gpu, m, k, n, dt):
    """rt_linear_backward (one paired launch where it can) gives the bits of
    rt_gemm TN with the fused colsum plus rt_gemm NT; dx may be skipped."""
    r = np.random.default_rng(m + k + n)
    x = gpu.upload(r.standard_normal((m, k)).astype(np.float32), dt)
    d = gpu.upload(r.standard_normal((m, n)).astype(np.float32), dt)
    w = gpu.upload(r.standard_normal((k, n)).astype(np.float32), dt)
    dx1, dw1, db1 = gpu.zeros((m, k)), gpu.zeros((k, n)), gpu.zeros((1, n))
    gpu.linear_backward(x, d, w, dx1, dw1, db1)
    dx2, dw2, db2 = gpu.zeros((m, k)), gpu.zeros((k, n)), gpu.zeros((1, n))
    gpu.gemm(G.TN, x, d, dw2, colsum=db2)
    gpu.gemm(G.NT, d, w, dx2)
    for a, b in ((dx1, dx2), (dw1, dw2), (db1, db2)):
        assert np.array_equal(gpu.download(a).view(np.uint32), gpu.download(b).view(np.uint32))
    dw3 = gpu.zeros((k, n))
    gpu.linear_backward(x, d, w, None, dw3, None)
    assert np.array_equal(gpu.download(dw3).view(np.uint32), gpu.download(dw2).view(np.uint32))
    with pytest.raises(G.RtError):
        gpu.linear_backward(x, d, gpu.zeros((k + 1, n)), dx1, dw1, db1)


@pytest.mark.parametrize("dt", [G.F32, G.BF16])
def test_zero_sized_dimensions(gpu, dt):
    """Empty inner and outer dimensions as the CPU path treats them: K = 0
    sums nothing, so C is the epilogue applied to zero (tensor.rs:318-373 with
    k = 0) and the fused column sums are zero; zero rows or columns launch
    nothing and leave the outputs alone; output buffers start as garbage."""
    m, n = 70, 130
    bias = np.linspace(-1, 1, n, dtype=np.float32).reshape(1, n)
    junk = np.full((m, n), 7.0, np.float32)
    a0, b0 = np.zeros((m, 0), np.float32), np.zeros((0, n), np.float32)
    want = np.maximum(O.matmul(a0, b0) + bias, 0)
    c = gpu.upload(junk)
    gpu.gemm(G.NN, gpu.upload(a0, dt), gpu.upload(b0, dt), c, G.EPI_BIAS_RELU, gpu.upload(bias))
    assert np.array_equal(gpu.download(c), want)
    # TN with the bias gradient fused, over zero rows of δ
    c, cs = gpu.upload(junk), gpu.upload(np.full((1, n), 3.0, np.float32))
    gpu.gemm(G.TN, gpu.upload(np.zeros((0, m), np.float32), dt), gpu.upload(b0, dt), c, colsum=cs)
    assert np.array_equal(gpu.download(c), O.matmul(a0, b0))
    assert np.array_equal(gpu.download(cs), O.reduce_to(b0, (1, n)))
    # split-K over K = 0: every slice is empty, the reduce writes zeros
    c, cs = gpu.upload(junk), gpu.upload(np.full((1, n), 3.0, np.float32))
    parts = gpu.upload(np.full((4 * m * n + 4 * n,), 5.0, np.float32))
    gpu.split_k(gpu.upload(np.zeros((0, m), np.float32), dt), gpu.upload(b0, dt), c, parts, 4, True, colsum=cs)
    assert not gpu.download(c).any() and not gpu.download(cs).any()
    # M = 0 and N = 0: nothing to write
    gpu.gemm(G.NN, gpu.upload(np.zeros((0, 5), np.float32), dt), gpu.upload(np.ones((5, n), np.float32), dt),
             gpu.zeros((0, n)))
    gpu.gemm(G.NN, gpu.upload(np.ones((m, 5), np.float32), dt), gpu.upload(np.zeros((5, 0), np.float32), dt),
             gpu.zeros((m, 0)))
    gpu.sync()


def test_zero_rows_in_row_ops(gpu):
    """Column sums of zero rows are zero (reduce_to sums nothing); the loss
    and argmax of an empty batch launch nothing; the accuracy of an empty
    batch is 0/0 = NaN and of zero columns 0 (no predictions), as
    losses.rs:181-185 computes them."""
    cs = gpu.upload(np.full((1, 9), 2.0, np.float32))
    gpu.colsum(gpu.zeros((0, 9)), cs)
    assert np.array_equal(gpu.download(cs), O.reduce_to(np.zeros((0, 9), np.float32), (1, 9)))
    z, lab = gpu.zeros((0, 10)), gpu.upload(np.zeros(0, np.uint32))
    gpu.softmax_xent(z, lab, gpu.zeros((0, 10)), gpu.zeros((0,)))
    gpu.argmax_rows(z, gpu.upload(np.zeros(0, np.uint32)))
    acc = gpu.accuracy(z, lab)
    assert np.isnan(acc) and np.isnan(O.accuracy(np.zeros((0, 10), np.float32), np.zeros(0, np.uint32)))
    lab3 = gpu.upload(np.zeros(3, np.uint32))
    assert gpu.accuracy(gpu.zeros((3, 0)), lab3) == O.accuracy(np.zeros((3, 0), np.float32), np.zeros(3, np.uint32)) == 0.0
    with pytest.raises(G.RtError):
        gpu.argmax_rows(gpu.zeros((3, 0)), gpu.upload(np.zeros(3, np.uint32)))
    gpu.sync()


@pytest.mark.parametrize("m,n,k", [(256, 10, 512), (33, 1, 128), (1000, 16, 384), (5, 7, 1024)])
@pytest.mark.parametrize("bias", [False, True])
def test_narrow_f32_product(gpu, m, n, k, bias):
    """Narrow f32 NN products (<= 16 columns, K a multiple of 128: an output
    layer's logits) run on the output-layer kernel: as close to the float64
    product as the oracle's sequential f32 sum is, or 1e-5, and within 1e-4
    of the oracle (N(0,1) data: sums over K of unit terms)."""
    r = np.random.default_rng(m + n + k)
    a, w = r.standard_normal((m, k)).astype(np.float32), r.standard_normal((k, n)).astype(np.float32)
    b = r.standard_normal((1, n)).astype(np.float32)
    c = gpu.upload(np.full((m, n), 9.0, np.float32))
    if bias:
        gpu.gemm(G.NN, gpu.upload(a), gpu.upload(w), c, G.EPI_BIAS, gpu.upload(b))
        cpu = O.matmul(a, w) + b
        exact = a.astype(np.float64) @ w.astype(np.float64) + b
    else:
        gpu.matmul(gpu.upload(a), gpu.upload(w), c)
        cpu = O.matmul(a, w)
        exact = a.astype(np.float64) @ w.astype(np.float64)
    got = gpu.download(c)
    assert O.erro_rel(got, cpu) < 1e-4
    assert_near_exact(got, exact, cpu, what=f"narrow {m}x{n}x{k}")


def test_contexts_are_independent_and_usable_from_other_threads():
    """Two contexts in one process keep their own streams, buffers and caches,
    and a context opened on one thread works from another (every entry point
    makes the context's device current first)."""
    import threading

    r = np.random.default_rng(31)
    a, b = r.standard_normal((130, 70)).astype(np.float32), r.standard_normal((70, 90)).astype(np.float32)
    want = O.matmul(a, b)
    g1, g2 = G.Gpu(0), G.Gpu(0)
    try:
        c1 = g1.empty((130, 90))
        c2 = g2.empty((130, 90))
        g1.matmul(g1.upload(a), g1.upload(b), c1)
        g2.matmul(g2.upload(a), g2.upload(b), c2)
        out = {}

        def worker():
            c = g1.empty((130, 90))
            g1.matmul(g1.upload(a), g1.upload(b), c)
            out["c"] = g1.download(c)

        t = threading.Thread(target=worker)
        t.start()
        t.join()
        for got in (g1.download(c1), g2.download(c2), out["c"]):
            assert O.erro_rel(got, want) < 1e-5
        with pytest.raises(G.RtError):
            g2._call("rt_free", g2._h, c1.handle)  # a buffer of the other context
    finally:
        g1.close()
        g2.close()


@pytest.mark.parametrize("k,slices", [(4096, 64), (16384, 64), (65536, 32)])
@pytest.mark.parametrize("dt", [G.F16, G.BF16])
def test_half_split_k_streaming_shapes(gpu, k, slices, dt):
    """Split-K half GEMMs with few 256x256 output tiles (512x512: 4 tiles)
    and many slices (1 to 16 stages of 64 k per slice): NN and TN with the
    bias gradient fused, against the oracle on the same rounded inputs, and
    deterministic."""
    m = n = 512
    r = np.random.default_rng(k + slices)
    a = r.standard_normal((k, m)).astype(np.float32) / np.float32(16.0)
    b = r.standard_normal((k, n)).astype(np.float32) / np.float32(16.0)
    if dt == G.F16:
        ar, br = a.astype(np.float16).astype(np.float32), b.astype(np.float16).astype(np.float32)
    else:
        ar, br = G.bf16_bits_to_f32(G.f32_to_bf16_bits(a)), G.bf16_bits_to_f32(G.f32_to_bf16_bits(b))
    want = O.matmul(O.transpose(ar), br)
    exact = ar.T.astype(np.float64) @ br.astype(np.float64)
    ga, gb = gpu.upload(a, dt), gpu.upload(b, dt)
    part = gpu.zeros((slices * (m * n + n),))
    c, cs = gpu.zeros((m, n)), gpu.zeros((1, n))
    gpu.split_k(ga, gb, c, part, slices, True, colsum=cs)
    got = gpu.download(c)
    assert O.erro_rel(got, want) < 1e-4
    assert_near_exact(got, exact, want, what=f"TN split {k}/{slices}")
    assert O.erro_rel(gpu.download(cs), br.astype(np.float64).sum(0, keepdims=True)) < 1e-5
    c2 = gpu.zeros((m, n))
    gpu.split_k(ga, gb, c2, part, slices, True, colsum=cs)
    assert np.array_equal(got, gpu.download(c2))
    # NN: A stored [M, K]
    gat = gpu.upload(np.ascontiguousarray(a.T), dt)
    c3 = gpu.zeros((m, n))
    gpu.split_k(gat, gb, c3, part, slices, False)
    assert O.erro_rel(gpu.download(c3), want) < 1e-4
