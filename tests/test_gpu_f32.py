"""GPU parity of the f32 kernels (gemm/gemv, softmax, LayerNorm, RMSNorm, GELU,
argmax) against the oracle's scalar restatements and float64.

Bars (per element):
  * gemm / gemv: |gpu - f64| <= k * 2^-23 * sum_l |a_l b_l| + 1e-30, the
    reassociation bound of an f32 dot product of length k (the GPU sums in a
    different order than the reference's left fold); the oracle satisfies the
    same bound.
  * softmax: |gpu - f64| <= (cols + 4) * 2^-23 * f64 (the oracle meets it too);
    LN, RMSNorm, GELU: |gpu - oracle| <= atol + rtol |oracle| as written per test.
  * argmax: exact, including ties (lowest index) and NaN (never wins).
"""
import numpy as np
import pytest

from vokra_amd import hip

pytestmark = pytest.mark.gpu
U = 2.0 ** -23


@pytest.fixture(scope="module")
def ctx():
    c = hip.HipContext(0)
    yield c
    c.close()


def dot_bound(a, b, k):
    return k * U * (np.abs(a.astype(np.float64)) @ np.abs(b.astype(np.float64))) + 1e-30


@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (3, 5, 7), (64, 64, 16), (65, 130, 33), (200, 51, 1280),
                                   (17, 300, 2048), (130, 260, 96), (257, 128, 1280), (1, 4, 32)])
def test_gemm_f32(ctx, oracle, m, n, k):
    print(f"[case] gemm_f32 {m}x{n}x{k}", flush=True)
    g = np.random.default_rng(m * 31 + n * 7 + k)
    a = g.standard_normal((m, k)).astype(np.float32)
    b = g.standard_normal((k, n)).astype(np.float32)
    bias = g.standard_normal(n).astype(np.float32)
    got = ctx.gemm_f32(m, n, k, a, b, bias)
    exact = a.astype(np.float64) @ b.astype(np.float64) + bias
    bound = dot_bound(a, b, k + 1) + U * np.abs(bias)
    assert np.all(np.abs(got - exact) <= bound)
    want = oracle.gemm_f32(m, n, k, a, b, bias)
    assert np.all(np.abs(want - exact) <= bound)


@pytest.mark.parametrize("m,n,k", [(100, 77, 64), (3000, 1280, 384), (5, 402, 400)])
def test_gemm_f32_b_transposed_tiled(ctx, m, n, k):
    """B stored [n, k] (weights [out, in]) through the tiled kernel (k % 16 == 0),
    ragged m and n; GELU epilogue path via the bias-free product."""
    print(f"[case] gemm_f32 b^T tiled {m}x{n}x{k}", flush=True)
    g = np.random.default_rng(m + n + k)
    a = g.standard_normal((m, k)).astype(np.float32)
    e = (g.standard_normal((n, k)) * 0.05).astype(np.float32)
    bias = g.standard_normal(n).astype(np.float32)
    d_a, d_e, d_b = (hip.DeviceBuffer.from_array(ctx, x) for x in (a, e, bias))
    d_o = hip.DeviceBuffer(ctx, m * n * 4)
    ctx.gemm_f32_dev(m, n, k, d_a, d_e, d_o, d_bias=d_b, b_trans=True)
    got = d_o.download(np.float32, m * n).reshape(m, n)
    exact = a.astype(np.float64) @ e.astype(np.float64).T + bias
    assert np.all(np.abs(got - exact) <= dot_bound(a, e.T, k + 1) + U * np.abs(bias))


def test_gemm_f32_b_transposed_dev(ctx):
    """Logits shape: h[64, 1280] . E^T with E [V, 1280] read as b [n, k]."""
    print("[case] gemm_f32 b^T (logits)", flush=True)
    m, n, k = 64, 5187, 1280
    g = np.random.default_rng(9)
    h = g.standard_normal((m, k)).astype(np.float32)
    e = (g.standard_normal((n, k)) * 0.02).astype(np.float32)
    d_h, d_e = hip.DeviceBuffer.from_array(ctx, h), hip.DeviceBuffer.from_array(ctx, e)
    d_o = hip.DeviceBuffer(ctx, m * n * 4)
    ctx.gemm_f32_dev(m, n, k, d_h, d_e, d_o, b_trans=True)
    got = d_o.download(np.float32, m * n).reshape(m, n)
    exact = h.astype(np.float64) @ e.astype(np.float64).T
    assert np.all(np.abs(got - exact) <= dot_bound(h, e.T, k))


@pytest.mark.parametrize("m,k", [(1, 1), (7, 3), (513, 1280), (5187, 1280), (100, 1001)])
def test_gemv_f32(ctx, oracle, m, k):
    print(f"[case] gemv_f32 {m}x{k}", flush=True)
    g = np.random.default_rng(m + k)
    a = g.standard_normal((m, k)).astype(np.float32)
    x = g.standard_normal(k).astype(np.float32)
    bias = g.standard_normal(m).astype(np.float32)
    got = ctx.gemv_f32(m, k, a, x, bias)
    exact = a.astype(np.float64) @ x + bias
    bound = (k + 1) * U * (np.abs(a.astype(np.float64)) @ np.abs(x)) + U * np.abs(bias) + 1e-30
    assert np.all(np.abs(got - exact) <= bound)
    assert np.all(np.abs(oracle.gemv_f32(m, k, a, x, bias) - exact) <= bound)


def close(got, want, atol=1e-6, rtol=1e-5):
    return np.all(np.abs(np.asarray(got, np.float64) - want) <= atol + rtol * np.abs(want))


@pytest.mark.parametrize("rows,cols", [(1, 1), (3, 7), (64, 1500), (2, 51866)])
def test_softmax(ctx, oracle, rows, cols):
    g = np.random.default_rng(rows * cols)
    x = (g.standard_normal((rows, cols)) * 4).astype(np.float32)
    got = ctx.softmax_f32(x, rows, cols)
    # float64 truth; both the GPU's tree sum and the reference's sequential
    # f32 sum stay within the summation bound (cols + 4) * 2^-23 relative
    x64 = x.astype(np.float64)
    e = np.exp(x64 - x64.max(axis=1, keepdims=True))
    exact = e / e.sum(axis=1, keepdims=True)
    bound = (cols + 4) * U * exact + 1e-30
    assert np.all(np.abs(got - exact) <= bound)
    assert np.all(np.abs(oracle.softmax_f32(x, rows, cols) - exact) <= bound)
    assert np.allclose(got.sum(axis=1), 1.0, atol=1e-5)


@pytest.mark.parametrize("rows,cols", [(1, 1), (5, 64), (1500, 1280), (3, 5120)])
def test_layer_norm(ctx, oracle, rows, cols):
    g = np.random.default_rng(rows + cols)
    x = (g.standard_normal((rows, cols)) * 3 + 1).astype(np.float32)
    gamma = g.standard_normal(cols).astype(np.float32)
    beta = g.standard_normal(cols).astype(np.float32)
    got = ctx.layer_norm_f32(x, rows, cols, gamma, beta)
    want = oracle.layer_norm_f32(x, rows, cols, gamma, beta)
    assert close(got, want, atol=1e-5, rtol=1e-4)


def test_layer_norm_constant_row_gives_beta(ctx):
    """scalar.rs layer_norm test: a constant row normalises to beta exactly."""
    g = np.random.default_rng(2)
    gamma = g.standard_normal(64).astype(np.float32)
    beta = g.standard_normal(64).astype(np.float32)
    got = ctx.layer_norm_f32(np.full((3, 64), 2.5, np.float32), 3, 64, gamma, beta)
    assert np.array_equal(got, np.tile(beta, (3, 1)))


def test_rms_norm(ctx, oracle):
    g = np.random.default_rng(3)
    x = g.standard_normal((32, 2048)).astype(np.float32)
    gamma = g.standard_normal(2048).astype(np.float32)
    got = ctx.rms_norm_f32(x, 32, 2048, gamma, 1e-6)
    assert close(got, oracle.rms_norm_f32(x, gamma, 1e-6, 32, 2048), atol=1e-5, rtol=1e-5)
    one = ctx.rms_norm_f32(np.array([[1, 2, 3, 4]], np.float32), 1, 4, np.ones(4, np.float32), 0.0)
    assert abs(float((one.astype(np.float64) ** 2).mean()) - 1.0) < 1e-5


def test_gelu(ctx, oracle):
    g = np.random.default_rng(4)
    x = np.concatenate([g.standard_normal(100000) * 3, np.linspace(-8, 8, 1001), [0.0, -0.0]]).astype(np.float32)
    got = ctx.gelu_f32(x)
    assert close(got, oracle.gelu_f32(x), atol=1e-6, rtol=1e-6)
    assert got[-2] == 0.0


def test_argmax_rules(ctx, oracle):
    rows = np.array([[1, 3, 3, 2], [np.nan, 1, 5, 5], [-np.inf, -np.inf, -np.inf, -np.inf],
                     [np.nan, np.nan, np.nan, np.nan]], np.float32)
    g = np.random.default_rng(5)
    big = g.standard_normal((3, 51866)).astype(np.float32)
    big[1, 777] = big[1, 40000] = 100.0
    # ties and NaN at the edges of the 2048-column slices the kernel merges
    edge = g.standard_normal((6, 6200)).astype(np.float32)
    edge[0, 2047] = edge[0, 2048] = 50.0
    edge[1, 4096] = edge[1, 6199] = 50.0
    edge[2] = 0.0
    edge[2, :2048] = -0.0
    edge[3, ::2] = np.nan
    edge[3, 4095] = 9.0
    edge[4] = -np.inf
    edge[4, 6199] = -1e30
    edge[5] = np.nan
    for mat in (rows, big, edge):
        d_l = hip.DeviceBuffer.from_array(ctx, mat)
        d_o = hip.DeviceBuffer(ctx, mat.shape[0] * 4)
        ctx.argmax_f32_dev(d_l, mat.shape[0], mat.shape[1], d_o)
        got = d_o.download(np.int32, mat.shape[0])
        want = [oracle.argmax(r) for r in mat]
        assert got.tolist() == want


def test_f32_rejections(ctx):
    with pytest.raises(hip.InvalidArgument, match="gemm b length 5 does not match expected 6"):
        ctx.gemm_f32(2, 3, 2, np.zeros(4), np.zeros(5))
    with pytest.raises(hip.InvalidArgument, match="gemv x length"):
        ctx.gemv_f32(2, 3, np.zeros(6), np.zeros(2))
    with pytest.raises(hip.InvalidArgument):
        ctx.layer_norm_f32(np.zeros(8), 2, 4, np.zeros(3), np.zeros(4))


def fused_logits(ctx, x, e, write=True):
    n, d = x.shape
    v = e.shape[0]
    d_x, d_e = hip.DeviceBuffer.from_array(ctx, x), hip.DeviceBuffer.from_array(ctx, e)
    d_l = hip.DeviceBuffer(ctx, n * v * 4) if write else None
    d_n = hip.DeviceBuffer(ctx, n * 4)
    ctx.logits_argmax_dev(n, v, d, d_x, d_e, d_l, d_n)
    logits = d_l.download(np.float32, n * v).reshape(n, v) if write else None
    return logits, d_n.download(np.int32, n)


@pytest.mark.parametrize("n,v,d", [(1, 51866, 1280), (5, 1000, 128), (16, 4099, 384), (17, 333, 512),
                                   (33, 2049, 256), (64, 51866, 1280), (70, 777, 640)])
def test_logits_argmax(ctx, oracle, n, v, d):
    """Fused tied logits + argmax: logits within the f32 dot-product bound of
    float64; next = the sampler's argmax of the kernel's own logits, exactly,
    with and without the logits written."""
    print(f"[case] logits_argmax n={n} v={v} d={d}", flush=True)
    g = np.random.default_rng(n * 1000 + d)
    x = g.standard_normal((n, d)).astype(np.float32)
    e = (g.standard_normal((v, d)) * 0.05).astype(np.float32)
    logits, nxt = fused_logits(ctx, x, e)
    exact = x.astype(np.float64) @ e.astype(np.float64).T
    assert np.all(np.abs(logits - exact) <= dot_bound(x, e.T, d))
    assert nxt.tolist() == [oracle.argmax(r) for r in logits]
    _, nxt2 = fused_logits(ctx, x, e, write=False)
    assert np.array_equal(nxt, nxt2)


def test_logits_argmax_rules(ctx, oracle):
    """Ties across workgroups keep the lowest index, NaN rows never win, +inf
    wins at its first index, and rows with nothing above -inf give 0."""
    print("[case] logits_argmax rules", flush=True)
    g = np.random.default_rng(77)
    n, v, d = 6, 40100, 256
    x = np.abs(g.standard_normal((n, d))).astype(np.float32) + 0.1
    e = (g.standard_normal((v, d)) * 0.01).astype(np.float32)
    e[40001] = e[7] = e[33] = 0.5       # equal maxima in three workgroups
    e[3] = np.nan                       # a NaN logit for every stream
    logits, nxt = fused_logits(ctx, x, e)
    assert np.isnan(logits[:, 3]).all()
    assert np.array_equal(logits[:, 7], logits[:, 40001]) and np.array_equal(logits[:, 7], logits[:, 33])
    assert nxt.tolist() == [7] * n == [oracle.argmax(r) for r in logits]
    e[39000] = np.inf
    e[39500] = np.inf
    logits, nxt = fused_logits(ctx, x, e)
    assert nxt.tolist() == [39000] * n == [oracle.argmax(r) for r in logits]
    for fill in (-np.inf, np.nan):
        _, nxt = fused_logits(ctx, x[:, :128].copy(), np.full((300, 128), fill, np.float32), write=False)
        assert nxt.tolist() == [0] * n


def test_logits_argmax_rejections(ctx):
    x = hip.DeviceBuffer(ctx, 4 * 200)
    e = hip.DeviceBuffer(ctx, 4 * 200 * 10)
    nx = hip.DeviceBuffer(ctx, 16)
    with pytest.raises(hip.InvalidArgument, match="multiple of 128"):
        ctx.logits_argmax_dev(1, 10, 200, x, e, None, nx)
    with pytest.raises(hip.InvalidArgument, match="vocab"):
        ctx.logits_argmax_dev(1, 0, 128, x, e, None, nx)
