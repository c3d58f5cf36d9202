"""GPU parity of the Q4_K path (dequantize + K-quant INT8 matmul) against the
oracle, through the C ABI.

Bars (written per test):
  * kquant_dequantize: bit-exact (NaN scales: NaN in the same places).
  * gemm_q_f32 Q4_K: bit-exact f32 outputs. The integer group sums are exact
    and the combine acc += s * (d_eff * isum - m_eff * gsum) runs in the
    reference's block-then-group order (kquant.rs:590-629), so nothing is
    left to a tolerance. Independently of the oracle, outputs stay within
    2x the reference's int8_error_bound (kquant.rs:471-495) of an f64
    dequant-then-dot, the bound the reference's own parity tests use.
"""
import numpy as np
import pytest

from tests.helpers import Rng, hand_q4k_ints, random_kquant_blocks
from vokra_amd import hip

pytestmark = pytest.mark.gpu

W_Q4_K = 12


@pytest.fixture(scope="module")
def ctx():
    c = hip.HipContext(0)
    yield c
    c.close()


def same_bits(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    return np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32))


def q4k_weights(seed, n, k):
    """Reference-style random blocks (kquant_gemm_parity.rs:45-62)."""
    return random_kquant_blocks(Rng(seed), n * (k // 256))


def test_dequantize_random_blocks(ctx, oracle):
    print("[case] q4k dequantize random", flush=True)
    w = q4k_weights(0x51, 300, 256)
    got = ctx.kquant_dequantize(hip.WDtype.Q4_K, w, 300 * 256)
    want = oracle.kquant_dequantize(W_Q4_K, w, 300 * 256)
    assert same_bits(got, want)


def test_dequantize_every_d_pattern(ctx, oracle):
    """All 65536 f16 bit patterns of d and of dmin (subnormals, inf, NaN)."""
    print("[case] q4k dequantize all d/dmin", flush=True)
    g = np.random.default_rng(4)
    blocks = g.integers(0, 256, size=(65536, 144), dtype=np.uint8)
    pat = np.arange(65536)
    blocks[:, 0], blocks[:, 1] = pat & 0xFF, pat >> 8
    perm = g.permutation(65536)
    blocks[:, 2], blocks[:, 3] = perm & 0xFF, perm >> 8
    got = ctx.kquant_dequantize(hip.WDtype.Q4_K, blocks.reshape(-1), 65536 * 256)
    want = oracle.kquant_dequantize(W_Q4_K, blocks.reshape(-1), 65536 * 256)
    assert same_bits(got, want)


def test_dequantize_closed_form(ctx):
    """Against an independent numpy parse: y = d*sc*q - dmin*m."""
    print("[case] q4k dequantize closed form", flush=True)
    w = q4k_weights(0x77, 40, 256)
    q, d_eff, m_eff = hand_q4k_ints(w)
    want = (np.repeat(d_eff, 16, axis=1) * q.astype(np.float32) - np.repeat(m_eff, 16, axis=1)).astype(np.float32)
    got = ctx.kquant_dequantize(hip.WDtype.Q4_K, w, 40 * 256).reshape(40, 256)
    assert same_bits(got, want)


def test_dequantize_rejections(ctx):
    with pytest.raises(hip.InvalidArgument):
        ctx.kquant_dequantize(hip.WDtype.Q4_K, np.zeros(144, np.uint8), 255)
    with pytest.raises(hip.InvalidArgument):
        ctx.kquant_dequantize(hip.WDtype.Q4_K, np.zeros(143, np.uint8), 256)
    with pytest.raises(hip.UnsupportedOp):
        ctx.kquant_dequantize(hip.WDtype.Q8_0, np.zeros(144, np.uint8), 256)


GEMM_SHAPES = [(1, 16, 256), (1, 37, 512), (3, 64, 768), (17, 100, 768), (16, 33, 1280), (40, 48, 1024),
               (64, 80, 512), (130, 20, 256)]


@pytest.mark.parametrize("m,n,k", GEMM_SHAPES)
@pytest.mark.parametrize("with_bias", [False, True])
def test_gemm_q4k_bit_exact(ctx, oracle, m, n, k, with_bias):
    print(f"[case] q4k gemm m={m} n={n} k={k} bias={with_bias}", flush=True)
    g = np.random.default_rng(m * 1000 + n + k)
    a = g.standard_normal((m, k)).astype(np.float32)
    a[0, :16] = 0.0                       # an all-zero group: scale 0, gsum 0
    if m > 2:
        a[2, 16:32] *= 1e-30              # tiny but nonzero amax
    w = q4k_weights(m * 7 + n, n, k)
    bias = g.standard_normal(n).astype(np.float32) if with_bias else None
    got = ctx.gemm_q_f32(m, n, k, a, w, hip.WDtype.Q4_K, bias=bias)
    want = oracle.gemm_q_f32(W_Q4_K, m, n, k, a, w, bias)
    assert same_bits(got, want)


def test_gemm_q4k_activation_edge_values(ctx, oracle):
    """The K-quant activation pass (kquant.rs:418-441: amax over the group
    with NaN ignored, s = amax / 127, q = clamp(round(v / s)) with NaN -> 0,
    integer group sum) on groups random inputs do not reach, through the
    matmul, bit-exact: an all-NaN group (amax 0: s = 0, every q 0), one NaN
    in a normal group, +Inf and -Inf elements (s = inf, every q 0, so the
    row's outputs are NaN in the same places), exact half ties of v / s
    (round half away from zero), a subnormal-only group, groups near the
    largest finite value, and a row count that leaves padding rows."""
    print("[case] q4k gemm activation edge values", flush=True)
    m, n, k = 21, 48, 512
    g = np.random.default_rng(77)
    a = g.standard_normal((m, k)).astype(np.float32)
    a[0, :16] = 0.0
    a[1, 16:32] = np.nan
    a[1, 40] = np.nan
    a[2, 48] = np.inf
    a[3, 64] = -np.inf
    # amax = 127 / 8, so s = 1/8 exactly and v / s = these values exactly
    ties = np.array([127, 63.5, -63.5, 0.5, -0.5, 1.5, -2.5, 126.5, -126.5, 3, 0, 7.5, -7.5, 100.5, -0.25, 0.75])
    a[4, 80:96] = (ties / 8).astype(np.float32)
    a[5, 96:112] = (np.arange(16) - 8).astype(np.float32) * np.float32(1e-40)
    a[6, 112:128] = (np.finfo(np.float32).max * (g.random(16) * 2 - 1)).astype(np.float32)
    a[7, 128:144] = np.float32(np.finfo(np.float32).max)
    w = q4k_weights(0x77, n, k)
    got = ctx.gemm_q_f32(m, n, k, a, w, hip.WDtype.Q4_K)
    want = oracle.gemm_q_f32(W_Q4_K, m, n, k, a, w, None)
    assert np.isnan(want[2]).all() and np.isnan(want[3]).all()  # the Inf rows
    assert np.isfinite(want[[0, 1, 4, 5]]).all()
    assert same_bits(got, want)


def test_gemm_q4k_equals_repeated_gemv(ctx):
    """GEMM == n_act independent GEMVs bit for bit (kquant_gemm_parity.rs:129-160)."""
    print("[case] q4k gemm == repeated gemv", flush=True)
    m, n, k = 24, 96, 1024
    g = np.random.default_rng(9)
    a = g.standard_normal((m, k)).astype(np.float32)
    w = q4k_weights(0x99, n, k)
    full = ctx.gemm_q_f32(m, n, k, a, w, hip.WDtype.Q4_K)
    for i in range(m):
        one = ctx.gemm_q_f32(1, n, k, a[i:i + 1], w, hip.WDtype.Q4_K)
        assert same_bits(one[0], full[i])


def test_gemm_q4k_within_int8_bound(ctx, oracle):
    """|int8 - f64 dequant dot| <= 2 * int8_error_bound + f32 noise, per output."""
    print("[case] q4k gemm vs f64 bound", flush=True)
    m, n, k = 4, 32, 2048
    g = np.random.default_rng(11)
    a = g.standard_normal((m, k)).astype(np.float32)
    w = q4k_weights(0x1234, n, k)
    got = ctx.gemm_q_f32(m, n, k, a, w, hip.WDtype.Q4_K)
    deq = oracle.kquant_dequantize(W_Q4_K, w, n * k).reshape(n, k).astype(np.float64)
    exact = a.astype(np.float64) @ deq.T
    rb = (k // 256) * 144
    for i in range(m):
        for j in range(n):
            bound = oracle.int8_error_bound(W_Q4_K, w[j * rb:(j + 1) * rb], a[i])
            noise = 1e-5 * np.abs(a[i].astype(np.float64) * deq[j]).sum()
            assert abs(got[i, j] - exact[i, j]) <= 2 * bound + noise, (i, j)


def test_gemm_q4k_config4_shapes(ctx, oracle):
    """Speech-LLM decode (batch 32) linears at full size: q/o and gate/up/down."""
    for (n, k) in [(2048, 2048), (256, 2048), (5632, 2048), (2048, 5632)]:
        print(f"[case] q4k config4 n={n} k={k}", flush=True)
        m = 32
        g = np.random.default_rng(n + k)
        a = g.standard_normal((m, k)).astype(np.float32)
        w = q4k_weights(n ^ k, n, k)
        got = ctx.gemm_q_f32(m, n, k, a, w, hip.WDtype.Q4_K)
        rows = [0, 13, 31]
        want = oracle.gemm_q_f32(W_Q4_K, len(rows), n, k, a[rows], w)
        assert same_bits(got[rows], want)


def test_gemm_q4k_resident_and_qact(ctx, oracle):
    """Resident weight + separate activation pass == copy mode, and a second,
    smaller call on the same buffers is unaffected by the first."""
    print("[case] q4k resident/qact", flush=True)
    n, k = 160, 1536
    g = np.random.default_rng(21)
    w = q4k_weights(0x4242, n, k)
    W = ctx.upload_qweight(hip.WDtype.Q4_K, n, k, w)
    qa = ctx.qact(48, k)
    for m in (48, 5):
        a = g.standard_normal((m, k)).astype(np.float32)
        d_a = hip.DeviceBuffer.from_array(ctx, a)
        d_out = hip.DeviceBuffer(ctx, m * n * 4)
        qa.quantize(m, d_a, hip.ActQuant.KQUANT)
        ctx.gemm_qact_dev(W, qa, d_out)
        got = d_out.download(np.float32, m * n).reshape(m, n)
        want = oracle.gemm_q_f32(W_Q4_K, m, n, k, a, w)
        assert same_bits(got, want)
        d_out2 = hip.DeviceBuffer(ctx, m * n * 4)
        ctx.gemm_q_f32_dev(W, m, d_a, d_out2)   # act ignored for Q4_K
        assert same_bits(d_out2.download(np.float32, m * n).reshape(m, n), want)


def test_gemm_q4k_rejections(ctx):
    a = np.zeros((2, 512), np.float32)
    w = np.zeros(3 * 2 * 144, np.uint8)
    with pytest.raises(hip.InvalidArgument):
        ctx.gemm_q_f32(2, 3, 500, np.zeros((2, 500), np.float32), w, hip.WDtype.Q4_K)
    with pytest.raises(hip.InvalidArgument):
        ctx.gemm_q_f32(2, 3, 512, a, w[:-1], hip.WDtype.Q4_K)
    with pytest.raises(hip.InvalidArgument):
        ctx.gemm_q_f32(0, 3, 512, np.zeros((0, 512), np.float32), w, hip.WDtype.Q4_K)
    W = ctx.upload_qweight(hip.WDtype.Q4_K, 3, 512, w)
    qa = ctx.qact(2, 512)
    qa.quantize(2, hip.DeviceBuffer.from_array(ctx, a), hip.ActQuant.AMAX127)
    with pytest.raises(hip.InvalidArgument):
        ctx.gemm_qact_dev(W, qa, hip.DeviceBuffer(ctx, 2 * 3 * 4))
    W8 = ctx.upload_qweight(hip.WDtype.Q8_0, 3, 512, np.zeros(3 * 16 * 34, np.uint8))
    qa.quantize(2, hip.DeviceBuffer.from_array(ctx, a), hip.ActQuant.KQUANT)
    with pytest.raises(hip.InvalidArgument):
        ctx.gemm_qact_dev(W8, qa, hip.DeviceBuffer(ctx, 2 * 3 * 4))
