"""GPU parity of Q5_K and Q6_K, the rest of the reference's KQuantDtype
(crates/vokra-backend-cpu/src/kernels/kquant.rs:56-63), against the oracle
through the C ABI.

Bars (as for Q4_K):
  * kquant_dequantize: bit-exact (every f16 pattern of the super-block
    scales included), and against an independent numpy parse;
  * gemm_q_f32: bit-exact f32 outputs (unpack_block_i8's unified INT8 form,
    kquant.rs:332-407: exact integer group sums, then the reference combine
    in block-then-group order), GEMM == repeated GEMV, and within 2x
    int8_error_bound of an f64 dequant-then-dot;
  * a text-decoder session over Q5_K / Q6_K linears: the step == the entry
    points one at a time, bit for bit (test_gpu_textdec.py).
"""
import numpy as np
import pytest

from tests.helpers import KQ_BLOCK_BYTES, Rng, hand_kquant_ints, random_kquant_blocks
from vokra_amd import hip

pytestmark = pytest.mark.gpu

W_Q5_K, W_Q6_K = 13, 14
DT = {W_Q5_K: hip.WDtype.Q5_K, W_Q6_K: hip.WDtype.Q6_K}


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


def weights(wd, seed, n, k):
    return random_kquant_blocks(Rng(seed), n * (k // 256), wd)


@pytest.mark.parametrize("wd", [W_Q5_K, W_Q6_K])
def test_dequantize_random_and_hand_parse(ctx, oracle, wd):
    print(f"[case] kquant {wd} dequantize", flush=True)
    w = weights(wd, 0x51 + wd, 300, 256)
    got = ctx.kquant_dequantize(DT[wd], w, 300 * 256)
    assert same_bits(got, oracle.kquant_dequantize(wd, w, 300 * 256))
    q, d_eff, m_eff = hand_kquant_ints(w, wd)
    if wd == W_Q5_K:
        want = (np.repeat(d_eff, 16, axis=1) * q.astype(np.float32)).astype(np.float32) - np.repeat(m_eff, 16, axis=1)
    else:
        want = (np.repeat(d_eff, 16, axis=1) * (q.astype(np.float32) - np.float32(32.0))).astype(np.float32)
    assert same_bits(got.reshape(300, 256), want)


@pytest.mark.parametrize("wd", [W_Q5_K, W_Q6_K])
def test_dequantize_every_scale_pattern(ctx, oracle, wd):
    """All 65536 f16 bit patterns of d (and of dmin for Q5_K): subnormals,
    inf and NaN land where the reference puts them."""
    print(f"[case] kquant {wd} dequantize all scale patterns", flush=True)
    bb = KQ_BLOCK_BYTES[wd]
    g = np.random.default_rng(4 + wd)
    blocks = g.integers(0, 256, size=(65536, bb), dtype=np.uint8)
    pat = np.arange(65536)
    if wd == W_Q5_K:
        blocks[:, 0], blocks[:, 1] = pat & 0xFF, pat >> 8
        perm = g.permutation(65536)
        blocks[:, 2], blocks[:, 3] = perm & 0xFF, perm >> 8
    else:
        blocks[:, 208], blocks[:, 209] = pat & 0xFF, pat >> 8
    got = ctx.kquant_dequantize(DT[wd], blocks.reshape(-1), 65536 * 256)
    assert same_bits(got, oracle.kquant_dequantize(wd, blocks.reshape(-1), 65536 * 256))


def test_dequantize_rejections(ctx):
    with pytest.raises(hip.InvalidArgument):
        ctx.kquant_dequantize(hip.WDtype.Q5_K, np.zeros(175, np.uint8), 256)
    with pytest.raises(hip.InvalidArgument):
        ctx.kquant_dequantize(hip.WDtype.Q6_K, np.zeros(210, np.uint8), 255)


GEMM_SHAPES = [(1, 16, 256), (1, 37, 512), (3, 64, 768), (17, 100, 768), (32, 48, 1024), (64, 80, 512),
               (130, 20, 256)]


@pytest.mark.parametrize("wd", [W_Q5_K, W_Q6_K])
@pytest.mark.parametrize("m,n,k", GEMM_SHAPES)
def test_gemm_bit_exact(ctx, oracle, wd, m, n, k):
    print(f"[case] kquant {wd} gemm m={m} n={n} k={k}", flush=True)
    g = np.random.default_rng(m * 1000 + n + k + wd)
    a = g.standard_normal((m, k)).astype(np.float32)
    a[0, :16] = 0.0                       # an all-zero group: scale 0, gsum 0
    w = weights(wd, m * 7 + n, n, k)
    bias = g.standard_normal(n).astype(np.float32) if m % 2 else None
    got = ctx.gemm_q_f32(m, n, k, a, w, DT[wd], bias=bias)
    assert same_bits(got, oracle.gemm_q_f32(wd, m, n, k, a, w, bias))


@pytest.mark.parametrize("wd", [W_Q5_K, W_Q6_K])
def test_gemm_equals_repeated_gemv_and_bound(ctx, oracle, wd):
    print(f"[case] kquant {wd} gemm == gemv, bound", flush=True)
    m, n, k = 12, 40, 1024
    g = np.random.default_rng(9 + wd)
    a = g.standard_normal((m, k)).astype(np.float32)
    w = weights(wd, 0x99 + wd, n, k)
    full = ctx.gemm_q_f32(m, n, k, a, w, DT[wd])
    for i in range(m):
        assert same_bits(ctx.gemm_q_f32(1, n, k, a[i:i + 1], w, DT[wd])[0], full[i])
    deq = oracle.kquant_dequantize(wd, w, n * k).reshape(n, k).astype(np.float64)
    exact = a.astype(np.float64) @ deq.T
    rb = (k // 256) * KQ_BLOCK_BYTES[wd]
    for i in range(0, m, 5):
        for j in range(n):
            bound = oracle.int8_error_bound(wd, w[j * rb:(j + 1) * rb], a[i])
            noise = 1e-5 * np.abs(a[i].astype(np.float64) * deq[j]).sum()
            assert abs(full[i, j] - exact[i, j]) <= 2 * bound + noise, (i, j)


@pytest.mark.parametrize("wd", [W_Q5_K, W_Q6_K])
def test_gemm_config4_shapes(ctx, oracle, wd):
    """Speech-LLM linears (batch 32) at full size, resident weights."""
    for (n, k) in [(2048, 2048), (5632, 2048), (2048, 5632)]:
        print(f"[case] kquant {wd} config4 n={n} k={k}", flush=True)
        m = 32
        g = np.random.default_rng(n + k + wd)
        a = g.standard_normal((m, k)).astype(np.float32)
        w = weights(wd, n ^ k, n, k)
        W = ctx.upload_qweight(DT[wd], n, k, w)
        d_a = hip.DeviceBuffer.from_array(ctx, a)
        d_out = hip.DeviceBuffer(ctx, m * n * 4)
        ctx.gemm_q_f32_dev(W, m, d_a, d_out)
        got = d_out.download(np.float32, m * n).reshape(m, n)
        rows = [0, 31]
        assert same_bits(got[rows], oracle.gemm_q_f32(wd, len(rows), n, k, a[rows], w))
