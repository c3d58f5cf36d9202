"""The oracle's Q5_K and Q6_K (the rest of the reference's KQuantDtype,
crates/vokra-backend-cpu/src/kernels/kquant.rs:56-63), pinned without it:
  * dequantize: the reference's own closed-form block tests
    (crates/vokra-core/src/gguf/quant/q5_k.rs:84-167, q6_k.rs:76-160) and an
    independent numpy parse of random blocks, bit for bit;
  * the INT8 route (unpack_block_i8, kquant.rs:332-407): GEMM == repeated GEMV
    (kquant_gemm_parity.rs:129-160), == an independent exact-integer route
    with the reference combine order in float32, and within 2x
    int8_error_bound of the f32 dequant-then-dot (kquant_gemm_parity.rs:
    204-236)."""
import numpy as np
import pytest

from tests.helpers import KQ_BLOCK_BYTES, Rng, hand_kquant_ints, random_kquant_blocks

W_Q5_K, W_Q6_K = 13, 14
F16_ONE, F16_HALF = 0x3C00, 0x3800


def pack_scales(sc, m):
    """q5_k.rs tests pack_scales: the inverse of get_scale_min_k4."""
    s = [0] * 12
    for j in range(8):
        if j < 4:
            s[j] = sc[j] & 63
            s[j + 4] = m[j] & 63
        else:
            s[j + 4] = (sc[j] & 0xF) | ((m[j] & 0xF) << 4)
            s[j - 4] |= (sc[j] >> 4) << 6
            s[j] |= (m[j] >> 4) << 6
    return bytes(s)


def q5k_block(d, dmin, scales, quants5):
    """q5_k.rs tests build_block: 256 chosen 5-bit quants."""
    qs, qh = bytearray(128), bytearray(32)
    for k in range(4):
        for l in range(32):
            lo, hi = quants5[64 * k + l], quants5[64 * k + 32 + l]
            qs[32 * k + l] = (lo & 0xF) | ((hi & 0xF) << 4)
            if lo & 0x10:
                qh[l] |= 1 << (2 * k)
            if hi & 0x10:
                qh[l] |= 1 << (2 * k + 1)
    return d.to_bytes(2, "little") + dmin.to_bytes(2, "little") + scales + bytes(qh) + bytes(qs)


def q6k_block(d, scales, quants):
    """q6_k.rs tests build_block: 256 signed quants in [-32, 31], 16 int8 scales."""
    ql, qh = bytearray(128), bytearray(64)
    for n, qn in enumerate(quants):
        half, o = divmod(n, 128)
        quarter, l = divmod(o, 32)
        stored = qn + 32
        low4, hi2 = stored & 0xF, (stored >> 4) & 3
        if quarter == 0:
            ql[64 * half + l] |= low4
            qh[32 * half + l] |= hi2
        elif quarter == 1:
            ql[64 * half + l + 32] |= low4
            qh[32 * half + l] |= hi2 << 2
        elif quarter == 2:
            ql[64 * half + l] |= low4 << 4
            qh[32 * half + l] |= hi2 << 4
        else:
            ql[64 * half + l + 32] |= low4 << 4
            qh[32 * half + l] |= hi2 << 6
    return bytes(ql) + bytes(qh) + bytes(np.array(scales, np.int8).view(np.uint8)) + d.to_bytes(2, "little")


def u8(b):
    return np.frombuffer(b, np.uint8).copy()


def test_q5k_closed_form_exercises_the_fifth_bit(oracle):
    sc, m = [1, 2, 3, 4, 5, 6, 7, 8], [2] * 8
    blk = q5k_block(F16_ONE, F16_HALF, pack_scales(sc, m), [i % 32 for i in range(256)])
    out = oracle.kquant_dequantize(W_Q5_K, u8(blk), 256)
    for n in range(256):
        k = n // 64
        sub = 2 * k if n % 64 < 32 else 2 * k + 1
        want = np.float32(np.float32(sc[sub]) * np.float32(n % 32)) - np.float32(0.5) * np.float32(m[sub])
        assert out[n] == want, n   # d = 1: every product and difference is exact


def test_q5k_max_quant_uses_high_bit(oracle):
    blk = q5k_block(F16_ONE, 0, pack_scales([1] * 8, [0] * 8), [31] * 256)
    assert np.all(oracle.kquant_dequantize(W_Q5_K, u8(blk), 256) == 31.0)


def test_q6k_closed_form_matches_signed_quants_and_scales(oracle):
    scales = [k - 8 for k in range(16)]
    quants = [(n % 64) - 32 for n in range(256)]
    out = oracle.kquant_dequantize(W_Q6_K, u8(q6k_block(F16_ONE, scales, quants)), 256)
    for n in range(256):
        half, o = divmod(n, 128)
        quarter, l = divmod(o, 32)
        idx = 8 * half + l // 16 + 2 * quarter
        assert out[n] == np.float32(scales[idx] * quants[n]), n


def test_q6k_zero_quant_and_negative_scale(oracle):
    assert np.all(oracle.kquant_dequantize(W_Q6_K, u8(q6k_block(F16_ONE, [1] * 16, [-32] * 256)), 256) == -32.0)
    assert np.all(oracle.kquant_dequantize(W_Q6_K, u8(q6k_block(F16_ONE, [-2] * 16, [16] * 256)), 256) == -32.0)


@pytest.mark.parametrize("wd", [W_Q5_K, W_Q6_K])
def test_dequant_matches_hand_parse(oracle, wd):
    rng = Rng(0x5600 + wd)
    w = random_kquant_blocks(rng, 40, wd)
    got = oracle.kquant_dequantize(wd, w, 40 * 256)
    q, d_eff, m_eff = hand_kquant_ints(w, wd)
    if wd == W_Q5_K:   # y = d_eff * q - m_eff, two roundings (q5_k.rs:63-70)
        want = (np.repeat(d_eff, 16, axis=1) * q.astype(np.float32)).astype(np.float32) - np.repeat(m_eff, 16, axis=1)
    else:              # y = (d * sc) * (q - 32) (q6_k.rs:64-67)
        want = (np.repeat(d_eff, 16, axis=1) * (q.astype(np.float32) - np.float32(32.0))).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.astype(np.float32).reshape(-1).view(np.uint32))


def _np_quant_act16(x):
    g = x.astype(np.float32).reshape(-1, 16)
    amax = np.abs(g).max(axis=1)
    s = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        r = np.where(s[:, None] > 0, g / s[:, None], 0).astype(np.float32)
    q = np.clip(np.sign(r) * np.floor(np.abs(r) + np.float32(0.5)), -127, 127).astype(np.int8)
    s = np.where(amax == 0, 0, s).astype(np.float32)
    return q.reshape(-1), s, q.astype(np.int32).sum(axis=1)


def int8_route(w, wd, x, m, k):
    """Exact integer group sums in int64, then the combine
    acc += s * (d_eff * isum - m_eff * gsum) in block-then-group order, f32."""
    nb = k // 256
    q, d_eff, m_eff = hand_kquant_ints(w, wd)
    q, d_eff, m_eff = q.reshape(m, nb, 256), d_eff.reshape(m, nb, 16), m_eff.reshape(m, nb, 16)
    qa, sa, ga = _np_quant_act16(x)
    out = np.zeros(m, np.float32)
    for i in range(m):
        acc = np.float32(0.0)
        for b in range(nb):
            isum = (q[i, b].astype(np.int64).reshape(16, 16) *
                    qa[b * 256:(b + 1) * 256].astype(np.int64).reshape(16, 16)).sum(axis=1)
            for g in range(16):
                t1 = np.float32(d_eff[i, b, g] * np.float32(isum[g]))
                t2 = np.float32(m_eff[i, b, g] * np.float32(ga[b * 16 + g]))
                acc = np.float32(acc + np.float32(sa[b * 16 + g] * np.float32(t1 - t2)))
        out[i] = acc
    return out


@pytest.mark.parametrize("wd", [W_Q5_K, W_Q6_K])
def test_int8_gemv_equals_independent_integer_route(oracle, wd):
    rng = Rng(0x5115_0033 + wd)
    m, k = 5, 512
    w = random_kquant_blocks(rng, m * (k // 256), wd)
    x = np.array(rng.vec(k), np.float32)
    got = oracle.kquant_gemv_i8(wd, m, k, w, x)
    assert np.array_equal(got.view(np.uint32), int8_route(w, wd, x, m, k).view(np.uint32))


@pytest.mark.parametrize("wd", [W_Q5_K, W_Q6_K])
def test_int8_gemm_equals_repeated_gemv_and_tracks_f32(oracle, wd):
    rng = Rng(0x5115_0031 + wd)
    for (m, n_act, k) in [(1, 1, 256), (3, 5, 512), (4, 3, 768)]:
        nb = k // 256
        w = random_kquant_blocks(rng, m * nb, wd)
        x = np.array(rng.vec(n_act * k), np.float32)
        gemm = oracle.kquant_gemm_i8(wd, m, k, n_act, w, x)
        rb = nb * KQ_BLOCK_BYTES[wd]
        for t in range(n_act):
            xt = x[t * k:(t + 1) * k]
            assert np.array_equal(gemm[t], oracle.kquant_gemv_i8(wd, m, k, w, xt))
            for i in range(m):
                row = w[i * rb:(i + 1) * rb]
                wf = oracle.kquant_dequantize(wd, row, k)
                f32_dot = np.add.accumulate((wf * xt).astype(np.float32), dtype=np.float32)[-1]
                bound = max(oracle.int8_error_bound(wd, row, xt), 1e-6)
                assert abs(gemm[t, i] - f32_dot) <= 2.0 * bound, (m, n_act, k, t, i)


def test_rejects_malformed(oracle):
    with pytest.raises(Exception):
        oracle.kquant_gemv_i8(W_Q6_K, 1, 256, np.zeros(209, np.uint8), np.zeros(256, np.float32))
    with pytest.raises(Exception):
        oracle.kquant_dequantize(W_Q5_K, np.zeros(175, np.uint8), 256)
