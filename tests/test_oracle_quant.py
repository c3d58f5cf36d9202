"""Pins the oracle's INT8 quantized matmuls (A8-A10 and the block-format
INT8 extension) with closed forms, exact integer brute force in numpy and the
reference's own internal-oracle rules:

  gguf/quant/q4_k.rs:71-177 (closed-form super-blocks),
  gguf/quant/mod.rs all_zero_kquant_blocks_decode_to_zeros,
  tests/kquant_gemm_parity.rs:129-236 (GEMM == repeated GEMV exactly; f32
  tracking within 2x int8_error_bound), convert/quantize.rs round trip.
"""
import numpy as np
import pytest

from tests.helpers import Rng, exact_fmaf, hand_q4k_ints, hand_qblock_ints, random_kquant_blocks


def pack_scales(sc, m):
    # q4_k.rs tests: pack_scales (inverse of get_scale_min_k4)
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


def build_block(d, dmin, scales, quants):
    qs = bytearray(128)
    for k in range(4):
        for l in range(32):
            qs[32 * k + l] = (quants[64 * k + l] & 0xF) | ((quants[64 * k + 32 + l] & 0xF) << 4)
    return np.frombuffer(d.to_bytes(2, "little") + dmin.to_bytes(2, "little") + scales + bytes(qs),
                         np.uint8)


def test_q4k_closed_form_distinct(oracle):
    sc = [1, 2, 3, 4, 5, 6, 7, 8]
    m = [8, 7, 6, 5, 4, 3, 2, 1]
    quants = [i % 16 for i in range(256)]
    blk = build_block(0x3C00, 0x3800, pack_scales(sc, m), quants)
    out = oracle.kquant_dequantize(12, blk, 256)
    for n in range(256):
        k = n // 64
        sub = 2 * k if n % 64 < 32 else 2 * k + 1
        want = 1.0 * sc[sub] * (n % 16) - 0.5 * m[sub]
        assert out[n] == np.float32(want)


def test_q4k_constant_and_two_blocks(oracle):
    blk = build_block(0x4000, 0x3C00, pack_scales([3] * 8, [5] * 8), [4] * 256)
    assert np.all(oracle.kquant_dequantize(12, blk, 256) == 19.0)
    b0 = build_block(0x3C00, 0, pack_scales([1] * 8, [0] * 8), [7] * 256)
    b1 = build_block(0x3C00, 0, pack_scales([2] * 8, [0] * 8), [3] * 256)
    out = oracle.kquant_dequantize(12, np.concatenate([b0, b1]), 512)
    assert np.all(out[:256] == 7.0) and np.all(out[256:] == 6.0)
    assert np.all(oracle.kquant_dequantize(12, np.zeros(144, np.uint8), 256) == 0.0)
    with pytest.raises(oracle.OracleError):
        oracle.kquant_dequantize(12, np.zeros(100, np.uint8), 256)


def test_q4k_dequant_matches_hand_parse(oracle):
    rng = Rng(0x4B)
    w = random_kquant_blocks(rng, 8)
    got = oracle.kquant_dequantize(12, w, 8 * 256)
    q, d_eff, m_eff = hand_q4k_ints(w)
    want = (d_eff.repeat(16, axis=-1) * q.astype(np.float32) - m_eff.repeat(16, axis=-1)).reshape(-1)
    assert np.array_equal(got, want.astype(np.float32))


def test_q4k_quantizer_round_trip(oracle):
    """convert/quantize.rs: uniform sc = m = 63, affine map step*q + base."""
    g = np.random.default_rng(3)
    x = (g.standard_normal(1024) * 0.02).astype(np.float32)
    w = oracle.kquant_quantize(12, x)
    assert w.size == 4 * 144
    assert np.all(w.reshape(4, 144)[:, 4:16] == 0xFF)
    y = oracle.kquant_dequantize(12, w, 1024)
    for b in range(4):
        blk = x[b * 256:(b + 1) * 256]
        step = (blk.max() - min(blk.min(), 0.0)) / 15.0
        assert np.abs(y[b * 256:(b + 1) * 256] - blk).max() <= 0.51 * step + 1e-3 * step


def test_kquant_activation_quantization(oracle):
    x = np.zeros(32, np.float32)
    x[:16] = np.linspace(-2, 1, 16)
    q, s, g = oracle.kquant_quantize_activations(x)
    assert s[1] == 0.0 and g[1] == 0 and np.all(q[16:] == 0)
    assert s[0] == np.float32(np.float32(2.0) / np.float32(127.0))
    assert q[0] == -127 and g[0] == int(q[:16].astype(np.int64).sum())
    assert np.abs(q.astype(np.int32)).max() <= 127


def _int8_ref_gemv(w, x, m, k):
    """Independent exact-integer route: numpy int64 group sums, then the
    reference combine order in float32 (kquant.rs:447-449, 590-629)."""
    nb = k // 256
    q, d_eff, m_eff = hand_q4k_ints(w)
    q, d_eff, m_eff = q.reshape(m, nb, 256), d_eff.reshape(m, nb, 16), m_eff.reshape(m, nb, 16)
    qa, sa, ga = _np_quant_act16(x)
    out = np.zeros(m, np.float32)
    for i in range(m):
        acc = np.float32(0.0)
        for b in range(nb):
            isum = (q[i, b].astype(np.int64).reshape(16, 16) *
                    qa[b * 256:(b + 1) * 256].astype(np.int64).reshape(16, 16)).sum(axis=1)
            for grp in range(16):
                t1 = np.float32(d_eff[i, b, grp] * np.float32(isum[grp]))
                t2 = np.float32(m_eff[i, b, grp] * np.float32(ga[b * 16 + grp]))
                acc = np.float32(acc + np.float32(sa[b * 16 + grp] * np.float32(t1 - t2)))
        out[i] = acc
    return out


def _np_quant_act16(x):
    x = x.astype(np.float32)
    g = x.reshape(-1, 16)
    amax = np.abs(g).max(axis=1)
    s = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        r = np.where(s[:, None] > 0, g / s[:, None], 0).astype(np.float32)
    q = np.clip(np.sign(r) * np.floor(np.abs(r) + np.float32(0.5)), -127, 127).astype(np.int8)
    s = np.where(amax == 0, 0, s).astype(np.float32)
    return q.reshape(-1), s, q.astype(np.int32).sum(axis=1)


def test_kquant_gemv_equals_independent_integer_route(oracle):
    rng = Rng(0x5115_0033)
    m, k = 6, 512
    w = random_kquant_blocks(rng, m * (k // 256))
    x = np.array(rng.vec(k), np.float32)
    got = oracle.kquant_gemv_i8(12, m, k, w, x)
    want = _int8_ref_gemv(w, x, m, k)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_kquant_gemm_equals_repeated_gemv(oracle):
    # kquant_gemm_parity.rs:129-160
    rng = Rng(0x5115_0031)
    for (m, n_act, k) in [(1, 1, 256), (3, 5, 512), (7, 2, 256), (4, 3, 768)]:
        w = random_kquant_blocks(rng, m * (k // 256))
        x = np.array(rng.vec(n_act * k), np.float32)
        gemm = oracle.kquant_gemm_i8(12, m, k, n_act, w, x)
        for t in range(n_act):
            gv = oracle.kquant_gemv_i8(12, m, k, w, x[t * k:(t + 1) * k])
            assert np.array_equal(gemm[t], gv)


def test_kquant_gemm_tracks_f32_within_derived_bound(oracle):
    # kquant_gemm_parity.rs:204-236
    rng = Rng(0x5115_0033)
    m, k, n_act = 6, 512, 3
    nb = k // 256
    w = random_kquant_blocks(rng, m * nb)
    x = np.array(rng.vec(n_act * k), np.float32)
    got = oracle.kquant_gemm_i8(12, m, k, n_act, w, x)
    rb = nb * 144
    for i in range(m):
        row = w[i * rb:(i + 1) * rb]
        wf = oracle.kquant_dequantize(12, row, k)
        for t in range(n_act):
            xt = x[t * k:(t + 1) * k]
            f32_dot = np.add.accumulate((wf * xt).astype(np.float32), dtype=np.float32)[-1]
            bound = max(oracle.int8_error_bound(12, row, xt), 1e-6)
            assert abs(got[t, i] - f32_dot) <= 2.0 * bound


def test_kquant_rejects_malformed(oracle):
    w = np.zeros(144, np.uint8)
    with pytest.raises(oracle.OracleError):
        oracle.kquant_gemm_i8(12, 1, 256, 0, w, np.zeros(0, np.float32))
    with pytest.raises(oracle.OracleError):
        oracle.kquant_gemv_i8(12, 1, 255, w, np.zeros(255, np.float32))
    with pytest.raises(oracle.OracleError):
        oracle.kquant_gemv_i8(12, 2, 256, w, np.zeros(256, np.float32))


def test_gemm_q_f32_bias_after(oracle):
    rng = Rng(11)
    m, n, k = 3, 4, 256
    w = random_kquant_blocks(rng, n)
    a = np.array(rng.vec(m * k), np.float32)
    bias = np.array(rng.vec(n), np.float32)
    nob = oracle.gemm_q_f32(12, m, n, k, a, w)
    wb = oracle.gemm_q_f32(12, m, n, k, a, w, bias)
    assert np.array_equal(wb, (nob + bias).astype(np.float32))


# ---- block-format INT8 (Q8_0 / Q4_0 / Q5_0 weights) ----------------------

@pytest.mark.parametrize("wd,mode", [(8, 3), (2, 1), (6, 2)])
def test_qblock_block_dots_exact_vs_numpy(oracle, wd, mode):
    g = np.random.default_rng(wd)
    m, n, k = 5, 7, 128
    w = (g.standard_normal((n, k)) * 0.02).astype(np.float32)
    wq = oracle.pack_matrix_to_bytes(mode, w, n, k // 32)
    a = g.standard_normal((m, k)).astype(np.float32)
    dots = oracle.qblock_block_dots(wd, m, n, k, a, wq)
    qw, dw = hand_qblock_ints(mode, wq, n, k)
    qa = np.stack([_np_quant_act32(a[i])[0] for i in range(m)])
    want = np.einsum("mbt,nbt->mnb", qa.reshape(m, k // 32, 32).astype(np.int64),
                     qw.reshape(n, k // 32, 32).astype(np.int64))
    assert np.array_equal(dots, want)


def _np_quant_act32(x):
    x = x.astype(np.float32)
    g = x.reshape(-1, 32)
    amax = np.abs(g).max(axis=1)
    s = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        r = np.where(s[:, None] > 0, g / s[:, None], 0).astype(np.float32)
    q = np.clip(np.sign(r) * np.floor(np.abs(r) + np.float32(0.5)), -127, 127).astype(np.int8)
    return q.reshape(-1), np.where(amax == 0, 0, s).astype(np.float32)


def test_quantize_act_b32_matches_numpy(oracle):
    g = np.random.default_rng(5)
    x = g.standard_normal(32 * 40).astype(np.float32)
    x[64:96] = 0.0
    q, s, gs = oracle.quantize_act_b32(x)
    q2, s2 = _np_quant_act32(x)
    assert np.array_equal(q, q2) and np.array_equal(s, s2)
    assert np.array_equal(gs, q.astype(np.int32).reshape(-1, 32).sum(axis=1))


@pytest.mark.parametrize("wd,mode", [(8, 3), (2, 1), (6, 2)])
def test_qblock_gemm_combine_and_bound(oracle, wd, mode):
    """f32 output = fmaf-combine of the exact block dots in block order, and
    within 2x the activation-rounding bound of the f32 dequant GEMV oracle."""
    g = np.random.default_rng(100 + wd)
    m, n, k = 4, 6, 256
    w = (g.standard_normal((n, k)) * 0.02).astype(np.float32)
    wq = oracle.pack_matrix_to_bytes(mode, w, n, k // 32)
    a = g.standard_normal((m, k)).astype(np.float32)
    bias = g.standard_normal(n).astype(np.float32)
    out = oracle.gemm_qblock_i8(wd, m, n, k, a, wq, bias)
    dots = oracle.qblock_block_dots(wd, m, n, k, a, wq)
    _, dw = hand_qblock_ints(mode, wq, n, k)
    nb = k // 32
    for i in range(m):
        _, sa = _np_quant_act32(a[i])
        for j in range(n):
            acc = np.float32(0.0)
            for b in range(nb):
                prod = np.float32(sa[b] * dw[j, b])
                acc = exact_fmaf(prod, np.float32(dots[i, j, b]), acc)
            assert out[i, j] == np.float32(acc + bias[j])
    rb = nb * oracle.KV_BLOCK_BYTES[mode]
    f32ref = np.stack([oracle.dequant_gemv_scalar(mode, wq, n, nb, a[i]) for i in range(m)])
    for i in range(m):
        for j in range(n):
            bound = oracle.qblock_error_bound(wd, wq[j * rb:(j + 1) * rb], a[i])
            assert abs((out[i, j] - bias[j]) - f32ref[i, j]) <= 2 * bound + 1e-6
