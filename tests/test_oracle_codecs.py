"""Pins the oracle's codecs (A1-A7) against the reference's own unit-test
vectors and against independent routines (numpy float16, hand-parsed bytes).

Reference tests restated here:
  kv_quant/half.rs:153-218, gguf/quant/mod.rs tests, kv_quant/q8_0.rs:90-169,
  kv_quant/q4_0.rs:107-197, kv_quant/q5_0.rs tests, kv_quant/mod.rs tests,
  kv_quant/dequant_gemm.rs:229-351, kv_quant/gpu_ops.rs:133-193.
"""
import math
import struct

import numpy as np
import pytest


def f32(x):
    return struct.unpack("<f", struct.pack("<f", x))[0]


# ---- A1 binary16 ---------------------------------------------------------

def test_half_known_values_round_trip(oracle):
    # half.rs known_positive_values_round_trip
    for x in [1.0, 2.0, -2.0, 0.5, 0.25, 3.25, 65504.0, -65504.0]:
        assert oracle.f16_bits_to_f32(oracle.f32_to_f16_bits(x)) == x


def test_half_corners(oracle):
    # half.rs zero_signs / overflow / underflow / nan / subnormal / RNE
    assert oracle.f32_to_f16_bits(0.0) == 0
    assert oracle.f32_to_f16_bits(-0.0) == 0x8000
    assert oracle.f32_to_f16_bits(1.0e5) == 0x7C00
    assert oracle.f32_to_f16_bits(-1.0e5) == 0xFC00
    assert oracle.f32_to_f16_bits(math.inf) == 0x7C00
    assert oracle.f32_to_f16_bits(1.0e-10) == 0
    assert oracle.f32_to_f16_bits(-1.0e-10) == 0x8000
    n = oracle.f32_to_f16_bits(math.nan)
    assert (n >> 10) & 0x1F == 0x1F and n & 0x3FF != 0
    assert math.isnan(oracle.f16_bits_to_f32(n))
    sub = 2.0 ** -24
    assert oracle.f16_bits_to_f32(oracle.f32_to_f16_bits(sub)) == sub
    x = struct.unpack("<f", struct.pack("<I", 0x3F800800))[0]
    assert oracle.f32_to_f16_bits(x) & 0x3FF == 0


def test_gguf_f16_known_values(oracle):
    # gguf/quant/mod.rs f16_to_f32_matches_known_values
    assert oracle.gguf_f16_to_f32(0x3C00) == 1.0
    assert oracle.gguf_f16_to_f32(0x4000) == 2.0
    assert oracle.gguf_f16_to_f32(0xC000) == -2.0
    assert oracle.gguf_f16_to_f32(0x0000) == 0.0
    assert oracle.gguf_f16_to_f32(0x3800) == 0.5
    assert oracle.gguf_f16_to_f32(0x0001) == 2.0 ** -24
    assert math.isinf(oracle.gguf_f16_to_f32(0x7C00))
    assert math.isnan(oracle.gguf_f16_to_f32(0x7E00))


def test_f16_decode_exhaustive_vs_numpy(oracle):
    """All 65,536 bit patterns against numpy's IEEE binary16 (independent)."""
    bits = np.arange(65536, dtype=np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_bits_to_f32(int(b)) for b in bits], np.float32)
    got2 = np.array([oracle.gguf_f16_to_f32(int(b)) for b in bits], np.float32)
    fin = np.isfinite(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))
    assert np.array_equal(got2[fin].view(np.uint32), want[fin].view(np.uint32))
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(np.isinf(got), np.isinf(want))


def test_f16_encode_vs_numpy_rne(oracle):
    """f32 -> f16 RNE on every half's neighbourhood (midpoints included) and
    random f32 across the whole range, against numpy's float16 cast."""
    rng = np.random.default_rng(7)
    halves = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float32)
    mids = []
    h = np.arange(0, 0x7BFF, dtype=np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).astype(np.uint16).view(np.float16).astype(np.float64)
    mids = ((lo + hi) / 2).astype(np.float32)  # exact midpoints are f32-representable
    rnd = rng.standard_normal(20000).astype(np.float32) * np.float32(1e3)
    tiny = rng.standard_normal(20000).astype(np.float32) * np.float32(1e-6)
    xs = np.concatenate([halves, mids, np.nextafter(mids, np.float32(np.inf)),
                         np.nextafter(mids, np.float32(-np.inf)), rnd, tiny])
    xs = np.concatenate([xs, -xs])
    want = xs.astype(np.float16).view(np.uint16)
    enc1 = np.array([oracle.f32_to_f16_bits(float(x)) for x in xs], np.uint16)
    enc2 = np.array([oracle.convert_f32_to_f16(float(x)) for x in xs], np.uint16)
    assert np.array_equal(enc1, want)
    assert np.array_equal(enc2, want)


# ---- A2/A3 block codecs ---------------------------------------------------

RAMP = np.array([(i / 31.0) * 2.0 - 1.0 for i in range(32)], np.float32)


@pytest.mark.parametrize("mode,div", [(3, 127.0), (1, 7.0), (2, 15.0)])
def test_round_trip_within_quantization_step(oracle, mode, div):
    # q8_0.rs / q4_0.rs / q5_0.rs round_trip_within_quantization_step
    blk = oracle.pack_block(mode, RAMP)
    out = oracle.unpack_block(mode, blk)
    amax = np.abs(RAMP).max()
    tol = np.float32(0.6) * np.float32(amax / np.float32(div))
    assert np.all(np.abs(RAMP - out) <= tol)


@pytest.mark.parametrize("mode", [1, 2, 3])
def test_all_zeros_round_trip_exactly(oracle, mode):
    blk = oracle.pack_block(mode, np.zeros(32, np.float32))
    assert blk[0] == 0 and blk[1] == 0
    assert np.all(oracle.unpack_block(mode, blk) == 0.0)


def test_saturation_at_range_edges(oracle):
    x = np.zeros(32, np.float32)
    x[0], x[1] = 1000.0, -1000.0
    q8 = oracle.pack_block(3, x)
    assert q8[2] == 127 and q8[3].astype(np.int8) == -127
    q4 = oracle.pack_block(1, x)
    assert q4[2] & 0x0F == 15 and (q4[2] >> 4) & 0x0F == 1
    q5 = oracle.pack_block(2, x)
    b0 = (q5[6] & 0x0F) | ((q5[2] & 1) << 4)
    b1 = ((q5[6] >> 4) & 0x0F) | (((q5[2] >> 1) & 1) << 4)
    assert b0 == 31 and b1 == 1
    # q4_0.rs negative_bias_reaches_lowest_sentinel
    y = np.zeros(32, np.float32)
    y[0], y[1] = -1000.0, 500.0
    assert oracle.pack_block(1, y)[2] & 0x0F == 1


def test_block_sizes(oracle):
    assert [oracle.lib().vo_kv_block_bytes(m) for m in (0, 1, 2, 3)] == [128, 18, 22, 34]


def test_precision_ordering(oracle):
    outs = {m: oracle.unpack_block(m, oracle.pack_block(m, RAMP)) for m in (1, 2, 3)}
    sse = {m: float(((RAMP - o) ** 2).sum()) for m, o in outs.items()}
    assert sse[3] <= sse[2] <= sse[1]


def _hand_decode(mode, blk):
    """Independent wire-format parse (numpy float16 for the scale)."""
    d = np.frombuffer(bytes(blk[:2]), np.float16)[0].astype(np.float32)
    if mode == 3:
        q = np.frombuffer(bytes(blk[2:34]), np.int8).astype(np.float32)
    elif mode == 1:
        b = np.asarray(blk[2:18], np.int32)
        q = np.empty(32, np.float32)
        q[0::2] = (b & 0xF) - 8
        q[1::2] = (b >> 4) - 8
    else:
        qh = int.from_bytes(bytes(blk[2:6]), "little")
        b = np.asarray(blk[6:22], np.int32)
        lo = np.empty(32, np.int32)
        lo[0::2] = b & 0xF
        lo[1::2] = b >> 4
        hi = np.array([(qh >> i) & 1 for i in range(32)], np.int32)
        q = ((hi << 4) | lo).astype(np.float32) - 16
    return q * d


@pytest.mark.parametrize("mode", [1, 2, 3])
def test_dequantize_matches_hand_parse(oracle, mode):
    rng = np.random.default_rng(mode)
    x = (rng.standard_normal(32 * 64) * 0.5).astype(np.float32)
    data = oracle.pack_matrix_to_bytes(mode, x, 64, 1)
    got = oracle.dequantize_bytes(mode, data)
    bb = oracle.KV_BLOCK_BYTES[mode]
    want = np.concatenate([_hand_decode(mode, data[i * bb:(i + 1) * bb]) for i in range(64)])
    assert np.array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32))


def test_dequantize_rejects(oracle):
    with pytest.raises(oracle.OracleError):
        oracle.dequantize_bytes(0, np.zeros(128, np.uint8))
    with pytest.raises(oracle.OracleError):
        oracle.dequantize_bytes(3, np.zeros(33, np.uint8))


# ---- A6/A7 dequant GEMV ---------------------------------------------------

def _make_shape():
    # dequant_gemm.rs:233-246 make_shape
    n_rows, n_bpr = 4, 2
    per_row = 64
    a = np.array([(i / (n_rows * per_row)) * 2.0 - 1.0 for i in range(n_rows * per_row)],
                 np.float32)
    x = np.array([math.sin(i / per_row) for i in range(per_row)], np.float32)
    return a, x, n_rows, n_bpr


def test_two_stage_bit_identical(oracle):
    """dequant_gemm.rs two_stage_bit_identical_to_fused_scalar, with the second
    stage computed independently by numpy's sequential float32 accumulate."""
    a, x, n_rows, n_bpr = _make_shape()
    for mode in (1, 2, 3):
        data = oracle.pack_matrix_to_bytes(mode, a, n_rows, n_bpr)
        fused = oracle.dequant_gemv_scalar(mode, data, n_rows, n_bpr, x)
        deq = oracle.dequantize_bytes(mode, data).reshape(n_rows, -1)
        seq = np.add.accumulate((deq * x).astype(np.float32), axis=1, dtype=np.float32)[:, -1]
        assert np.array_equal(fused.view(np.uint32), seq.view(np.uint32))
        assert np.array_equal(fused, oracle.dense_gemv_f32(deq, n_rows, x))


def test_q8_0_gemv_within_bound_vs_fp32(oracle):
    a, x, n_rows, n_bpr = _make_shape()
    y32 = oracle.dense_gemv_f32(a, n_rows, x)
    data = oracle.pack_matrix_to_bytes(3, a, n_rows, n_bpr)
    y8 = oracle.dequant_gemv_scalar(3, data, n_rows, n_bpr, x)
    tol = (np.abs(a).max() / 127.0 * 0.5) * 64 * np.abs(x).max() * 1.5
    assert np.all(np.abs(y32 - y8) <= tol)


def test_gemv_precision_ordering(oracle):
    a, x, n_rows, n_bpr = _make_shape()
    y32 = a.reshape(n_rows, -1).astype(np.float64) @ x.astype(np.float64)
    sse = []
    for mode in (1, 2, 3):
        data = oracle.pack_matrix_to_bytes(mode, a, n_rows, n_bpr)
        y = oracle.dequant_gemv_scalar(mode, data, n_rows, n_bpr, x)
        sse.append(float(((y32 - y) ** 2).sum()))
    assert sse[2] <= sse[1] <= sse[0]


def test_validate_dequant_gemv(oracle):
    # gpu_ops.rs:133-193
    assert oracle.validate_dequant_gemv(0, 0, 0, 0, 0) == oracle.INVALID_ARGUMENT
    assert oracle.validate_dequant_gemv(3, 4 * 2 * 34, 4, 2, 63) == oracle.INVALID_ARGUMENT
    assert oracle.validate_dequant_gemv(3, 100, 4, 2, 64) == oracle.INVALID_ARGUMENT
    assert oracle.validate_dequant_gemv(1, 144, 4, 2, 64) == oracle.OK
    assert oracle.validate_dequant_gemv(2, 176, 4, 2, 64) == oracle.OK
    assert oracle.validate_dequant_gemv(3, 272, 4, 2, 64) == oracle.OK


def test_rand_vec_matches_independent_xorshift(oracle):
    """parity_kernels_cuda.rs:23-34 rand_vec, re-derived in Python integers."""
    for seed in (0xD3 ^ (16 * 131 + 2), 0xE5 ^ 64, 0):
        x = seed | 1
        want = []
        for _ in range(50):
            x ^= x >> 12
            x ^= (x << 25) & 0xFFFFFFFFFFFFFFFF
            x ^= x >> 27
            bits = ((x * 0x2545F4914F6CDD1D) & 0xFFFFFFFFFFFFFFFF) >> 40
            want.append(f32(f32(f32(bits / float(1 << 24)) * 2.0) - 1.0))
        got = oracle.xorshift_rand_vec(seed, 50)
        assert np.array_equal(got, np.array(want, np.float32))


def test_splitmix_gaussian_matches_independent(oracle):
    """rng/mod.rs:111-175 SplitMix64 + Box-Muller, re-derived in Python."""
    M = 0xFFFFFFFFFFFFFFFF
    state = 1234
    out = []
    while len(out) < 20:
        us = []
        for _ in range(2):
            state = (state + 0x9E3779B97F4A7C15) & M
            z = state
            z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M
            z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M
            z ^= z >> 31
            us.append((np.float32(z >> 40) + np.float32(0.5)) / np.float32(1 << 24))
        r = np.sqrt(np.float32(-2.0) * np.log(us[0]))
        th = np.float32(2.0 * np.float32(np.pi)) * us[1]
        out += [r * np.cos(th), r * np.sin(th)]
    got = oracle.splitmix_gaussian(1234, 20)
    # libm vs numpy transcendental may differ in the last ulp
    assert np.allclose(got, np.array(out, np.float32), rtol=1e-6, atol=1e-7)
    assert abs(float(got.astype(np.float64).mean())) < 1.0


def test_argmax_first_max_wins(oracle):
    assert oracle.argmax(np.array([1.0, 3.0, 3.0, 2.0], np.float32)) == 1
    assert oracle.argmax(np.array([-np.inf, -np.inf], np.float32)) == 0
    assert oracle.argmax(np.array([np.nan, 1.0, np.nan, 1.0], np.float32)) == 1
