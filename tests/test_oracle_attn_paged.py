"""Pins the oracle's f32 kernels (A11, A12), attention (A13, A14) and the
quantized paged KV cache (A15).

Reference tests restated: kernels/scalar.rs:224-330, cache/paged_quant.rs:
559-843; attention is pinned by invariants (uniform keys -> mean of V, rows
sum to one, causal mask) and float64 brute force on small shapes.
"""
import math

import numpy as np
import pytest


def test_scalar_kernels_reference_values(oracle):
    # scalar.rs erf_matches_reference_values
    for x, want in [(0.0, 0.0), (0.5, 0.5204999), (1.0, 0.8427008), (2.0, 0.9953223),
                    (-1.0, -0.8427008)]:
        assert abs(oracle.erf_as(x) - want) < 1e-5
    # A&S 7.1.26 stays within its published 1.5e-7 of the true erf
    for x in np.linspace(-4, 4, 81):
        assert abs(oracle.erf_as(float(x)) - math.erf(float(np.float32(x)))) < 5e-7
    g = oracle.gelu_f32(np.array([0.0, 1.0, -1.0], np.float32))
    assert abs(g[0]) < 1e-6 and abs(g[1] - 0.841192) < 1e-3 and -0.2 < g[2] < 0.0
    out = oracle.gemm_f32(2, 2, 2, [1, 0, 0, 1], [1, 2, 3, 4], [10, 20])
    assert out.reshape(-1).tolist() == [11.0, 22.0, 13.0, 24.0]
    assert oracle.gemm_f32(1, 1, 3, [1, 2, 3], [1, 0, -1]).reshape(-1).tolist() == [-2.0]
    a = np.array([1, 2, 3, 4, 5, 6], np.float32)
    assert oracle.gemv_f32(2, 3, a, [1, 0, -1]).tolist() == [-2.0, -2.0]
    assert oracle.gemv_f32(2, 3, a, [1, 0, -1], [10, 20]).tolist() == [8.0, 18.0]
    a2 = np.array([0.5, -1.5, 2.25, -0.75, 3.0, 0.125], np.float32)
    x2 = np.array([1.25, -0.5, 0.75], np.float32)
    assert np.array_equal(oracle.gemm_f32(2, 1, 3, a2, x2).reshape(-1), oracle.gemv_f32(2, 3, a2, x2))
    s = oracle.softmax_f32([1.0, 2.0, 3.0, 4.0], 1, 4)
    assert abs(s.sum() - 1.0) < 1e-6
    s2 = oracle.softmax_f32([101.0, 102.0, 103.0, 104.0], 1, 4)
    assert np.allclose(s, s2, atol=1e-6)


def test_gemm_threads_bit_identical(oracle):
    g = np.random.default_rng(0)
    a = g.standard_normal((37, 19)).astype(np.float32)
    b = g.standard_normal((19, 23)).astype(np.float32)
    bias = g.standard_normal(23).astype(np.float32)
    one = oracle.gemm_f32(37, 23, 19, a, b, bias, threads=1)
    many = oracle.gemm_f32(37, 23, 19, a, b, bias, threads=5)
    assert np.array_equal(one, many)
    assert np.allclose(one, a.astype(np.float64) @ b + bias, rtol=1e-5, atol=1e-5)


def test_layer_norm_invariants(oracle):
    g = np.random.default_rng(1)
    gamma = g.standard_normal(64).astype(np.float32)
    beta = g.standard_normal(64).astype(np.float32)
    const = np.full((3, 64), 2.5, np.float32)
    assert np.array_equal(oracle.layer_norm_f32(const, 3, 64, gamma, beta), np.tile(beta, (3, 1)))
    x = g.standard_normal((5, 64)).astype(np.float32)
    got = oracle.layer_norm_f32(x, 5, 64, gamma, beta)
    x64 = x.astype(np.float64)
    mu = x64.mean(1, keepdims=True)
    want = (x64 - mu) / np.sqrt(((x64 - mu) ** 2).mean(1, keepdims=True) + 1e-5) * gamma + beta
    assert np.allclose(got, want, rtol=1e-5, atol=1e-5)
    r = oracle.rms_norm_f32(x, gamma, 1e-6, 5, 64)
    want_r = x64 / np.sqrt((x64 ** 2).mean(1, keepdims=True) + 1e-6) * gamma
    assert np.allclose(r, want_r, rtol=1e-5, atol=1e-5)


def _sdpa64(q, k, v, n_head, hd, scale, causal, q_off, scale_on_q=True):
    t_q, t_kv = q.shape[0], k.shape[0]
    out = np.zeros((t_q, n_head * hd))
    for h in range(n_head):
        sl = slice(h * hd, (h + 1) * hd)
        s = (q[:, sl].astype(np.float64) @ k[:, sl].T.astype(np.float64)) * scale
        if causal:
            for i in range(t_q):
                s[i, q_off + i + 1:] = -np.inf
        p = np.exp(s - s.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        out[:, sl] = p @ v[:, sl]
    return out


@pytest.mark.parametrize("t_q,t_kv,n_head,hd,causal,q_off",
                         [(3, 7, 2, 64, False, 0), (1, 9, 4, 64, True, 8), (5, 5, 3, 32, True, 0),
                          (2, 40, 2, 128, False, 0)])
def test_sdpa_whisper_vs_float64(oracle, t_q, t_kv, n_head, hd, causal, q_off):
    g = np.random.default_rng(t_q * 100 + t_kv)
    d = n_head * hd
    q = g.standard_normal((t_q, d)).astype(np.float32)
    k = g.standard_normal((t_kv, d)).astype(np.float32)
    v = g.standard_normal((t_kv, d)).astype(np.float32)
    got = oracle.sdpa_whisper(t_q, t_kv, n_head, hd, q, k, v, causal, q_off)
    want = _sdpa64(q, k, v, n_head, hd, hd ** -0.5, causal, q_off)
    assert np.allclose(got, want, rtol=1e-4, atol=1e-5)


def test_sdpa_uniform_keys_give_mean_of_v(oracle):
    g = np.random.default_rng(9)
    t_kv, d = 11, 2 * 64
    q = g.standard_normal((2, d)).astype(np.float32)
    k = np.tile(g.standard_normal((1, d)).astype(np.float32), (t_kv, 1))
    v = g.standard_normal((t_kv, d)).astype(np.float32)
    got = oracle.sdpa_whisper(2, t_kv, 2, 64, q, k, v)
    assert np.allclose(got, np.tile(v.astype(np.float64).mean(0), (2, 1)), atol=1e-5)
    # causal with offset 0: query 0 sees only key 0
    got_c = oracle.sdpa_whisper(1, t_kv, 2, 64, q[:1], k, v, True, 0)
    assert np.array_equal(got_c[0], v[0])


def test_gqa_attention_vs_float64(oracle):
    g = np.random.default_rng(4)
    t, t_kv, hq, hk, hd = 2, 13, 8, 2, 32
    q = g.standard_normal((t, hq * hd)).astype(np.float32)
    k = g.standard_normal((t_kv, hk * hd)).astype(np.float32)
    v = g.standard_normal((t_kv, hk * hd)).astype(np.float32)
    scale = float(np.float32(hd ** -0.5))
    got = oracle.gqa_attention(t, t_kv, hq, hk, hd, q, k, v, scale, t_kv - t)
    kx = np.repeat(k.reshape(t_kv, hk, hd), hq // hk, axis=1).reshape(t_kv, -1)
    vx = np.repeat(v.reshape(t_kv, hk, hd), hq // hk, axis=1).reshape(t_kv, -1)
    want = _sdpa64(q, kx, vx, hq, hd, scale, True, t_kv - t)
    assert np.allclose(got, want, rtol=1e-4, atol=1e-5)


# ---- A15 quantized paged KV cache (paged_quant.rs tests) ----------------

def test_paged_rejections(oracle):
    with pytest.raises(oracle.OracleError):
        oracle.PagedCache(1, 1, 32, 1, 4, 4, oracle.FP32)
    with pytest.raises(oracle.OracleError):
        oracle.PagedCache(1, 1, 33, 1, 4, 4, oracle.Q8_0)
    with pytest.raises(oracle.OracleError):
        oracle.PagedCache(0, 1, 32, 1, 4, 4, oracle.Q8_0)
    c = oracle.PagedCache(1, 1, 32, 1, 4, 4, oracle.Q8_0)
    assert c.free_pages() == 1 and c.pages_in_use() == 0
    assert c.read_step(0, 0, 0) is None
    assert c.read_step(1, 0, 0) is None and c.read_step(0, 4, 0) is None
    assert c.append_step(0, 0, 0, np.zeros(32, np.float32), np.zeros(32, np.float32)) == oracle.OK
    assert c.append_step(1, 0, 0, np.zeros(32), np.zeros(32)) == oracle.INVALID_ARGUMENT


def test_paged_round_trip_q8_0(oracle):
    c = oracle.PagedCache(1, 1, 64, 1, 4, 4, oracle.Q8_0)
    k = np.array([(i / 63.0) * 2 - 1 for i in range(64)], np.float32)
    v = np.array([((63 - i) / 63.0) * 2 - 1 for i in range(64)], np.float32)
    assert c.append_step(0, 0, 0, k, v) == oracle.OK
    ko, vo = c.read_step(0, 0, 0)
    tol = 0.6 * (np.abs(k).max() / 127.0)
    assert np.all(np.abs(ko - k) <= tol) and np.all(np.abs(vo - v) <= tol)
    # numerics are the per-row Q8_0 codec, independent of the page layout
    assert np.array_equal(ko, oracle.dequantize_bytes(3, oracle.pack_matrix_to_bytes(3, k, 1, 2)))


def test_paged_allocator_lifo_and_exhaustion(oracle):
    c = oracle.PagedCache(2, 2, 32, 1, 8, 2, oracle.Q8_0)   # 4 pages/layer, 8 pages
    row = np.ones(64, np.float32)
    order = []
    for t in range(8):
        assert c.append_step(0, t, 0, row, row) == oracle.OK
        order.append(c.page_of(0, t))
    assert order == [0, 0, 1, 1, 2, 2, 3, 3]
    assert c.pages_in_use() == 4
    assert c.release_layer(0) == oracle.OK and c.pages_in_use() == 0
    # LIFO: the most recently released page (3) is handed out first
    assert c.append_step(1, 0, 0, row, row) == oracle.OK and c.page_of(1, 0) == 3
    c.reset()
    assert c.free_pages() == 8
    small = oracle.PagedCache(1, 1, 32, 1, 4, 2, oracle.Q8_0)
    for t in range(4):
        assert small.append_step(0, t, 0, row[:32], row[:32]) == oracle.OK
    assert small.free_pages() == 0
    assert small.release_layer(1) == oracle.INVALID_ARGUMENT


def test_paged_decreasing_error_across_modes(oracle):
    k = np.sin(np.arange(64) / 63.0).astype(np.float32)
    errs = []
    for mode in (oracle.Q4_0, oracle.Q5_0, oracle.Q8_0):
        c = oracle.PagedCache(1, 2, 32, 1, 4, 4, mode)
        c.append_step(0, 0, 0, k, np.zeros(64, np.float32))
        errs.append(float(((c.read_step(0, 0, 0)[0] - k) ** 2).sum()))
    assert errs[2] <= errs[1] <= errs[0]


def test_rms_norm_reference_case_and_float64(oracle):
    """text_decoder.rs rms_norm_normalises_row_to_unit_rms (gamma = 1, eps = 0,
    [1, 2, 3, 4] -> unit RMS), and float64 on random rows with gamma, eps."""
    out = oracle.rms_norm_f32(np.array([1, 2, 3, 4], np.float32), np.ones(4, np.float32), 0.0, 1, 4)
    assert abs(float((out.astype(np.float64) ** 2).mean()) - 1.0) < 1e-5
    assert np.allclose(out[0], np.array([1, 2, 3, 4]) / np.sqrt(7.5), rtol=1e-6)
    g = np.random.default_rng(12)
    x = g.standard_normal((6, 128)).astype(np.float32)
    gamma = g.standard_normal(128).astype(np.float32)
    got = oracle.rms_norm_f32(x, gamma, 1e-6, 6, 128)
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + 1e-6) * gamma
    assert np.allclose(got, want, rtol=1e-5, atol=1e-6)
