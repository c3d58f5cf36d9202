"""Pins the oracle's speech-LLM text-decoder primitives (RMSNorm, RoPE, SiLU,
Hadamard / SwiGLU) and its step composition.

Reference tests restated: crates/vokra-models/src/voxtral/text_decoder.rs:
1840-2140 (rms_norm, silu, hadamard, rope_apply cases). Beyond those, every
function is held against a float64 evaluation of its formula with a bound
derived from the f32 roundings it performs, so a dropped term, a wrong pair
index, a wrong sign or a wrong frequency exponent fails.
"""
import math

import numpy as np
import pytest

from tests import model_oracle

U = 2.0 ** -24  # unit roundoff of f32


# ---- rms_norm (text_decoder.rs:801-822) ----------------------------------
def test_rms_norm_reference_cases(oracle):
    out = oracle.rms_norm_f32(np.array([1, 2, 3, 4], np.float32), np.ones(4, np.float32), 0.0, 1, 4)
    assert abs(float(np.mean(out.astype(np.float64) ** 2)) - 1.0) < 1e-5           # unit RMS
    out = oracle.rms_norm_f32(np.zeros(4, np.float32), np.ones(4, np.float32), 1e-5, 1, 4)
    assert np.all(np.abs(out) < 1e-6)                                                # eps guards 0
    g = np.array([10, 20, 30, 40], np.float32)
    out = oracle.rms_norm_f32(np.full(4, 2.0, np.float32), g, 0.0, 1, 4)
    assert np.all(np.abs(out[0] - g) < 1e-4)                                          # gamma per channel
    # epsilon scales predictably: x = [1,1,1,1], eps = 3 -> 1 / sqrt(1 + 3) = 0.5
    out = oracle.rms_norm_f32(np.ones(4, np.float32), np.ones(4, np.float32), 3.0, 1, 4)
    assert np.all(np.abs(out - 0.5) < 1e-6)
    # rows are independent
    x = np.array([[1, 2, 3, 4], [2, 2, 2, 2]], np.float32)
    both = oracle.rms_norm_f32(x, np.ones(4, np.float32), 0.0, 2, 4)
    assert np.array_equal(both[1], oracle.rms_norm_f32(x[1], np.ones(4, np.float32), 0.0, 1, 4)[0])


def test_rms_norm_vs_float64(oracle):
    g = np.random.default_rng(0)
    d = 2048
    x = g.standard_normal((4, d)).astype(np.float32) * 3
    gamma = (1 + 0.1 * g.standard_normal(d)).astype(np.float32)
    got = oracle.rms_norm_f32(x, gamma, 1e-5, 4, d).astype(np.float64)
    xd = x.astype(np.float64)
    want = xd / np.sqrt((xd ** 2).mean(axis=1, keepdims=True) + 1e-5) * gamma
    # a sequential f32 sum of d squares: relative error <= (d + 4) u, then 3 roundings
    assert np.all(np.abs(got - want) <= (d / 2 + 8) * U * np.abs(want) + 1e-30)


# ---- rope_apply (text_decoder.rs:858-891) --------------------------------
def test_rope_reference_cases(oracle):
    x = np.array([1, 2, 3, 4], np.float32)
    assert np.array_equal(oracle.rope_apply(x, 1, 4, 10000.0, 0), x)                  # position 0
    x = np.array([1, 0, 0, 1, 2, 3, 4, 5], np.float32)
    r = oracle.rope_apply(x, 2, 4, 10000.0, 3).reshape(2, 4)
    assert np.allclose(np.linalg.norm(r, axis=1), np.linalg.norm(x.reshape(2, 4), axis=1), atol=1e-4)
    r = oracle.rope_apply(np.array([1, 0, 0, 0], np.float32), 1, 4, 10000.0, 5)       # theta_0 = 1
    assert abs(r[0] - math.cos(5.0)) < 1e-6 and abs(r[2] - math.sin(5.0)) < 1e-6
    r = oracle.rope_apply(np.array([0, 1, 0, 0], np.float32), 1, 4, 10000.0, 1)       # theta_1 = 0.01
    assert abs(r[1] - math.cos(0.01)) < 1e-7 and abs(r[3] - math.sin(0.01)) < 1e-7
    full = oracle.rope_apply(np.tile(np.array([1, 2, 3, 4], np.float32), 5), 5, 4, 10000.0, 0)
    single = oracle.rope_apply(np.array([1, 2, 3, 4], np.float32), 1, 4, 10000.0, 3)
    assert np.array_equal(single, full[12:16])                                        # offset invariance
    with pytest.raises(oracle.OracleError):
        oracle.rope_apply(np.array([1, 2, 3], np.float32), 1, 3, 10000.0, 0)          # odd head_dim
    with pytest.raises(oracle.OracleError):
        oracle.rope_apply(np.array([1, 2, 3], np.float32), 1, 4, 10000.0, 0)          # length mismatch


@pytest.mark.parametrize("base,hd", [(1e6, 128), (1e4, 64)])
def test_rope_vs_float64_rotation(oracle, base, hd):
    """Against the exact rotation by m * base^(-2j/hd) in float64. The f32
    path rounds theta (powf, <= 1 ulp), the product m * theta and sin / cos,
    so the angle error is at most m ulp(theta) + ulp(angle): the bound below
    is 4 ulp of the angle plus 4 ulp of the outputs."""
    g = np.random.default_rng(hd)
    positions = [0, 1, 2, 17, 511, 512, 1000, 2047, 4095]
    x = g.standard_normal((len(positions), hd)).astype(np.float32)
    half = hd // 2
    for r, m in enumerate(positions):
        got = oracle.rope_apply(x[r], 1, hd, base, m).astype(np.float64)
        j = np.arange(half)
        theta = float(base) ** (-2.0 * j / hd)
        ang = m * theta
        a, b = x[r, :half].astype(np.float64), x[r, half:].astype(np.float64)
        want = np.concatenate([a * np.cos(ang) - b * np.sin(ang), a * np.sin(ang) + b * np.cos(ang)])
        mag = np.concatenate([np.abs(a) + np.abs(b)] * 2)
        ang_err = 4 * np.spacing(np.maximum(ang, 1e-30).astype(np.float32)).astype(np.float64)
        bound = mag * (np.concatenate([ang_err] * 2) + 8 * U)
        assert np.all(np.abs(got - want) <= bound + 1e-30), (m, float(np.max(np.abs(got - want) - bound)))


def test_rope_heads_is_per_head(oracle):
    g = np.random.default_rng(1)
    x = g.standard_normal((3, 4 * 64)).astype(np.float32)
    r = oracle.rope_heads(x, 4, 64, 1e6, 10)
    for h in range(4):
        want = oracle.rope_apply(x[:, 64 * h:64 * (h + 1)], 3, 64, 1e6, 10).reshape(3, 64)
        assert np.array_equal(r[:, 64 * h:64 * (h + 1)], want)


# ---- silu / hadamard (text_decoder.rs:826-847) ---------------------------
def test_silu_reference_cases(oracle):
    s = oracle.silu(np.array([0.0, 5.0, -5.0, 1.0], np.float32))
    assert abs(s[0]) < 1e-6
    assert abs(s[1] - 5.0 / (1.0 + math.exp(-5.0))) < 1e-5
    assert abs(s[2]) < 0.05
    assert abs(s[3] - 0.7310586) < 1e-3
    h = 1e-3
    d = (oracle.silu(np.array([h], np.float32))[0] - oracle.silu(np.array([-h], np.float32))[0]) / (2 * h)
    assert abs(d - 0.5) < 1e-2
    assert abs(oracle.silu(np.array([50.0], np.float32))[0] - 50.0) < 1e-3
    assert abs(oracle.silu(np.array([-50.0], np.float32))[0]) < 1e-10


def test_silu_vs_float64(oracle):
    x = np.linspace(-30, 30, 6001).astype(np.float32)
    got = oracle.silu(x).astype(np.float64)
    xd = x.astype(np.float64)
    want = xd / (1.0 + np.exp(-xd))
    # expf (<= 1 ulp), the add, the divide and the product: <= 4 ulp + slack
    assert np.all(np.abs(got - want) <= 6 * U * np.abs(want) + 1e-38)


def test_hadamard_and_swiglu(oracle):
    assert oracle.hadamard([1, 2, 3], [4, 5, 6]).tolist() == [4.0, 10.0, 18.0]
    with pytest.raises(oracle.OracleError):
        oracle.hadamard([1, 2], [1])
    gate = np.array([1, 2, 3, 4], np.float32)
    sw = oracle.swiglu(gate, gate)
    want = gate.astype(np.float64) / (1 + np.exp(-gate.astype(np.float64))) * gate
    assert np.all(np.abs(sw - want) < 1e-4)
    # the sequence is silu first, then the product (two roundings)
    assert np.array_equal(sw, oracle.silu(gate) * gate)


# ---- the step composition -------------------------------------------------
def test_text_decoder_step_composition(oracle):
    """The oracle step at a toy size equals a float64 re-derivation of the
    same sequence to within the INT8 activation rounding of its linears (a
    structural check: a skipped residual, RoPE on the wrong operand or a
    missing norm fails by O(1))."""
    g = np.random.default_rng(7)
    d, hq, hkv, hd, ff, V = 256, 4, 2, 64, 512, 64
    layers = [model_oracle.random_text_layer(oracle, g, d, hq, hkv, hd, ff) for _ in range(2)]
    tok = (g.standard_normal((V, d)) * 0.5).astype(np.float32)
    fin = (1 + 0.1 * g.standard_normal(d)).astype(np.float32)
    head = oracle.kquant_quantize(12, (g.standard_normal((V, d)) * 0.05).astype(np.float32).reshape(-1))
    dec = model_oracle.TextDecoder(oracle, layers, tok, fin, head, hq, hkv, hd, ff, 1, 64, 16, 1e6, 1e-5)
    # float64 path with the weights dequantized (activations unquantized)
    W = {}
    for li, L in enumerate(layers):
        for name, n, k in (("wq", hq * hd, d), ("wk", hkv * hd, d), ("wv", hkv * hd, d), ("wo", d, hq * hd),
                           ("w_gate", ff, d), ("w_up", ff, d), ("w_down", d, ff)):
            W[li, name] = oracle.kquant_dequantize(12, L[name], n * k).reshape(n, k).astype(np.float64)
    Hd = oracle.kquant_dequantize(12, head, V * d).reshape(V, d).astype(np.float64)
    Ks = [[] for _ in layers]
    Vs = [[] for _ in layers]
    toks = [3, 9, 27]
    for pos, t in enumerate(toks):
        logits, _ = dec.step(0, t, pos)
        h = tok[t].astype(np.float64)
        for li, L in enumerate(layers):
            x = h / np.sqrt((h ** 2).mean() + 1e-5) * L["attn_norm_gamma"]
            q = W[li, "wq"] @ x
            k = W[li, "wk"] @ x
            v = W[li, "wv"] @ x

            def rot(z, nh):
                z = z.reshape(nh, hd).copy()
                j = np.arange(hd // 2)
                ang = pos * 1e6 ** (-2.0 * j / hd)
                a, b = z[:, :hd // 2].copy(), z[:, hd // 2:].copy()
                z[:, :hd // 2] = a * np.cos(ang) - b * np.sin(ang)
                z[:, hd // 2:] = a * np.sin(ang) + b * np.cos(ang)
                return z.reshape(-1)
            q, k = rot(q, hq), rot(k, hkv)
            Ks[li].append(k)
            Vs[li].append(v)
            K, Vv = np.stack(Ks[li]), np.stack(Vs[li])
            att = np.zeros(hq * hd)
            for h_ in range(hq):
                kh = h_ // (hq // hkv)
                s = K[:, kh * hd:(kh + 1) * hd] @ q[h_ * hd:(h_ + 1) * hd] / math.sqrt(hd)
                p = np.exp(s - s.max())
                att[h_ * hd:(h_ + 1) * hd] = (p / p.sum()) @ Vv[:, kh * hd:(kh + 1) * hd]
            h = h + W[li, "wo"] @ att
            x = h / np.sqrt((h ** 2).mean() + 1e-5) * L["ffn_norm_gamma"]
            gt, up = W[li, "w_gate"] @ x, W[li, "w_up"] @ x
            h = h + W[li, "w_down"] @ (gt / (1 + np.exp(-gt)) * up)
        x = h / np.sqrt((h ** 2).mean() + 1e-5) * fin
        want = Hd @ x
        rms = float(np.sqrt(np.mean(want ** 2)))
        # INT8 activations (per 16, step amax/127) move each linear by well under 2 %
        assert np.max(np.abs(logits - want)) <= 0.05 * rms, (pos, np.max(np.abs(logits - want)), rms)
