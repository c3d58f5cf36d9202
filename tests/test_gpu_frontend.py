"""GPU parity of the Whisper front end: log-mel, conv1d and the encoder's
conv stem, against the reference's upstream golden vectors and the oracle.

Bars:
  * log-mel: the reference's own bound for its front end against upstream,
    atol 5e-5 (crates/vokra-models/tests/parity_voxtral.rs:76), on both golden
    clips (tests/golden/); against the oracle over the full [n_mels, 3000]
    grid, atol 1e-4 (the DFT is an f32 GEMM here, f64 in the oracle);
  * conv1d: the reference's hand fixtures exactly; random shapes within the
    f32 dot-product bound k 2^-23 sum|w x|;
  * encode (stem + blocks + ln_post): the oracle composition within
    0.1 rms, the session bar (INT8 rounding flips propagate).
"""
import os

import numpy as np
import pytest

from tests import model_oracle
from vokra_amd import hip

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def ctx():
    c = hip.HipContext(0)
    yield c
    c.close()


def jfk():
    z = np.load(os.path.join(GOLDEN, "jfk_pcm_i16.npz"))
    return z["pcm"].astype(np.float32) / np.float32(32768.0), int(z["voxtral_samples"])


@pytest.mark.parametrize("name,n_mels", [("whisper_base", 80), ("voxtral", 128)])
def test_log_mel_golden_and_oracle(ctx, oracle, name, n_mels):
    print(f"[case] log_mel {name}", flush=True)
    pcm, n_vox = jfk()
    x = pcm if name == "whisper_base" else pcm[:n_vox]
    got = ctx.log_mel(x, n_mels)
    assert got.shape == (n_mels, 3000)
    want = np.fromfile(os.path.join(GOLDEN, f"logmel_{name}.f32"), np.float32).reshape(n_mels, 100)
    assert np.abs(got[:, :100] - want).max() <= 5e-5
    assert np.abs(got - oracle.log_mel(x, n_mels)).max() <= 1e-4


def test_log_mel_batch_and_reference_behaviour(ctx, oracle):
    print("[case] log_mel batch / behaviour", flush=True)
    sr = 16000
    g = np.random.default_rng(3)
    clips = (0.2 * g.standard_normal((3, 3 * sr))).astype(np.float32)
    batch = ctx.log_mel(clips, 80)
    for i in range(3):
        assert np.array_equal(batch[i], ctx.log_mel(clips[i], 80))  # clips are independent
    silence = ctx.log_mel(np.zeros(sr, np.float32), 80)
    assert np.isfinite(silence).all() and np.abs(silence - oracle.log_mel(np.zeros(sr, np.float32), 80)).max() <= 1e-4
    tone = np.sin(2 * np.pi * 440 * np.arange(sr) / sr).astype(np.float32)
    t = ctx.log_mel(tone, 80)
    assert np.isfinite(t).all() and t.min() > -2 and t.max() < 2
    assert np.abs(t - oracle.log_mel(tone, 80)).max() <= 1e-4
    empty = ctx.log_mel(np.zeros(0, np.float32), 80)
    assert empty.shape == (80, 3000) and np.isfinite(empty).all()
    big = (0.1 * g.standard_normal(480000 + 5000)).astype(np.float32)
    assert np.array_equal(ctx.log_mel(big, 80), ctx.log_mel(big[:480000], 80))  # trimmed to 30 s


def test_log_mel_rejections(ctx):
    with pytest.raises(hip.InvalidArgument):
        ctx.log_mel(np.zeros(16, np.float32), 0)


@pytest.mark.parametrize("args,want", [
    (([1, 2, 3, 4, 5], 1, 5, [1, 1, 1], 1, 3, None, 1, 0), [[6, 9, 12]]),
    (([1, 2, 3], 1, 3, [1, 0, -1], 1, 3, [10], 1, 1), [[8, 8, 12]]),
    (([1, 2, 3, 4, 10, 20, 30, 40], 2, 4, [1, 1, 1, 1], 1, 2, None, 2, 0), [[33, 77]]),
    (([1, 2, 3, 4, 5, 6], 1, 6, [1, 1], 1, 2, None, 3, 0), [[3, 9]]),
    (([2, 3], 1, 2, [1], 1, 1, None, 1, 2), [[0, 0, 2, 3, 0, 0]]),
])
def test_conv1d_reference_hand_fixtures(ctx, args, want):
    got = ctx.conv1d_f32(*[np.asarray(a, np.float32) if isinstance(a, list) else a for a in args])
    assert np.array_equal(got, np.array(want, np.float32))


@pytest.mark.parametrize("in_ch,in_len,out_ch,kernel,stride,padding", [(3, 17, 5, 3, 1, 1), (4, 20, 2, 3, 2, 1),
                                                                     (80, 3000, 64, 3, 1, 1), (64, 3000, 64, 3, 2, 1)])
def test_conv1d_vs_oracle(ctx, oracle, in_ch, in_len, out_ch, kernel, stride, padding):
    print(f"[case] conv1d {in_ch}x{in_len} -> {out_ch} k{kernel} s{stride} p{padding}", flush=True)
    g = np.random.default_rng(in_ch * 7 + in_len)
    x = g.standard_normal((in_ch, in_len)).astype(np.float32)
    w = (g.standard_normal((out_ch, in_ch, kernel)) * 0.1).astype(np.float32)
    b = g.standard_normal(out_ch).astype(np.float32)
    got = ctx.conv1d_f32(x, in_ch, in_len, w, out_ch, kernel, b, stride, padding)
    want = oracle.conv1d_f32(x, in_ch, in_len, w, out_ch, kernel, b, stride, padding)
    k = in_ch * kernel
    bound = 2 * k * 2.0 ** -23 * (np.abs(w).reshape(out_ch, -1).sum(1)[:, None] * np.abs(x).max() + np.abs(b)[:, None])
    assert np.all(np.abs(got - want) <= bound + 1e-6)


def test_conv1d_rejections(ctx):
    with pytest.raises(hip.InvalidArgument, match="smaller than kernel"):
        ctx.conv1d_f32(np.zeros(2, np.float32), 1, 2, np.ones(5, np.float32), 1, 5)
    with pytest.raises(hip.InvalidArgument, match="stride"):
        ctx.conv1d_f32(np.zeros(2, np.float32), 1, 2, np.ones(1, np.float32), 1, 1, stride=0)


def test_encode_from_audio_config0(ctx, oracle):
    """Whisper-base dims (80 mels, d=512, 8 heads, FFN 2048), one block: PCM ->
    log-mel -> conv stem -> block -> ln_post, against the oracle's chain."""
    print("[case] encode config0 one block from audio", flush=True)
    from tests.test_gpu_sessions import W_Q8_0, enc_layer, rand_norm
    pcm, _ = jfk()
    n_mels, d, H, ff = 80, 512, 8, 2048
    g = np.random.default_rng(77)
    layers = [enc_layer(ctx, g, W_Q8_0, d, ff, scale=0.02)]
    lpg, lpb = rand_norm(g, d)
    c1w = (g.standard_normal((d, n_mels, 3)) * 0.05).astype(np.float32)
    c1b = (g.standard_normal(d) * 0.05).astype(np.float32)
    c2w = (g.standard_normal((d, d, 3)) * 0.02).astype(np.float32)
    c2b = (g.standard_normal(d) * 0.05).astype(np.float32)
    pos = (g.standard_normal((1500, d)) * 0.1).astype(np.float32)
    enc = hip.Encoder(ctx, W_Q8_0, d, H, ff, layers, lpg, lpb, max_rows=1500)
    enc.set_stem(n_mels, 3000, c1w, c1b, c2w, c2b, pos)
    got = enc.encode(ctx.log_mel(pcm, n_mels)[None])[0]
    # oracle chain
    mel = oracle.log_mel(pcm, n_mels)
    c1 = oracle.gelu_f32(oracle.conv1d_f32(mel, n_mels, 3000, c1w, d, 3, c1b, 1, 1))
    c2 = oracle.gelu_f32(oracle.conv1d_f32(c1, d, 3000, c2w, d, 3, c2b, 2, 1))
    h = (c2.T + pos).astype(np.float32)
    want = model_oracle.encoder(oracle, W_Q8_0, layers, lpg, lpb, h[None], H, ff)[0]
    rms = float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
    assert np.abs(got - want).max() <= 0.1 * rms, (np.abs(got - want).max(), rms)
