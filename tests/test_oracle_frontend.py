"""Pins the oracle's Whisper front end (log-mel, conv1d) on the CPU.

* log-mel: against the reference's own upstream golden vectors
  (tests/golden/, copied from tests/parity/whisper_base and tests/parity/voxtral
  by tests/golden/make_mel_fixtures.py) at the reference's tightest bound,
  atol 5e-5 (crates/vokra-models/tests/parity_voxtral.rs:76), and the
  behaviour tests of crates/vokra-models/src/whisper/mel.rs:239-290;
* the periodic Hann window against its closed form; the filter bank against
  properties a wrong edge, scale or norm would break;
* conv1d: the reference's hand fixtures (crates/vokra-backend-cpu/src/kernels/
  mod.rs:906-1010), exact, and random shapes against float64.
"""
import os

import numpy as np
import pytest

from oracle import oracle as orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def jfk():
    z = np.load(os.path.join(GOLDEN, "jfk_pcm_i16.npz"))
    return z["pcm"].astype(np.float32) / np.float32(32768.0), int(z["voxtral_samples"])


@pytest.mark.parametrize("name,n_mels", [("whisper_base", 80), ("voxtral", 128)])
def test_log_mel_matches_upstream_golden(name, n_mels):
    pcm, n_vox = jfk()
    x = pcm if name == "whisper_base" else pcm[:n_vox]
    got = orc.log_mel(x, n_mels)
    assert got.shape == (n_mels, 3000)
    want = np.fromfile(os.path.join(GOLDEN, f"logmel_{name}.f32"), np.float32).reshape(n_mels, 100)
    assert np.abs(got[:, :100] - want).max() <= 5e-5


def test_log_mel_reference_behaviour():
    sr = 16000
    silence = orc.log_mel(np.zeros(sr, np.float32), 80)
    assert silence.shape == (80, 3000) and np.isfinite(silence).all()
    tone = np.sin(2 * np.pi * 440 * np.arange(sr) / sr).astype(np.float32)
    t = orc.log_mel(tone, 80)
    assert np.isfinite(t).all() and t.min() > -2 and t.max() < 2
    empty = orc.log_mel(np.zeros(0, np.float32), 80)
    assert empty.shape == (80, 3000) and np.isfinite(empty).all()
    big = orc.log_mel(np.full(480000 + 5000, 0.1, np.float32), 80)
    assert big.shape == (80, 3000) and np.isfinite(big).all()
    # trimming: samples past 30 s do not change anything
    g = np.random.default_rng(1).standard_normal(480000 + 777).astype(np.float32) * 0.1
    assert np.array_equal(orc.log_mel(g, 80), orc.log_mel(g[:480000], 80))


def test_hann_periodic_closed_form():
    n = np.arange(400)
    w = orc.hann_periodic(400)
    assert np.abs(w - (0.5 - 0.5 * np.cos(2 * np.pi * n / 400))).max() < 1e-7
    assert w[0] == 0.0 and np.array_equal(w[1:], w[1:][::-1])  # periodic: symmetric about n = 200


def test_mel_filterbank_properties():
    for n_mels in (80, 128):
        fb = orc.mel_filterbank(n_mels).astype(np.float64)
        assert fb.shape == (n_mels, 201) and (fb >= 0).all()
        assert all(fb[m].max() > 0 for m in range(n_mels))  # no empty filter
        # Slaney norm: area over Hz (40 Hz bins) is 1 for filters wider than a few bins
        area = fb.sum(axis=1) * 40.0
        wide = [m for m in range(n_mels) if (fb[m] > 0).sum() >= 6]
        assert np.allclose(area[wide], 1.0, rtol=0.05)
        # centres move up monotonically; Slaney is linear (66.7 Hz per mel) below 1 kHz
        peaks = fb.argmax(axis=1)
        assert (np.diff(peaks) >= 0).all()
    fb80 = orc.mel_filterbank(80).astype(np.float64)
    # the first filter's peak sits at the first band centre, 8000/81 * ... on the mel axis:
    # below 1 kHz mel = f / (200/3), so centre_1 = max_mel / 81 * (200/3) Hz
    max_mel = 15.0 + np.log(8.0) / (np.log(6.4) / 27.0)
    c1 = max_mel / 81.0 * 200.0 / 3.0
    assert abs(fb80[0].argmax() * 40.0 - c1) <= 20.0


@pytest.mark.parametrize("args,want", [
    (([1, 2, 3, 4, 5], 1, 5, [1, 1, 1], 1, 3, None, 1, 0), [[6, 9, 12]]),
    (([1, 2, 3], 1, 3, [1, 0, -1], 1, 3, [10], 1, 1), [[8, 8, 12]]),
    (([1, 2, 3, 4, 10, 20, 30, 40], 2, 4, [1, 1, 1, 1], 1, 2, None, 2, 0), [[33, 77]]),
    (([1, 2, 3, 4, 5, 6], 1, 6, [1, 1], 1, 2, None, 3, 0), [[3, 9]]),
    (([2, 3], 1, 2, [1], 1, 1, None, 1, 2), [[0, 0, 2, 3, 0, 0]]),
])
def test_conv1d_reference_hand_fixtures(args, want):
    assert np.array_equal(orc.conv1d_f32(*args), np.array(want, np.float32))


def test_conv1d_rejections():
    with pytest.raises(orc.OracleError):
        orc.conv1d_f32([1, 2], 1, 2, [1] * 5, 1, 5, None, 1, 0)
    with pytest.raises(orc.OracleError):
        orc.conv1d_f32([1, 2], 1, 2, [1], 1, 1, None, 0, 0)


@pytest.mark.parametrize("in_ch,in_len,out_ch,kernel,stride,padding", [(3, 17, 5, 3, 1, 1), (4, 20, 2, 3, 2, 1),
                                                                     (80, 50, 16, 3, 1, 1)])
def test_conv1d_vs_float64(in_ch, in_len, out_ch, kernel, stride, padding):
    g = np.random.default_rng(in_ch + in_len)
    x = g.standard_normal((in_ch, in_len)).astype(np.float32)
    w = g.standard_normal((out_ch, in_ch, kernel)).astype(np.float32)
    b = g.standard_normal(out_ch).astype(np.float32)
    got = orc.conv1d_f32(x, in_ch, in_len, w, out_ch, kernel, b, stride, padding)
    xp = np.pad(x.astype(np.float64), ((0, 0), (padding, padding)))
    out_len = (in_len + 2 * padding - kernel) // stride + 1
    want = np.stack([np.einsum("ck,ck->", w[o].astype(np.float64),
                               xp[:, t * stride:t * stride + kernel]) + b[o]
                     for o in range(out_ch) for t in range(out_len)]).reshape(out_ch, out_len)
    k = in_ch * kernel
    assert np.abs(got - want).max() <= k * 2.0 ** -23 * (np.abs(w).sum() * np.abs(x).max() + abs(b).max()) + 1e-6
