"""Writes the log-mel golden fixtures from the reference's own parity data.

Run in a container that has the reference checkout (read-only) at
/root/reference; the outputs are plain data and are committed:

  jfk_pcm_i16.npz          the 30 s, 16 kHz mono input both reference fixtures
                           were made from (tests/parity/whisper_base/input_pcm.f32;
                           the voxtral input_pcm.f32 is its first 176000
                           samples), stored as the exact int16 values (x 32768)
  logmel_whisper_base.f32  [80, 100]: the first 100 frames of the upstream
                           openai/whisper-base log-mel of the full 30 s input
                           (tests/parity/whisper_base/logmel.f32; atol 0.01)
  logmel_voxtral.f32       [128, 100]: the first 100 frames of the upstream
                           128-mel front end of the first 176000 samples,
                           zero-padded to 30 s (tests/parity/voxtral/log_mel.f32.bin;
                           the reference test holds it to atol 5e-5)
"""
import os
import sys

import numpy as np

REF = "/root/reference/tests/parity"
HERE = os.path.dirname(os.path.abspath(__file__))


def main() -> int:
    pcm = np.fromfile(os.path.join(REF, "whisper_base", "input_pcm.f32"), np.float32)
    vox = np.fromfile(os.path.join(REF, "voxtral", "input_pcm.f32"), np.float32)
    assert pcm.size == 480000 and np.array_equal(pcm[: vox.size], vox), "voxtral input is a prefix"
    q = pcm * np.float32(32768.0)
    assert np.array_equal(q, np.round(q)), "samples are int16 / 32768"
    np.savez_compressed(os.path.join(HERE, "jfk_pcm_i16.npz"), pcm=q.astype(np.int16),
                        voxtral_samples=np.int64(vox.size))
    for src, dst, n in (("whisper_base/logmel.f32", "logmel_whisper_base.f32", 80 * 100),
                        ("voxtral/log_mel.f32.bin", "logmel_voxtral.f32", 128 * 100)):
        g = np.fromfile(os.path.join(REF, src), np.float32)
        assert g.size == n, (src, g.size)
        g.tofile(os.path.join(HERE, dst))
    return 0


if __name__ == "__main__":
    sys.exit(main())
