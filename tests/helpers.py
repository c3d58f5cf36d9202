"""Shared test helpers: the reference tests' reproducible input generators and
independent (numpy) parsers of the wire formats."""
from fractions import Fraction

import numpy as np


class Rng:
    """xorshift64* as in crates/vokra-backend-cpu/tests/kquant_gemm_parity.rs:19-43."""

    M = 0xFFFFFFFFFFFFFFFF

    def __init__(self, seed):
        self.s = (seed | 1) & self.M

    def next_u64(self):
        x = self.s
        x ^= x >> 12
        x ^= (x << 25) & self.M
        x ^= x >> 27
        self.s = x
        return (x * 0x2545F4914F6CDD1D) & self.M

    def next_f32(self):
        bits = np.float32(self.next_u64() >> 40)
        return np.float32(np.float32(bits / np.float32(1 << 24)) * np.float32(2.0)) - np.float32(1.0)

    def vec(self, n):
        return [self.next_f32() for _ in range(n)]

    def bytes(self, n):
        return bytes(((self.next_u64() >> 32) & 0xFF) for _ in range(n))


def random_kquant_blocks(rng, nb):
    """kquant_gemm_parity.rs:45-62 random_blocks for Q4_K: random payload with
    the f16 d / dmin high bytes pinned small (0x2C / 0x24)."""
    b = bytearray(rng.bytes(nb * 144))
    for i in range(nb):
        b[i * 144 + 1] = 0x2C
        b[i * 144 + 3] = 0x24
    return np.frombuffer(bytes(b), np.uint8).copy()


def _scale_min(j, s):
    if j < 4:
        return s[j] & 63, s[j + 4] & 63
    return (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4), (s[j + 4] >> 4) | ((s[j] >> 6) << 4)


def hand_q4k_ints(w):
    """Independent parse of Q4_K rows into integer quants and per-16 effective
    scales (numpy float16 decodes d / dmin)."""
    blocks = np.asarray(w, np.uint8).reshape(-1, 144)
    nbt = blocks.shape[0]
    q = np.zeros((nbt, 256), np.uint8)
    d_eff = np.zeros((nbt, 16), np.float32)
    m_eff = np.zeros((nbt, 16), np.float32)
    for i, blk in enumerate(blocks):
        d = np.frombuffer(bytes(blk[0:2]), np.float16)[0].astype(np.float32)
        dmin = np.frombuffer(bytes(blk[2:4]), np.float16)[0].astype(np.float32)
        sc = [int(v) for v in blk[4:16]]
        qs = blk[16:144]
        for j in range(8):
            s_j, m_j = _scale_min(j, sc)
            d_eff[i, 2 * j:2 * j + 2] = np.float32(d * np.float32(s_j))
            m_eff[i, 2 * j:2 * j + 2] = np.float32(dmin * np.float32(m_j))
            chunk = qs[32 * (j // 2):32 * (j // 2) + 32]
            q[i, 32 * j:32 * j + 32] = (chunk >> 4) if j % 2 else (chunk & 0xF)
    return q, d_eff, m_eff


def hand_qblock_ints(mode, wq, n, k):
    """Independent parse of row-major Q_0 blocks to (int8 quants [n,k],
    f32 scales [n,k/32]). mode: 1=Q4_0, 2=Q5_0, 3=Q8_0."""
    bb = {1: 18, 2: 22, 3: 34}[mode]
    nb = k // 32
    blocks = np.asarray(wq, np.uint8).reshape(n * nb, bb)
    d = blocks[:, 0:2].copy().view(np.float16).astype(np.float32).reshape(n, nb)
    if mode == 3:
        q = blocks[:, 2:34].view(np.int8).astype(np.int8)
    elif mode == 1:
        b = blocks[:, 2:18].astype(np.int16)
        q = np.empty((n * nb, 32), np.int8)
        q[:, 0::2] = (b & 0xF) - 8
        q[:, 1::2] = (b >> 4) - 8
    else:
        qh = blocks[:, 2:6].copy().view(np.uint32).reshape(-1).astype(np.int64)
        b = blocks[:, 6:22].astype(np.int16)
        lo = np.empty((n * nb, 32), np.int16)
        lo[:, 0::2] = b & 0xF
        lo[:, 1::2] = b >> 4
        hi = ((qh[:, None] >> np.arange(32)[None, :]) & 1).astype(np.int16)
        q = (((hi << 4) | lo) - 16).astype(np.int8)
    return q.reshape(n, k), d


def round_to_f32(x: Fraction) -> np.float32:
    """Correctly rounded (ties-to-even) conversion of an exact rational."""
    f = np.float32(float(x))
    best = f
    for cand in (np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))):
        if not np.isfinite(cand):
            continue
        dc = abs(Fraction(float(cand)) - x)
        db = abs(Fraction(float(best)) - x)
        if dc < db or (dc == db and (int(cand.view(np.uint32)) & 1) == 0):
            best = cand
    return np.float32(best)


def exact_fmaf(a, b, c) -> np.float32:
    """fmaf(a, b, c) with a single rounding, computed in exact rationals."""
    return round_to_f32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))
