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


KQ_BLOCK_BYTES = {12: 144, 13: 176, 14: 210}


def random_kquant_blocks(rng, nb, wd=12):
    """kquant_gemm_parity.rs:45-62 random_blocks: random payload with the f16
    d / dmin high bytes pinned small (Q4_K / Q5_K: 0x2C / 0x24; Q6_K: d's high
    byte, the block's last, 0x2C)."""
    bb = KQ_BLOCK_BYTES[wd]
    b = bytearray(rng.bytes(nb * bb))
    for i in range(nb):
        if wd == 14:
            b[i * bb + 209] = 0x2C
        else:
            b[i * bb + 1] = 0x2C
            b[i * bb + 3] = 0x24
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


def hand_kquant_ints(w, wd):
    """Independent parse of K-quant rows (Q4_K, Q5_K, Q6_K) into unsigned
    integer quants q and per-16 (d_eff, m_eff) with y = d_eff * q - m_eff: the
    GGUF layouts (ggml k_quants.h) read with numpy, scales decoded by numpy
    float16. Q6_K's q is the stored 6-bit value (q6 + 32) and m_eff = 32 d_eff."""
    if wd == 12:
        return hand_q4k_ints(w)
    bb = KQ_BLOCK_BYTES[wd]
    blocks = np.asarray(w, np.uint8).reshape(-1, bb)
    nbt = blocks.shape[0]
    q = np.zeros((nbt, 256), np.uint8)
    d_eff = np.zeros((nbt, 16), np.float32)
    m_eff = np.zeros((nbt, 16), np.float32)
    for i, blk in enumerate(blocks):
        if wd == 13:
            d = np.frombuffer(bytes(blk[0:2]), np.float16)[0].astype(np.float32)
            dmin = np.frombuffer(bytes(blk[2:4]), np.float16)[0].astype(np.float32)
            sc = [int(v) for v in blk[4:16]]
            qh, qs = blk[16:48], blk[48:176]
            for j in range(8):
                s_j, m_j = _scale_min(j, sc)
                d_eff[i, 2 * j:2 * j + 2] = np.float32(d * np.float32(s_j))
                m_eff[i, 2 * j:2 * j + 2] = np.float32(dmin * np.float32(m_j))
                chunk = qs[32 * (j // 2):32 * (j // 2) + 32]
                low = (chunk >> 4) if j % 2 else (chunk & 0xF)
                q[i, 32 * j:32 * j + 32] = low + 16 * ((qh >> j) & 1)
        else:
            d = np.frombuffer(bytes(blk[208:210]), np.float16)[0].astype(np.float32)
            sc = blk[192:208].view(np.int8)
            vals = np.zeros(256, np.uint8)
            for half in range(2):
                ql, qh = blk[64 * half:64 * half + 64], blk[128 + 32 * half:160 + 32 * half]
                o = 128 * half
                vals[o:o + 32] = (ql[:32] & 0xF) | ((qh & 3) << 4)
                vals[o + 32:o + 64] = (ql[32:] & 0xF) | (((qh >> 2) & 3) << 4)
                vals[o + 64:o + 96] = (ql[:32] >> 4) | (((qh >> 4) & 3) << 4)
                vals[o + 96:o + 128] = (ql[32:] >> 4) | (((qh >> 6) & 3) << 4)
            q[i] = vals
            for g in range(16):
                half, rem = divmod(g, 8)
                quarter, sub = divmod(rem, 2)
                d_eff[i, g] = np.float32(d * np.float32(sc[8 * half + sub + 2 * quarter]))
            m_eff[i] = (d_eff[i] * np.float32(32.0)).astype(np.float32)
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


def _f16_bits(x):
    return int(np.float16(x).view(np.uint16))


def quantize_kquant_test(w, wd):
    """Valid Q5_K / Q6_K payloads for f32 rows of 256-multiples (test
    infrastructure, not the reference's converter, which has no Q5_K / Q6_K
    quantizer): per super-block the f16 scales from the block's range, 6-bit
    (Q5_K) or int8 (Q6_K) sub-scales per 32 / 16 elements, nearest quants.
    The bytes follow ggml k_quants.h, so the reference dequantizes them."""
    x = np.asarray(w, np.float32).reshape(-1, 256)
    out = []
    for blk in x:
        if wd == 13:
            lo, hi = float(min(blk.min(), 0.0)), float(max(blk.max(), 0.0))
            d = np.float32(np.float16((hi - lo) / (31.0 * 63.0) if hi > lo else 0.0))
            dmin = np.float32(np.float16(-lo / 63.0))
            sc, mn, qv = [0] * 8, [0] * 8, np.zeros(256, np.int32)
            for j in range(8):
                seg = blk[32 * j:32 * j + 32]
                mn[j] = int(np.clip(np.ceil(-float(seg.min()) / dmin), 0, 63)) if dmin > 0 else 0
                base = -np.float32(dmin * mn[j])
                sc[j] = int(np.clip(np.ceil(float(seg.max() - base) / (31.0 * d)), 1, 63)) if d > 0 else 0
                step = np.float32(d * sc[j])
                qv[32 * j:32 * j + 32] = np.clip(np.rint((seg - base) / step), 0, 31) if step > 0 else 0
            scales = [0] * 12
            for j in range(8):
                if j < 4:
                    scales[j] = sc[j] & 63
                    scales[j + 4] = mn[j] & 63
                else:
                    scales[j + 4] = (sc[j] & 0xF) | ((mn[j] & 0xF) << 4)
                    scales[j - 4] |= (sc[j] >> 4) << 6
                    scales[j] |= (mn[j] >> 4) << 6
            qs, qh = bytearray(128), bytearray(32)
            for k in range(4):
                for l in range(32):
                    a, b = int(qv[64 * k + l]), int(qv[64 * k + 32 + l])
                    qs[32 * k + l] = (a & 0xF) | ((b & 0xF) << 4)
                    qh[l] |= ((a >> 4) & 1) << (2 * k)
                    qh[l] |= ((b >> 4) & 1) << (2 * k + 1)
            out.append(_f16_bits(d).to_bytes(2, "little") + _f16_bits(dmin).to_bytes(2, "little") + bytes(scales)
                       + bytes(qh) + bytes(qs))
        else:
            amax = float(np.abs(blk).max())
            d = np.float32(np.float16(amax / (32.0 * 127.0) if amax > 0 else 0.0))
            sc = np.zeros(16, np.int32)
            qv = np.zeros(256, np.int32)
            for g in range(16):
                seg = blk[16 * g:16 * g + 16]
                sc[g] = int(np.clip(np.ceil(float(np.abs(seg).max()) / (32.0 * d)), 1, 127)) if d > 0 else 0
                step = np.float32(d * sc[g])
                qv[16 * g:16 * g + 16] = np.clip(np.rint(seg / step), -32, 31) if step > 0 else 0
            # scale index of group g (128 half + 32 quarter + 16 sub) is 8 half + sub + 2 quarter
            scales = np.zeros(16, np.int8)
            for g in range(16):
                half, rem = divmod(g, 8)
                quarter, sub = divmod(rem, 2)
                scales[8 * half + sub + 2 * quarter] = sc[g]
            ql, qh = bytearray(128), bytearray(64)
            for n in range(256):
                half, o = divmod(n, 128)
                quarter, l = divmod(o, 32)
                st = int(qv[n]) + 32
                low4, hi2 = st & 0xF, (st >> 4) & 3
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
            out.append(bytes(ql) + bytes(qh) + bytes(scales.view(np.uint8)) + _f16_bits(d).to_bytes(2, "little"))
    return np.frombuffer(b"".join(out), np.uint8).copy()
