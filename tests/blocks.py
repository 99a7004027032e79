"""Hand-built GGML blocks with closed-form dequantized values.

Each builder writes one block from integer fields as the GGML block layouts
define them (Q8_0: d, qs[32]; Q5_0: d, qh[4], qs[16]; Q4_K: d, dmin,
scales[12], qs[128]; Q6_K: ql[128], qh[64], scales[16], d) and returns the
values those fields stand for, computed directly from the format's definition
(value = d * q for Q8_0, d * (q - 16) for Q5_0, d * sc * q - dmin * m for
Q4_K, d * sc * (q - 32) for Q6_K) with exactly representable d so the
expected values are exact.
"""

from __future__ import annotations

import numpy as np

F16_ONE = 0x3C00
F16_HALF = 0x3800
F16_TWO = 0x4000


def f16(bits: int) -> bytes:
    return int(bits).to_bytes(2, "little")


def q8_0(qs, d_bits=F16_ONE, d=1.0):
    qs = np.asarray(qs, dtype=np.int8)
    assert qs.size == 32
    return f16(d_bits) + qs.tobytes(), qs.astype(np.float64) * d


def q5_0(q, d_bits=F16_ONE, d=1.0):
    """q: 32 five-bit values (0..31)."""
    q = np.asarray(q, dtype=np.int64)
    assert q.size == 32 and q.min() >= 0 and q.max() <= 31
    qs = bytearray(16)
    qh = 0
    for j in range(16):
        qs[j] = int((q[j] & 0xF) | ((q[j + 16] & 0xF) << 4))
        qh |= ((q[j] >> 4) & 1) << j
        qh |= ((q[j + 16] >> 4) & 1) << (j + 16)
    return f16(d_bits) + int(qh).to_bytes(4, "little") + bytes(qs), (q - 16).astype(np.float64) * d


def _q4k_scales(sc, m):
    s = bytearray(12)
    for j in range(8):
        if j < 4:
            s[j] = sc[j] & 63
            s[j + 4] = m[j] & 63
    for j in range(4, 8):
        s[j + 4] = (sc[j] & 0xF) | ((m[j] & 0xF) << 4)
        s[j - 4] |= (sc[j] >> 4) << 6
        s[j] |= (m[j] >> 4) << 6
    return bytes(s)


def q4_k(sc, m, q, d_bits=F16_ONE, dmin_bits=F16_ONE, d=1.0, dmin=1.0):
    """sc, m: 8 six-bit sub-block scales/mins; q: 256 nibbles (element order)."""
    q = np.asarray(q, dtype=np.int64)
    assert q.size == 256 and q.max() <= 15
    qs = bytearray(128)
    for g in range(4):
        for l in range(32):
            qs[32 * g + l] = int(q[64 * g + l] | (q[64 * g + 32 + l] << 4))
    vals = np.empty(256)
    for i in range(256):
        sub = i // 32
        vals[i] = d * sc[sub] * q[i] - dmin * m[sub]
    return f16(d_bits) + f16(dmin_bits) + _q4k_scales(sc, m) + bytes(qs), vals


def q6_k(sc, q, d_bits=F16_ONE, d=1.0):
    """sc: 16 int8 group scales; q: 256 six-bit values (0..63), element order."""
    q = np.asarray(q, dtype=np.int64)
    assert q.size == 256 and q.max() <= 63
    ql = bytearray(128)
    qh = bytearray(64)
    for n in range(2):
        for l in range(32):
            e = 128 * n + l
            q1, q2, q3, q4 = q[e], q[e + 32], q[e + 64], q[e + 96]
            ql[64 * n + l] = int((q1 & 0xF) | ((q3 & 0xF) << 4))
            ql[64 * n + l + 32] = int((q2 & 0xF) | ((q4 & 0xF) << 4))
            qh[32 * n + l] = int((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6))
    scales = np.asarray(sc, dtype=np.int8)
    vals = np.array([d * int(scales[i // 16]) * (q[i] - 32) for i in range(256)], dtype=np.float64)
    return bytes(ql) + bytes(qh) + scales.tobytes() + f16(d_bits), vals


def kat_rows():
    """(type, row bytes, cols, expected values) for a set of corner cases."""
    rng = np.random.default_rng(1234)
    rows = []
    # Q8_0: extremes and a ramp, d = 1 and d = 0.5.
    b1, v1 = q8_0(np.arange(-128, 128, 8))
    b2, v2 = q8_0(np.r_[[-128, 127, 0, -1, 1], np.zeros(27, dtype=int)], F16_HALF, 0.5)
    rows.append((8, b1 + b2, 64, np.r_[v1, v2]))
    # Q5_0: every 5-bit value, high bits in both halves.
    b1, v1 = q5_0(np.arange(32))
    b2, v2 = q5_0(31 - np.arange(32), F16_TWO, 2.0)
    rows.append((6, b1 + b2, 64, np.r_[v1, v2]))
    # Q4_K: scale/min indices below and above 4 (the split 6-bit encoding),
    # including values >= 16 that use the two high bits.
    sc = [1, 2, 63, 17, 16, 47, 33, 63]
    m = [0, 5, 63, 31, 48, 1, 62, 15]
    b1, v1 = q4_k(sc, m, rng.integers(0, 16, 256))
    b2, v2 = q4_k([63] * 8, [0] * 8, np.full(256, 15), F16_HALF, F16_ONE, 0.5, 1.0)
    rows.append((12, b1 + b2, 512, np.r_[v1, v2]))
    # Q6_K: the +-32 corners and signed scales.
    sc = [1, -1, 127, -128, 2, -3, 5, 7, 1, 1, -1, 64, -64, 9, 11, -13]
    b1, v1 = q6_k(sc, rng.integers(0, 64, 256))
    b2, v2 = q6_k([1] * 16, np.r_[np.zeros(128, dtype=int), np.full(128, 63)])
    rows.append((14, b1 + b2, 512, np.r_[v1, v2]))
    return rows
