"""Independent ggml K-quant block ENCODERS, written from the block layouts.

The oracle only decodes; these pack chosen integer fields into bytes, so a
decode(encode(fields)) == fields check pins the decoder's index arithmetic
(sub-block order, nibble halves, the 6-bit scale packing, qh bit pairs)
without restating the decoder.  Layouts (ggml-common.h):

block_q4_K (144 B): d fp16 | dmin fp16 | scales[12] | qs[128]
  scales: sub-block s<4 -> bytes s (scale) and s+4 (min), low 6 bits;
          s>=4 -> low 4 bits in byte s+4 (scale low nibble, min high nibble),
          top 2 bits in the top 2 bits of byte s-4 (scale) and byte s (min).
  qs: element 64c+l (l<32) is the low nibble of qs[32c+l], element 64c+32+l
      the high nibble.
block_q6_K (210 B): ql[128] | qh[64] | scales int8[16] | d fp16
  element 128n + 32i + l: low 4 bits in ql[64n + 32*(i&1) + l] (low nibble for
  i<2, high for i>=2), high 2 bits in bits 2i..2i+1 of qh[32n + l].
block_q5_K (176 B): d fp16 | dmin fp16 | scales[12] (packed as in q4_K) |
  qh[32] | qs[128]; element 64c+l / 64c+32+l: low / high nibble of qs[32c+l],
  fifth bit = bit 2c / 2c+1 of qh[l].
block_q3_K (110 B): hmask[32] | qs[64] | scales[12] | d fp16
  element 128n + 32j + l: 2 bits at bit 2j of qs[32n + l], high bit = bit
  4n+j of hmask[l] (set: q3 = q2, clear: q3 = q2 - 4); 16 scales of 6 bits,
  stored as scale+32: low nibbles in bytes 0..7 (scale g<8 low nibble of byte
  g, g>=8 high nibble of byte g-8), top 2 bits in bytes 8..11 (byte 8 + g%4,
  bit pair g//4).
"""
from __future__ import annotations

import numpy as np


def fp16_bits(x: float) -> int:
    return int(np.array([x], dtype=np.float16).view(np.uint16)[0])


def pack_q4_K(d: float, dmin: float, sc, mn, q) -> np.ndarray:
    sc, mn, q = np.asarray(sc, int), np.asarray(mn, int), np.asarray(q, int)
    assert sc.shape == (8,) and mn.shape == (8,) and q.shape == (256,)
    assert sc.min() >= 0 and sc.max() < 64 and mn.min() >= 0 and mn.max() < 64
    assert q.min() >= 0 and q.max() < 16
    b = np.zeros(144, dtype=np.uint8)
    b[0:2] = np.array([fp16_bits(d)], dtype=np.uint16).view(np.uint8)
    b[2:4] = np.array([fp16_bits(dmin)], dtype=np.uint16).view(np.uint8)
    s = np.zeros(12, dtype=int)
    for j in range(4):
        s[j] = sc[j] | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = mn[j] | ((mn[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    b[4:16] = s
    for c in range(4):
        for l in range(32):
            b[16 + 32 * c + l] = q[64 * c + l] | (q[64 * c + 32 + l] << 4)
    return b


def expect_q4_K(d: float, dmin: float, sc, mn, q) -> np.ndarray:
    """Dequantised values in fp32 as written: (d*sc)*q - (dmin*m)."""
    d32 = np.float32(np.float16(d))
    m32 = np.float32(np.float16(dmin))
    out = np.empty(256, dtype=np.float32)
    for k in range(256):
        s = k // 32
        out[k] = np.float32(np.float32(d32 * np.float32(sc[s])) * np.float32(q[k])) - np.float32(m32 * np.float32(mn[s]))
    return out


def pack_q6_K(d: float, sc, q) -> np.ndarray:
    sc, q = np.asarray(sc, int), np.asarray(q, int)
    assert sc.shape == (16,) and q.shape == (256,)
    assert sc.min() >= -128 and sc.max() < 128 and q.min() >= 0 and q.max() < 64
    b = np.zeros(210, dtype=np.uint8)
    for n in range(2):
        for l in range(32):
            e = [128 * n + 32 * i + l for i in range(4)]
            b[64 * n + l] = (q[e[0]] & 15) | ((q[e[2]] & 15) << 4)
            b[64 * n + 32 + l] = (q[e[1]] & 15) | ((q[e[3]] & 15) << 4)
            b[128 + 32 * n + l] = ((q[e[0]] >> 4) | ((q[e[1]] >> 4) << 2) | ((q[e[2]] >> 4) << 4)
                                   | ((q[e[3]] >> 4) << 6))
    b[192:208] = sc.astype(np.int8).view(np.uint8)
    b[208:210] = np.array([fp16_bits(d)], dtype=np.uint16).view(np.uint8)
    return b


def expect_q6_K(d: float, sc, q) -> np.ndarray:
    d32 = np.float32(np.float16(d))
    return np.array([np.float32(np.float32(d32 * np.float32(sc[k // 16])) * np.float32(q[k] - 32))
                     for k in range(256)], dtype=np.float32)


def random_q4_K(rng, dscale=0.01):
    d = float(abs(rng.normal(0, dscale)))
    dmin = float(abs(rng.normal(0, dscale)))
    return d, dmin, rng.integers(0, 64, 8), rng.integers(0, 64, 8), rng.integers(0, 16, 256)


def random_q6_K(rng, dscale=0.01):
    return float(abs(rng.normal(0, dscale))), rng.integers(-128, 128, 16), rng.integers(0, 64, 256)


def fields_value_q4_K(d, dmin, sc, mn, q) -> np.ndarray:
    """fp64 value of each element straight from the fields."""
    d64, m64 = float(np.float16(d)), float(np.float16(dmin))
    s = np.arange(256) // 32
    return d64 * np.asarray(sc, float)[s] * np.asarray(q, float) - m64 * np.asarray(mn, float)[s]


def fields_value_q6_K(d, sc, q) -> np.ndarray:
    d64 = float(np.float16(d))
    return d64 * np.asarray(sc, float)[np.arange(256) // 16] * (np.asarray(q, float) - 32)


def pack_q5_K(d: float, dmin: float, sc, mn, q) -> np.ndarray:
    sc, mn, q = np.asarray(sc, int), np.asarray(mn, int), np.asarray(q, int)
    assert q.shape == (256,) and q.min() >= 0 and q.max() < 32
    b = np.zeros(176, dtype=np.uint8)
    # header and scales as a q4_K block with the low nibbles, then qh / qs
    head = pack_q4_K(d, dmin, sc, mn, q & 15)
    b[0:16] = head[0:16]
    b[48:176] = head[16:144]
    qh = np.zeros(32, dtype=int)
    for k in range(256):
        c, half, l = k // 64, (k // 32) % 2, k % 32
        qh[l] |= (q[k] >> 4) << (2 * c + half)
    b[16:48] = qh
    return b


def expect_q5_K(d: float, dmin: float, sc, mn, q) -> np.ndarray:
    return expect_q4_K(d, dmin, sc, mn, q)  # same fp32 expression, q now 0..31


def pack_q3_K(d: float, sc, q) -> np.ndarray:
    """sc: 16 signed scales in -32..31; q: 256 values in -4..3."""
    sc, q = np.asarray(sc, int), np.asarray(q, int)
    assert sc.shape == (16,) and q.shape == (256,)
    assert sc.min() >= -32 and sc.max() < 32 and q.min() >= -4 and q.max() < 4
    b = np.zeros(110, dtype=np.uint8)
    hm, qs = np.zeros(32, dtype=int), np.zeros(64, dtype=int)
    for k in range(256):
        n, j, l = k // 128, (k // 32) % 4, k % 32
        v = q[k] + 4 if q[k] < 0 else q[k]  # 2-bit part
        if q[k] >= 0:
            hm[l] |= 1 << (4 * n + j)
        qs[32 * n + l] |= v << (2 * j)
    u = sc + 32
    sb = np.zeros(12, dtype=int)
    for g in range(16):
        if g < 8:
            sb[g] |= u[g] & 15
        else:
            sb[g - 8] |= (u[g] & 15) << 4
        sb[8 + g % 4] |= (u[g] >> 4) << (2 * (g // 4))
    b[0:32], b[32:96], b[96:108] = hm, qs, sb
    b[108:110] = np.array([fp16_bits(d)], dtype=np.uint16).view(np.uint8)
    return b


def expect_q3_K(d: float, sc, q) -> np.ndarray:
    """(d*sc)*q3 in fp32."""
    d32 = np.float32(np.float16(d))
    return np.array([np.float32(np.float32(d32 * np.float32(sc[k // 16])) * np.float32(q[k]))
                     for k in range(256)], dtype=np.float32)


def random_q5_K(rng, dscale=0.01):
    d = float(abs(rng.normal(0, dscale)))
    dmin = float(abs(rng.normal(0, dscale)))
    return d, dmin, rng.integers(0, 64, 8), rng.integers(0, 64, 8), rng.integers(0, 32, 256)


def random_q3_K(rng, dscale=0.01):
    return float(abs(rng.normal(0, dscale))), rng.integers(-32, 32, 16), rng.integers(-4, 4, 256)


def fields_value_q5_K(d, dmin, sc, mn, q) -> np.ndarray:
    return fields_value_q4_K(d, dmin, sc, mn, q)


def fields_value_q3_K(d, sc, q) -> np.ndarray:
    d64 = float(np.float16(d))
    return d64 * np.asarray(sc, float)[np.arange(256) // 16] * np.asarray(q, float)


def random_block(qtype: int, rng):
    """(bytes, fp64 values) of a random block of ggml type qtype."""
    if qtype == 11:
        f = random_q3_K(rng)
        return pack_q3_K(*f), fields_value_q3_K(*f)
    if qtype == 12:
        f = random_q4_K(rng)
        return pack_q4_K(*f), fields_value_q4_K(*f)
    if qtype == 13:
        f = random_q5_K(rng)
        return pack_q5_K(*f), fields_value_q5_K(*f)
    f = random_q6_K(rng)
    return pack_q6_K(*f), fields_value_q6_K(*f)
