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
