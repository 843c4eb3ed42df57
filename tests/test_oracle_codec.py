"""Pins of the oracle's scalar helpers, block codecs and Q8_K quantiser.

Each check is against something the mathematics or the reference's own data
fixes -- numpy's IEEE float16, an independent encoder written from the block
layout, hand-built known answers, the tensor sizes in the reference's GGUF
dump -- never against a retyped copy of the oracle's formula.
"""
import numpy as np
import pytest

import qpack


def test_fp16_to_fp32_exhaustive(orc):
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([orc.fp16_to_fp32(int(b)) for b in bits], dtype=np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_fp32_to_fp16_round_to_nearest_even(orc):
    rng = np.random.default_rng(1)
    xs = np.concatenate([
        rng.normal(0, 0.01, 20000), rng.normal(0, 100, 2000), rng.uniform(-7e4, 7e4, 2000),
        rng.uniform(-1e-7, 1e-7, 2000),  # subnormal range
        [0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26,
         np.inf, -np.inf],
    ]).astype(np.float32)
    # exact ties: halfway between adjacent halves
    h = np.arange(0x0400, 0x7bff, 97, dtype=np.uint16).view(np.float16).astype(np.float32)
    h2 = np.nextafter(h.astype(np.float16), np.float16(np.inf)).astype(np.float32)
    xs = np.concatenate([xs, (h + h2) / 2])
    with np.errstate(over="ignore"):
        ref = xs.astype(np.float16).view(np.uint16)
    got = np.array([orc.fp32_to_fp16(float(x)) for x in xs], dtype=np.uint16)
    assert np.array_equal(got, ref)


def test_nearest_int_is_round_half_even(orc):
    rng = np.random.default_rng(2)
    xs = np.concatenate([rng.uniform(-300, 300, 5000), np.arange(-130, 130) + 0.5]).astype(np.float32)
    got = np.array([orc.nearest_int(float(x)) for x in xs])
    assert np.array_equal(got, np.rint(xs).astype(int))


def test_gguf_dump_tensor_sizes_pin_block_layout():
    """Tensor byte counts from the reference's OLMoE GGUF dump (notes/gguf_dump.txt:52-65):
    ffn_gate_exps q4_K [2048,1024,64] = 75497472, ffn_down_exps q6_K [1024,2048,64] = 110100480,
    attn_k q4_K [2048,2048] = 2359296, attn_v q6_K [2048,2048] = 3440640."""
    from hoard_amd import TYPE_Q4_K, TYPE_Q6_K, expert_bytes
    assert 64 * expert_bytes(TYPE_Q4_K, 1024, 2048) == 75497472
    assert 64 * expert_bytes(TYPE_Q6_K, 2048, 1024) == 110100480
    assert expert_bytes(TYPE_Q4_K, 2048, 2048) == 2359296
    assert expert_bytes(TYPE_Q6_K, 2048, 2048) == 3440640
    assert expert_bytes(TYPE_Q4_K, 1024, 2048) == 1179648  # per-expert stride, src/run_moe_stream.cpp:177


def test_q4_K_decode_of_independent_encoding(orc):
    rng = np.random.default_rng(3)
    for _ in range(200):
        f = qpack.random_q4_K(rng)
        got = orc.dequant(orc.TYPE_Q4_K, qpack.pack_q4_K(*f), 256)
        assert np.array_equal(got.view(np.uint32), qpack.expect_q4_K(*f).view(np.uint32))


def test_q4_K_scale_packing_high_sub_blocks(orc):
    # sub-blocks 4..7 keep their top two bits in other bytes; use scales/mins
    # that need all six bits and distinct values per sub-block
    sc = np.array([1, 2, 3, 4, 63, 48, 33, 17])
    mn = np.array([5, 6, 7, 8, 62, 49, 34, 16])
    q = np.full(256, 1)
    got = orc.dequant(orc.TYPE_Q4_K, qpack.pack_q4_K(1.0, 1.0, sc, mn, q), 256)
    want = np.repeat(sc - mn, 32).astype(np.float32)
    assert np.array_equal(got, want)


def test_q4_K_known_answers(orc):
    z = orc.dequant(orc.TYPE_Q4_K, np.zeros(144, np.uint8), 256)
    assert np.all(z == 0)
    # one nibble = 15 at element 37 (chunk 0, high half, l=5) with its sub-block scale 63
    sc = np.zeros(8, int); sc[1] = 63
    q = np.zeros(256, int); q[37] = 15
    y = orc.dequant(orc.TYPE_Q4_K, qpack.pack_q4_K(0.5, 0.0, sc, np.zeros(8, int), q), 256)
    want = np.zeros(256, np.float32); want[37] = 0.5 * 63 * 15
    assert np.array_equal(y, want)
    # min only: every element of sub-block 6 equals -dmin*m
    mn = np.zeros(8, int); mn[6] = 40
    y = orc.dequant(orc.TYPE_Q4_K, qpack.pack_q4_K(0.0, 0.25, np.zeros(8, int), mn, np.zeros(256, int)), 256)
    want = np.zeros(256, np.float32); want[192:224] = -10.0
    assert np.array_equal(y, want)


def test_q6_K_decode_of_independent_encoding(orc):
    rng = np.random.default_rng(4)
    for _ in range(200):
        f = qpack.random_q6_K(rng)
        got = orc.dequant(orc.TYPE_Q6_K, qpack.pack_q6_K(*f), 256)
        assert np.array_equal(got.view(np.uint32), qpack.expect_q6_K(*f).view(np.uint32))


def test_q6_K_known_answers(orc):
    # q = 0 and 63 extremes, negative scale
    q = np.full(256, 32); q[0] = 0; q[255] = 63; q[100] = 1
    sc = np.ones(16, int); sc[15] = -3
    y = orc.dequant(orc.TYPE_Q6_K, qpack.pack_q6_K(2.0, sc, q), 256)
    want = np.zeros(256, np.float32); want[0] = -64.0; want[255] = 2.0 * -3 * 31; want[100] = -62.0
    assert np.array_equal(y, want)


def test_feasibility_expert_sizes_pin_q3_q5_block_bytes():
    """Per-expert bytes from the reference's model table (notes/FEASIBILITY.md:75,77):
    OLMoE Q3_K gate/up + Q5_K down at n_ff 1024 is 3.09 MB and Qwen3.5-35B-A3B Q4_K
    gate/up + Q5_K down at n_ff 512 is 1.81 MB (MiB, n_embd 2048)."""
    from hoard_amd import TYPE_Q3_K, TYPE_Q4_K, TYPE_Q5_K, expert_bytes
    olmoe = 2 * expert_bytes(TYPE_Q3_K, 1024, 2048) + expert_bytes(TYPE_Q5_K, 2048, 1024)
    qwen35 = 2 * expert_bytes(TYPE_Q4_K, 512, 2048) + expert_bytes(TYPE_Q5_K, 2048, 512)
    assert round(olmoe / 2 ** 20, 2) == 3.09
    assert round(qwen35 / 2 ** 20, 2) == 1.81


def test_q5_K_decode_of_independent_encoding(orc):
    rng = np.random.default_rng(5)
    for _ in range(200):
        f = qpack.random_q5_K(rng)
        got = orc.dequant(orc.TYPE_Q5_K, qpack.pack_q5_K(*f), 256)
        assert np.array_equal(got.view(np.uint32), qpack.expect_q5_K(*f).view(np.uint32))


def test_q5_K_known_answers(orc):
    z = orc.dequant(orc.TYPE_Q5_K, np.zeros(176, np.uint8), 256)
    assert np.all(z == 0)
    # only the fifth bit of element 64*2+32+7 (chunk 2, high half): qh[7] bit 5
    b = np.zeros(176, np.uint8)
    b[0:2] = np.array([qpack.fp16_bits(0.5)], np.uint16).view(np.uint8)
    b[4 + 8 + 1] = 0x0f  # sub-block 5 scale low nibble 15 (byte s+4 = 9 for s = 5)
    b[16 + 7] = 1 << 5
    y = orc.dequant(orc.TYPE_Q5_K, b, 256)
    want = np.zeros(256, np.float32); want[64 * 2 + 32 + 7] = 0.5 * 15 * 16
    assert np.array_equal(y, want)
    # q = 31 everywhere with all scales 63 and mins 0: d * 63 * 31
    q = np.full(256, 31)
    y = orc.dequant(orc.TYPE_Q5_K, qpack.pack_q5_K(0.25, 0.0, np.full(8, 63), np.zeros(8, int), q), 256)
    assert np.all(y == np.float32(0.25 * 63 * 31))


def test_q3_K_decode_of_independent_encoding(orc):
    rng = np.random.default_rng(6)
    for _ in range(200):
        f = qpack.random_q3_K(rng)
        got = orc.dequant(orc.TYPE_Q3_K, qpack.pack_q3_K(*f), 256)
        assert np.array_equal(got.view(np.uint32), qpack.expect_q3_K(*f).view(np.uint32))


def test_q3_K_known_answers(orc):
    # all-zero bytes: scale 0 - 32 = -32 and q3 = 0 - 4 = -4 everywhere -> d * 128
    b = np.zeros(110, np.uint8)
    b[108:110] = np.array([qpack.fp16_bits(1.0)], np.uint16).view(np.uint8)
    assert np.all(orc.dequant(orc.TYPE_Q3_K, b, 256) == 128.0)
    # hmask all set, qs all zero, scales all +32 stored (=0 signed): all zero
    b[0:32] = 0xff
    b[96:104] = 0x00
    b[104:108] = 0xaa  # top bits 2 of every scale -> stored 32 -> signed 0
    assert np.all(orc.dequant(orc.TYPE_Q3_K, b, 256) == 0.0)
    # extremes: scale g = 15 stored 63 (signed 31), q3 = 3 at element 255; scale 0 stored 0 (-32), q3 = -4 at 0
    sc = np.zeros(16, int); sc[15] = 31; sc[0] = -32
    q = np.zeros(256, int); q[255] = 3; q[0] = -4
    y = orc.dequant(orc.TYPE_Q3_K, qpack.pack_q3_K(0.5, sc, q), 256)
    want = np.zeros(256, np.float32); want[255] = 0.5 * 31 * 3; want[0] = 0.5 * -32 * -4
    assert np.array_equal(y, want)


def test_q8_K_special_cases(orc):
    # all-zero block: d = 0, q = 0
    q = orc.quantize_q8k(np.zeros(256, np.float32))
    assert q["d"][0] == 0 and np.all(q["qs"] == 0) and np.all(q["bsums"] == 0)
    # the element of largest |x| maps to -127 and d takes the opposite sign of it
    rng = np.random.default_rng(5)
    x = rng.normal(0, 1, 256).astype(np.float32)
    i = int(np.argmax(np.abs(x)))
    q = orc.quantize_q8k(x)
    assert q["qs"][0][i] == -127
    assert np.sign(q["d"][0]) == -np.sign(x[i])
    # first index wins among equal magnitudes, with its own sign
    x = np.zeros(256, np.float32); x[10] = -4.0; x[20] = 4.0
    q = orc.quantize_q8k(x)
    assert q["qs"][0][10] == -127 and q["qs"][0][20] == 127 and q["d"][0] == np.float32(1.0) / np.float32(-127.0 / -4.0)
    # ties round to even: max = -127 gives iscale = 1 exactly
    x = np.zeros(256, np.float32); x[0] = -127.0; x[1:6] = [2.5, 3.5, -2.5, 0.5, 126.5]
    q = orc.quantize_q8k(x)
    assert list(q["qs"][0][:6]) == [-127, 2, 4, -2, 0, 126]
    assert q["d"][0] == 1.0


def test_q8_K_bounds_and_group_sums(orc):
    rng = np.random.default_rng(6)
    for scale in (1e-3, 1.0, 1e5):
        x = (rng.standard_t(3, 2048) * scale).astype(np.float32)
        q = orc.quantize_q8k(x)
        for b in range(8):
            xb = x[256 * b:256 * (b + 1)].astype(np.float64)
            qb = q["qs"][b].astype(np.float64)
            assert np.all(np.abs(qb) <= 127)
            assert np.array_equal(q["bsums"][b], q["qs"][b].astype(int).reshape(16, 16).sum(1))
            # reconstruction error is at most half a step (plus fp32 rounding of iscale*x)
            err = np.abs(qb * float(q["d"][b]) - xb)
            assert err.max() <= abs(float(q["d"][b])) * (0.5 + 1e-4)
