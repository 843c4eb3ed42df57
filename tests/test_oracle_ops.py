"""Pins of the oracle's dot products, router tail and layer composition.

The integer super-block dots are pinned by an fp64 brute force over operands
whose values come straight from the encoded fields (tests/qpack.py); the
router by an fp64 softmax and a brute-force top-k; the expert FFN and the
combine by an fp64 composition of the separately pinned pieces.  Plausible
slips -- a swapped gate/up, silu on the wrong branch, a wrong expert stride,
a missing min term, renorm on OLMoE -- each fail one of these.
"""
import numpy as np
import pytest

import qpack
from hoard_amd import TYPE_Q3_K, TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K
from hoard_amd import workloads as W


def _fp64_dot_bound(terms):
    return 8 * np.finfo(np.float32).eps * np.sum(np.abs(terms)) + 1e-30


@pytest.mark.parametrize("qtype", [TYPE_Q3_K, TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K])
def test_vec_dot_q_vs_fp64_brute_force(orc, qtype):
    rng = np.random.default_rng(10 + qtype)
    for trial in range(40):
        nb = int(rng.integers(1, 9))
        blocks, vals = [], []
        for _ in range(nb):
            b, v = qpack.random_block(qtype, rng)
            blocks.append(b)
            vals.append(v)
        row = np.concatenate(blocks)
        wv = np.concatenate(vals)
        x = (rng.normal(0, 1, 256 * nb) * (10.0 ** rng.integers(-2, 4))).astype(np.float32)
        q8 = orc.quantize_q8k(x)
        xv = orc.dequant_q8k(q8)
        terms = wv * xv
        got = orc.vec_dot_q(qtype, row, q8)
        assert abs(got - terms.sum()) <= _fp64_dot_bound(terms), (trial, got, terms.sum())


def test_vec_dot_q4_K_min_term_matters(orc):
    # all quants zero: the dot reduces to -dmin * sum_s m_s * sum_{sub-block} x
    rng = np.random.default_rng(11)
    mn = rng.integers(1, 64, 8)
    row = qpack.pack_q4_K(0.0, 0.5, np.zeros(8, int), mn, np.zeros(256, int))
    q8 = orc.quantize_q8k(rng.normal(0, 1, 256).astype(np.float32))
    xv = orc.dequant_q8k(q8)
    want = -0.5 * sum(mn[s] * xv[32 * s:32 * s + 32].sum() for s in range(8))
    assert np.isclose(orc.vec_dot_q(TYPE_Q4_K, row, q8), want, rtol=1e-6)


def test_vec_dot_q5_K_min_and_fifth_bit(orc):
    # quants 16 (fifth bit only) with unit scales: the dot is d*16*sum(x) - dmin*sum_s m_s*sum_s(x)
    rng = np.random.default_rng(13)
    mn = rng.integers(1, 64, 8)
    row = qpack.pack_q5_K(0.125, 0.5, np.ones(8, int), mn, np.full(256, 16))
    q8 = orc.quantize_q8k(rng.normal(0, 1, 256).astype(np.float32))
    xv = orc.dequant_q8k(q8)
    want = 0.125 * 16 * xv.sum() - 0.5 * sum(mn[s] * xv[32 * s:32 * s + 32].sum() for s in range(8))
    assert np.isclose(orc.vec_dot_q(TYPE_Q5_K, row, q8), want, rtol=1e-6)


def test_vec_dot_f32_vs_fp64(orc):
    rng = np.random.default_rng(12)
    for n in (32, 256, 2048, 2048 + 7):
        x = rng.normal(0, 1, n).astype(np.float32)
        y = rng.normal(0, 1, n).astype(np.float32)
        terms = x.astype(np.float64) * y
        assert abs(orc.vec_dot_f32(x, y) - terms.sum()) <= _fp64_dot_bound(terms) * 4


@pytest.mark.parametrize("shape", [W.OLMOE, W.QWEN3_30B, W.QWEN3_NEXT], ids=lambda s: s.name)
def test_route_vs_fp64_and_brute_force_topk(orc, shape):
    rng = np.random.default_rng(13)
    E, k, n = shape.n_expert, shape.n_used, shape.n_embd
    for _ in range(5):
        wr = rng.normal(0, 0.02, (E, n)).astype(np.float32)
        fx = W.rms_norm(rng.normal(0, 1, n).astype(np.float32))
        sel, w, p = orc.route(wr, fx, E, k, shape.renorm)
        lg = wr.astype(np.float64) @ fx.astype(np.float64)
        p64 = np.exp(lg - lg.max())
        p64 /= p64.sum()
        assert np.allclose(p, p64, rtol=2e-5, atol=1e-9)
        assert abs(p.astype(np.float64).sum() - 1.0) < 1e-5
        brute = sorted(range(E), key=lambda e: (-p[e], e))[:k]
        assert list(sel) == brute
        raw = p[sel]
        if shape.renorm:
            assert np.allclose(w, raw / raw.astype(np.float64).sum(), rtol=1e-6)
            assert abs(w.astype(np.float64).sum() - 1.0) < 1e-5
        else:
            assert np.array_equal(w, raw)  # OLMoE: no renorm (src/run_moe_stream.cpp:150)


def test_route_ties_take_lower_index(orc):
    n, E = 256, 16
    wr = np.zeros((E, n), np.float32)
    for e in (3, 7, 11, 12):
        wr[e, 0] = 1.0       # four experts share the top logit
    wr[5, 0] = 0.5
    fx = np.zeros(n, np.float32); fx[0] = 1.0
    sel, w, p = orc.route(wr, fx, E, 5, 0)
    assert list(sel) == [3, 7, 11, 12, 5]


def test_route_renorm_of_uniform_probabilities(orc):
    # all-equal logits: probabilities 1/E; top-k takes the k lowest indices and
    # renorm makes each weight 1/k (the 6.103515625e-5 clamp of
    # src/run_moe_stream.cpp:372 cannot bind: a top-k sum is at least k/E >= 1/1024)
    n, E = 256, 4
    sel, w, p = orc.route(np.zeros((E, n), np.float32), np.zeros(n, np.float32), E, 2, 1)
    assert list(sel) == [0, 1] and np.allclose(p, 0.25) and np.allclose(w, [0.5, 0.5])


def _fp64_expert(orc, shape, gate, up, down, fx):
    """fp64 composition of separately pinned parts, with Q8_K activations."""
    nf, ne = shape.n_ff, shape.n_embd
    gw = orc.dequant(shape.gate_type, gate, nf * ne).reshape(nf, ne).astype(np.float64)
    uw = orc.dequant(shape.up_type, up, nf * ne).reshape(nf, ne).astype(np.float64)
    dw = orc.dequant(shape.down_type, down, ne * nf).reshape(ne, nf).astype(np.float64)
    xq = orc.dequant_q8k(orc.quantize_q8k(fx))
    g, u = gw @ xq, uw @ xq
    h = g / (1.0 + np.exp(-g)) * u
    hq = orc.dequant_q8k(orc.quantize_q8k(h.astype(np.float32)))
    return dw @ hq


def _cmp(got, ref):
    got = got.astype(np.float64)
    err = np.abs(got - ref).max() / np.abs(ref).max()
    cos = got @ ref / np.linalg.norm(got) / np.linalg.norm(ref)
    return err, cos


@pytest.mark.parametrize("shape", [W.OLMOE, W.QWEN3_30B, W.QWEN3_NEXT, W.QWEN35, W.OLMOE_Q3],
                         ids=lambda s: s.name)
def test_moe_layer_vs_fp64_composition(orc, shape):
    hl = W.make_layer(shape, 0, 0)
    fx, res = W.make_hidden(shape, 0, 0)
    out, sel, w = orc.moe_layer(hl, fx, res)
    sel_r, w_r, _ = orc.route(hl.router, fx, shape.n_expert, shape.n_used, shape.renorm)
    assert np.array_equal(sel, sel_r) and np.array_equal(w, w_r)
    gs, us, ds = hl.stride("gate"), hl.stride("up"), hl.stride("down")
    y = np.zeros(shape.n_embd)
    for j, e in enumerate(sel):
        y += float(w[j]) * _fp64_expert(orc, shape, hl.gate[e * gs:(e + 1) * gs], hl.up[e * us:(e + 1) * us],
                                        hl.down[e * ds:(e + 1) * ds], fx)
    if shape.n_ff_shexp:
        shs = W.Shape("sh", 0, shape.n_embd, 1, 1, shape.n_ff_shexp, 0, shape.sh_gate_type, shape.sh_up_type,
                      shape.sh_down_type, 1)
        ysh = _fp64_expert(orc, shs, hl.sh_gate, hl.sh_up, hl.sh_down, fx)
        sg = 1.0 / (1.0 + np.exp(-(hl.sh_gate_inp.astype(np.float64) @ fx)))
        y += sg * ysh
    y += res
    err, cos = _cmp(out, y)
    assert cos >= 0.99999 and err <= 5e-4, (err, cos)


def test_moe_layer_batched_is_per_token(orc):
    shape = W.QWEN3_30B
    hl = W.make_layer(shape, 0, 0)
    toks = [W.make_hidden(shape, 0, 0, t) for t in range(4)]
    fx = np.stack([t[0] for t in toks])
    res = np.stack([t[1] for t in toks])
    out, sel, w = orc.moe_layer_batched(hl, fx, res)
    for t in range(4):
        o1, s1, w1 = orc.moe_layer(hl, fx[t], res[t])
        assert np.array_equal(out[t], o1) and np.array_equal(sel[t], s1) and np.array_equal(w[t], w1)


def test_rms_norm(orc):
    rng = np.random.default_rng(14)
    x = (rng.normal(0, 1, 2048) * 1e3).astype(np.float32)
    y = orc.rms_norm(x, 1e-6)
    ref = x / np.sqrt((x.astype(np.float64) ** 2).mean() + 1e-6)
    assert np.allclose(y, ref, rtol=1e-6)
    assert np.array_equal(y, W.rms_norm(x, 1e-6))
