"""Batches of 17..512 tokens: up to 32 the verify-sized path's expert groups (per-token
dots, or int8 MFMA in 16-column passes), above 32 the sorted-pair expert GEMM on int8 MFMA.

The counterpart of ggml_mul_mat_id over all T prompt tokens (src/run_m1.cpp:93-108).
Each token's result must be the single-token path's bit for bit (the folded MFMA
operands give the per-token integer sub-block sums exactly) and match the oracle's
batched layer (every token routed and computed independently) to the parity bar;
the per-expert histogram must count the call's (token, slot) pairs.

Shapes: Qwen3-30B (Q4_K gate/up, Q6_K down), OLMoE (all Q4_K), Qwen3-Next (a
shared expert), Qwen3.5 (Q5_K routed down rows beside a Q6_K shared expert) and
OLMoE in its Q3_K_M form (Q3_K gate/up, Q5_K down).
"""
import numpy as np
import pytest

import hoard_amd as H
import parity
from hoard_amd import workloads as W

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", params=[W.QWEN3_30B, W.OLMOE, W.QWEN3_NEXT, W.QWEN35, W.OLMOE_Q3],
                ids=lambda s: s.name)
def stage(request):
    from hoard_amd.runtime import MoEStage
    shape = request.param
    layers = {0: W.make_layer(shape, 8, 0)}
    st = MoEStage(shape, n_layer=1, layers=layers, max_tokens=512)
    yield shape, layers[0], st
    st.close()


def _tokens(shape, M, base, same=None):
    fx, res = zip(*(W.make_hidden(shape, 8, 0, base + t) for t in range(M)))
    fx = np.stack(fx)
    if same is not None:  # every token's fx one of `same` hiddens: large expert groups
        fx = fx[np.arange(M) % same]
    return fx, np.stack(res)


def _check(orc, st, shape, hl, fx, res, out, sel, w, what, every=1):
    ref, sel_o, _ = orc.moe_layer_batched(hl, fx, res)
    assert np.array_equal(sel, sel_o), what
    worst = {"max_rel": 0.0, "cos": 1.0}
    for t in range(0, fx.shape[0], every):
        o1, s1, w1 = st.layer(0, fx[t], res[t])
        assert np.array_equal(s1, sel[t]) and np.array_equal(w1.view(np.uint32), w[t].view(np.uint32)), (what, t)
        assert np.array_equal(o1.view(np.uint32), out[t].view(np.uint32)), f"{what}: token {t}"
    for t in range(fx.shape[0]):
        m = parity.assert_parity(out[t], ref[t], f"{what} token {t}")
        worst = {"max_rel": max(worst["max_rel"], m["max_rel"]), "cos": min(worst["cos"], m["cos"])}
    return worst


@pytest.mark.parametrize("M", [17, 32, 33, 128, 512])
def test_prefill_matches_single_token_and_oracle(orc, stage, M):
    shape, hl, st = stage
    fx, res = _tokens(shape, M, 1000 + M)
    print(f"prefill {shape.name} M={M}", flush=True)
    out, sel, w = st.forward_batched(0, fx, res)
    worst = _check(orc, st, shape, hl, fx, res, out, sel, w, f"prefill {shape.name} M={M}",
                   every=1 if M <= 128 else 3)
    print("   worst", worst, flush=True)
    stats = st.stats()
    counts = np.bincount(sel.ravel(), minlength=shape.n_expert)
    assert np.array_equal(np.array(stats.expert_hist[:shape.n_expert]), counts)
    assert stats.last_unique == int((counts > 0).sum())


@pytest.mark.parametrize("M,same", [(20, 1), (30, 2), (32, 1), (200, 1), (300, 3)],
                         ids=["20x1", "30x2", "32x1", "200x1", "300x3"])
def test_prefill_large_expert_groups(orc, stage, M, same):
    """Tokens sharing a few hiddens.  Up to 32 tokens the groups (15, 20 or 32
    tokens) run on MFMA in one or two 16-column passes over each weight tile;
    above, groups of 100-300 tokens are cut into several 64-pair units each."""
    shape, hl, st = stage
    fx, res = _tokens(shape, M, 3000 + M, same=same)
    print(f"prefill {shape.name} M={M}, {same} distinct hiddens", flush=True)
    out, sel, w = st.forward_batched(0, fx, res)
    assert st.stats().last_unique <= same * shape.n_used
    _check(orc, st, shape, hl, fx, res, out, sel, w, f"groups {shape.name} M={M}", every=7)


def test_prefill_caller_ids(orc, stage):
    """hoard_moe_ffn_combine_batched at M = 100: the oracle's routing, raw weights,
    tokens padded with a repeated id of weight 0, and one token with an id out of
    range (NaN row, the others unaffected); each token equals ffn_combine's bits."""
    shape, hl, st = stage
    M = 100
    fx, res = _tokens(shape, M, 5000)
    sel, w = zip(*(orc.route(hl.router, f, shape.n_expert, shape.n_used, shape.renorm)[:2] for f in fx))
    ids, w = np.stack(sel).astype(np.int32), np.stack(w).astype(np.float32)
    ids[3, -3:] = ids[3, 0]
    w[3, -3:] = 0.0
    w[10] *= 1.7
    ids[57, 2] = shape.n_expert + 5
    print(f"prefill caller ids {shape.name} M={M}", flush=True)
    out = st.ffn_combine_batched(0, fx, ids, w, res)
    assert np.all(np.isnan(out[57]))
    for t in range(M):
        if t == 57:
            continue
        o1 = st.ffn_combine(0, fx[t], ids[t], w[t], res[t])
        assert np.array_equal(o1.view(np.uint32), out[t].view(np.uint32)), f"token {t}"
        ref = orc.moe_ffn_combine(hl, fx[t], ids[t], w[t], res[t])
        parity.assert_parity(out[t], ref, f"caller ids token {t}")


def test_prefill_rejects_too_many_tokens(stage):
    shape, _, st = stage
    fx, res = _tokens(shape, 513, 7000)
    with pytest.raises(H.HoardError):
        st.forward_batched(0, fx, res)


def test_prefill_non_finite_token():
    """A token with a NaN in fx: its row is NaN (its selection out of range, its
    expert pairs joined once to expert 0's group), every other token is exact."""
    from hoard_amd.runtime import MoEStage
    shape = W.QWEN3_30B
    hl = W.make_layer(shape, 9, 0)
    st = MoEStage(shape, n_layer=1, layers={0: hl}, max_tokens=64)
    try:
        fx, res = _tokens(shape, 40, 9000)
        fx[7, 11] = np.nan
        out, sel, _ = st.forward_batched(0, fx, res)
        assert np.all(np.isnan(out[7])) and np.all(sel[7] == 2**31 - 1)
        for t in (0, 6, 8, 39):
            o1, _, _ = st.layer(0, fx[t], res[t])
            assert np.array_equal(o1.view(np.uint32), out[t].view(np.uint32)), t
    finally:
        st.close()
