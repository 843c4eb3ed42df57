"""Batched expert stage (M tokens, grouped by expert, int8 MFMA) through the C ABI.

Each token's result must be the single-token path's bit for bit (the MFMA
produces the same integer sub-block sums), and match the oracle's batched
layer (ggml's mul_mat_id semantics: every token routed and computed
independently) to the parity bar.  The per-expert histogram must count the
(token, slot) pairs of the call.
"""
import numpy as np
import pytest

import hoard_amd as H
import parity
from hoard_amd import workloads as W

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", params=[W.QWEN3_30B, W.OLMOE], ids=lambda s: s.name)
def stage(request):
    from hoard_amd.runtime import MoEStage
    shape = request.param
    layers = {0: W.make_layer(shape, 4, 0)}
    st = MoEStage(shape, n_layer=1, layers=layers, max_tokens=16)
    yield shape, layers[0], st
    st.close()


def _tokens(shape, M, base):
    fx, res = zip(*(W.make_hidden(shape, 4, 0, base + t) for t in range(M)))
    return np.stack(fx), np.stack(res)


@pytest.mark.parametrize("M", [1, 4, 8, 16])
def test_batched_matches_single_token_and_oracle(orc, stage, M):
    shape, hl, st = stage
    fx, res = _tokens(shape, M, 10 * M)
    print(f"batched {shape.name} M={M}", flush=True)
    out, sel, w = st.forward_batched(0, fx, res)
    ref, sel_o, w_o = orc.moe_layer_batched(hl, fx, res)
    assert np.array_equal(sel, sel_o)
    for t in range(M):
        o1, s1, w1 = st.layer(0, fx[t], res[t])
        assert np.array_equal(s1, sel[t]) and np.array_equal(w1.view(np.uint32), w[t].view(np.uint32))
        assert np.array_equal(o1.view(np.uint32), out[t].view(np.uint32)), f"token {t}"
        m = parity.assert_parity(out[t], ref[t], f"batched {shape.name} M={M} token {t}")
    print("   last token", m, flush=True)
    stats = st.stats()
    counts = np.bincount(sel.ravel(), minlength=shape.n_expert)
    assert np.array_equal(np.array(stats.expert_hist[:shape.n_expert]), counts)
    assert stats.last_unique == int((counts > 0).sum())


@pytest.mark.parametrize("M", [11, 12, 16])
def test_batched_large_expert_groups(orc, stage, M):
    """M copies of one token's fx (each with its own residual) put all M tokens
    in each of its k expert groups: 11 runs the per-token dot path at its
    largest group, 12 and 16 the MFMA path."""
    shape, hl, st = stage
    fx1, _ = _tokens(shape, 1, 700 + M)
    _, res = _tokens(shape, M, 800 + M)
    fx = np.repeat(fx1, M, axis=0)
    print(f"batched {shape.name} one token x M={M}", flush=True)
    out, sel, w = st.forward_batched(0, fx, res)
    stats = st.stats()
    assert stats.last_unique == shape.n_used
    assert sorted(set(np.array(stats.expert_hist[:shape.n_expert]).tolist())) == [0, M]
    ref, sel_o, _ = orc.moe_layer_batched(hl, fx, res)
    assert np.array_equal(sel, sel_o)
    for t in (0, M // 2, M - 1):
        o1, s1, _ = st.layer(0, fx[t], res[t])
        assert np.array_equal(s1, sel[t])
        assert np.array_equal(o1.view(np.uint32), out[t].view(np.uint32)), f"token {t}"
        parity.assert_parity(out[t], ref[t], f"batched {shape.name} M={M} token {t}")


def test_batched_aliasing_and_repeated_tokens(stage):
    """out may alias res; identical tokens in one call give identical rows."""
    shape, _, st = stage
    fx, res = _tokens(shape, 3, 500)
    fx = np.concatenate([fx, fx[:1]])
    res = np.concatenate([res, res[:1]])
    out, sel, _ = st.forward_batched(0, fx, res)
    assert np.array_equal(out[0].view(np.uint32), out[3].view(np.uint32))
    fx_d, res_d = st.dev(fx), st.dev(res)
    H.check(st.lib.hoard_moe_forward_batched(st.h, 0, 4, st.ptr(fx_d), st.ptr(res_d), st.ptr(res_d), None, None,
                                             st.stream()))
    torch.cuda.synchronize()
    assert np.array_equal(res_d.cpu().numpy().view(np.uint32), out.view(np.uint32))


def test_batched_rejects_too_many_tokens(stage):
    shape, _, st = stage
    fx, res = _tokens(shape, 17, 900)
    with pytest.raises(H.HoardError):
        st.forward_batched(0, fx, res)
