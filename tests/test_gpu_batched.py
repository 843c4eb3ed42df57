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


@pytest.fixture(scope="module", params=[W.QWEN3_30B, W.OLMOE, W.QWEN3_NEXT, W.QWEN35, W.OLMOE_Q3],
                ids=lambda s: s.name)
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


def _routing(orc, shape, hl, fx):
    sel, w = zip(*(orc.route(hl.router, f, shape.n_expert, shape.n_used, shape.renorm)[:2] for f in fx))
    return np.stack(sel).astype(np.int32), np.stack(w).astype(np.float32)


@pytest.mark.parametrize("M", [1, 5, 16])
def test_caller_ids_match_single_token(orc, stage, M):
    """hoard_moe_ffn_combine_batched over the oracle's routing, and over a verify-loop
    style selection (raw probabilities, one token padded with a repeated id of weight
    0), gives each token the single-token ffn_combine's bits."""
    shape, hl, st = stage
    fx, res = _tokens(shape, M, 7 * M + 3)
    ids, w = _routing(orc, shape, hl, fx)
    if M > 1:
        ids[1, -2:] = ids[1, 0]  # padding: fewer candidates than n_used
        w[1, -2:] = 0.0
        w[2] *= 1.7  # weights as given: no renormalisation
    print(f"caller ids {shape.name} M={M}", flush=True)
    out = st.ffn_combine_batched(0, fx, ids, w, res)
    for t in range(M):
        one = st.ffn_combine(0, fx[t], ids[t], w[t], res[t])
        assert np.array_equal(one.view(np.uint32), out[t].view(np.uint32)), f"token {t}"
    ref = orc.moe_ffn_combine(hl, fx[0], ids[0], w[0], res[0])
    parity.assert_parity(out[0], ref, "caller ids token 0 vs oracle")


def test_caller_ids_bad_id_poisons_its_token(stage):
    shape, hl, st = stage
    M = 4
    fx, res = _tokens(shape, M, 500)
    ids = np.tile(np.arange(shape.n_used, dtype=np.int32), (M, 1))
    w = np.full((M, shape.n_used), 0.125, np.float32)
    ids[2, 3] = shape.n_expert + 5
    print(f"caller ids bad id {shape.name}", flush=True)
    out = st.ffn_combine_batched(0, fx, ids, w, res)
    assert np.all(np.isnan(out[2]))
    for t in (0, 1, 3):
        one = st.ffn_combine(0, fx[t], ids[t], w[t], res[t])
        assert np.array_equal(one.view(np.uint32), out[t].view(np.uint32))


def test_verify_step_over_the_slot_pool(orc):
    """The verify loop's step on a K-slot pool (src/run_specloop.cpp:116-139): ensure
    every (token, expert) in order, then the batched products over the slots.  Bit-
    identical to the all-resident handle on expert ids; hits and misses as the host
    replay of the same order gives; more distinct experts than slots is refused."""
    import ctypes

    from hoard_amd.runtime import MoEStage
    shape, K, M = W.QWEN3_30B, 40, 4
    hl = W.make_layer(shape, 9, 0)
    ref = MoEStage(shape, n_layer=1, layers={0: hl}, max_tokens=16)
    st = MoEStage(shape, n_layer=1, layers={0: hl}, pool_k=K, max_tokens=16)
    lib = H.load_library()
    rp = ctypes.c_void_p()
    H.check(lib.hoard_slot_lru_create(1, shape.n_expert, K, 2, ctypes.byref(rp)))
    try:
        want_miss = 0
        for step in range(6):
            fx, res = _tokens(shape, M, 1000 + 3 * step)  # overlapping token sets give hits
            ids, w = _routing(orc, shape, hl, fx)
            print(f"verify step {step}: {len(np.unique(ids))} distinct experts", flush=True)
            slots = st.pool_ensure_batched(0, ids)
            rs = np.zeros(ids.size, np.int32)
            rm = np.zeros(ids.size, np.uint8)
            flat = np.ascontiguousarray(ids.ravel())
            H.check(lib.hoard_slot_lru_access(rp, 0, flat.ctypes.data, flat.size, rs.ctypes.data, rm.ctypes.data))
            assert np.array_equal(slots.ravel(), rs)
            want_miss += int(rm.sum())
            got = st.ffn_combine_batched(0, fx, slots, w, res)
            exp = ref.ffn_combine_batched(0, fx, ids, w, res)
            assert np.array_equal(got.view(np.uint32), exp.view(np.uint32)), step
        ps = st.stats()
        assert ps.misses == want_miss and ps.hits + ps.misses == ps.reqs
        many = np.arange(K + 1, dtype=np.int32)
        with pytest.raises(H.HoardError) as ei:
            st.pool_ensure_batched(0, many)
        assert ei.value.code == H.ERR_INVALID
    finally:
        lib.hoard_slot_lru_destroy(rp)
        st.close()
        ref.close()


@pytest.mark.parametrize("E,k", [(8, 2), (2, 1)])
def test_batched_few_experts(orc, E, k):
    """Fewer experts than twice the 8 Q8_K blocks of a 2048-wide fx: the route
    launch is narrower than the block count, and every block must still be
    quantised (each token against the oracle and the single-token path)."""
    from hoard_amd.runtime import MoEStage
    shape = W.Shape(f"e{E}", 5, 2048, E, k, 768, 1, H.TYPE_Q4_K, H.TYPE_Q4_K, H.TYPE_Q6_K, 1)
    hl = W.make_layer(shape, 6, 0)
    st = MoEStage(shape, n_layer=1, layers={0: hl}, max_tokens=16)
    try:
        fx, res = _tokens(shape, 5, 40)
        print(f"batched with {E} experts, top-{k}", flush=True)
        out, sel, _ = st.forward_batched(0, fx, res)
        ref, sel_o, _ = orc.moe_layer_batched(hl, fx, res)
        assert np.array_equal(sel, sel_o)
        for t in range(5):
            o1, _, _ = st.layer(0, fx[t], res[t])
            assert np.array_equal(o1.view(np.uint32), out[t].view(np.uint32)), f"token {t}"
            parity.assert_parity(out[t], ref[t], f"E={E} token {t}")
    finally:
        st.close()


def test_pooled_verify_step_above_256_ids(orc):
    """A pooled verify step of 48 tokens at top-8 (384 ids in one ensure, the
    prefill-sized kernels over slots): bit-identical to the all-resident handle,
    and the pool's hits and misses are the host replay's.  The cap is
    min(max_tokens, 512) * n_used ids; one more is refused."""
    import ctypes

    from hoard_amd.runtime import MoEStage
    shape, M = W.QWEN3_30B, 48
    K = shape.n_expert
    hl = W.make_layer(shape, 9, 0)
    ref = MoEStage(shape, n_layer=1, layers={0: hl}, max_tokens=M)
    st = MoEStage(shape, n_layer=1, layers={0: hl}, pool_k=K, max_tokens=M)
    lib = H.load_library()
    rp = ctypes.c_void_p()
    H.check(lib.hoard_slot_lru_create(1, shape.n_expert, K, 2, ctypes.byref(rp)))
    try:
        for step in range(2):
            fx, res = _tokens(shape, M, 3000 + 17 * step)
            ids, w = _routing(orc, shape, hl, fx)
            print(f"pooled verify step {step}: {ids.size} ids, {len(np.unique(ids))} distinct", flush=True)
            slots = st.pool_ensure_batched(0, ids)
            rs = np.zeros(ids.size, np.int32)
            rm = np.zeros(ids.size, np.uint8)
            flat = np.ascontiguousarray(ids.ravel())
            H.check(lib.hoard_slot_lru_access(rp, 0, flat.ctypes.data, flat.size, rs.ctypes.data, rm.ctypes.data))
            assert np.array_equal(slots.ravel(), rs)
            got = st.ffn_combine_batched(0, fx, slots, w, res)
            exp = ref.ffn_combine_batched(0, fx, ids, w, res)
            assert np.array_equal(got.view(np.uint32), exp.view(np.uint32)), step
            parity.assert_parity(got[0], orc.moe_ffn_combine(hl, fx[0], ids[0], w[0], res[0]), "pooled token 0")
        too_many = np.zeros(M * shape.n_used + 1, np.int32)
        with pytest.raises(H.HoardError) as ei:
            st.pool_ensure_batched(0, too_many)
        assert ei.value.code == H.ERR_INVALID
    finally:
        lib.hoard_slot_lru_destroy(rp)
        st.close()
        ref.close()


@pytest.mark.parametrize("M", [17, 32])
def test_qwen35_verify_sizes_above_16(orc, M):
    """Qwen3.5's Q5_K routed down rows beside its Q6_K shared down in one down
    launch, for groups of more than 16 tokens (the shared group holds all M, so
    its tile takes a second 16-column MFMA pass): every token the single-token
    path's bits, and the batch against the oracle."""
    from hoard_amd.runtime import MoEStage
    shape = W.QWEN35
    hl = W.make_layer(shape, 4, 0)
    st = MoEStage(shape, n_layer=1, layers={0: hl}, max_tokens=32)
    try:
        fx, res = _tokens(shape, M, 40 * M)
        print(f"batched {shape.name} M={M}", flush=True)
        out, sel, _ = st.forward_batched(0, fx, res)
        ref, sel_o, _ = orc.moe_layer_batched(hl, fx, res)
        assert np.array_equal(sel, sel_o)
        for t in range(M):
            o1, s1, _ = st.layer(0, fx[t], res[t])
            assert np.array_equal(s1, sel[t])
            assert np.array_equal(o1.view(np.uint32), out[t].view(np.uint32)), f"token {t}"
            parity.assert_parity(out[t], ref[t], f"batched {shape.name} M={M} token {t}")
    finally:
        st.close()
