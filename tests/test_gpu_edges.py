"""Edge cases of the stage on the device, each against the oracle or a stated rule:

* exact router ties at the k / k+1 boundary (and a three-way tie straddling it):
  the lower expert index wins, the rule of src/run_moe_stream.cpp:355 as built
  here, in all four top-k implementations (the per-layer route kernel's wave
  tail, the expert-per-XCD kernel's rank pass, the rows-spread kernel's bitwise
  search, the batched router);
* special values: an all-zero 256-element block of fx (Q8_K scale 0), weight
  super-blocks with d = dmin = 0, a selected expert whose gate and up rows are all
  zero (every block of h zero), NaN and infinity in the input;
* the failure paths forced from the host: a wait limit of 0 makes the one-launch
  decode's bounded waits give up (NaN rows, hoard_moe_sync_check reports
  HOARD_ERR_HIP, the next call is correct), and a slot upload that fails leaves
  the pool consistent.

NaN / infinity rule: a non-finite element of the router input makes every
router probability NaN, so the selection comes back as INT32_MAX (no expert)
with weight NaN and the token's output row is NaN, on every path; no call
faults or waits out its bound.  In the expert products alone
(hoard_moe_ffn_combine with the caller's ids) a NaN element of fx quantises to
0, as ggml's quantize_row_q8_K does (nearest_int of a NaN), so the output is
finite and equals the oracle's; an infinite element zeroes every expert's
output (see the test), so the output is the residual, again as the oracle's.
"""
import dataclasses

import numpy as np
import pytest

import hoard_amd as H
import parity
from hoard_amd import workloads as W

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

INT32_MAX = 2**31 - 1


def _stage(shape, layers, n_layer=None, **kw):
    from hoard_amd.runtime import MoEStage
    return MoEStage(shape, n_layer=n_layer or max(layers, default=0) + 1, layers=layers, **kw)


def _order(orc, shape, router, fx):
    """Experts by oracle probability, best first (lower index first on ties)."""
    _, _, p = orc.route(router, fx, shape.n_expert, shape.n_used, shape.renorm)
    return np.lexsort((np.arange(shape.n_expert), -np.asarray(p, np.float64)))


def _tie(orc, shape, router, fx, lower: bool, ways: int = 2):
    """Copy the router row of a boundary expert A (the k-th best, or the
    (k-1)-th where no expert below the top k sits on the wanted side of A's
    index) onto ways-1 experts ranked below the top k, all with a lower (or all
    a higher) index than A, so that their logits equal A's bit for bit and the
    tied group straddles the k / k+1 boundary.  Returns (router, tied group
    sorted by index, how many of the group the top k takes)."""
    k = shape.n_used
    order = _order(orc, shape, router, fx)
    for pos in (k - 1, k - 2):
        a = int(order[pos])
        below = [int(e) for e in order[k:] if (int(e) < a) == lower]
        if len(below) >= ways - 1:
            break
    assert len(below) >= ways - 1
    r = router.reshape(shape.n_expert, shape.n_embd).copy()
    for b in below[:ways - 1]:
        r[b] = r[a]
    return r.reshape(-1), sorted([a] + below[:ways - 1]), k - pos


def _expect_tie_rule(orc, shape, router, fx, tied, n_sel):
    """The oracle's selection on the tied router takes the n_sel lowest indices of
    the tied group and none of the others."""
    sel_o, w_o, p = orc.route(router, fx, shape.n_expert, shape.n_used, shape.renorm)
    assert len(set(p[tied].tolist())) == 1, "the copied rows must tie exactly"
    s = sel_o.tolist()
    assert all(e in s for e in tied[:n_sel]) and all(e not in s for e in tied[n_sel:]), (sel_o, tied, n_sel)
    return sel_o, w_o


TIE_CASES = [(True, 2), (False, 2), (True, 3), (False, 3)]
TIE_IDS = ["lower-2way", "higher-2way", "lower-3way", "higher-3way"]


@pytest.mark.parametrize("shape", [W.QWEN3_30B, W.QWEN3_NEXT, W.OLMOE, W.QWEN35], ids=lambda s: s.name)
def test_route_tie_at_boundary(orc, shape):
    """hoard_moe_route (and hoard_moe_layer) on routers with exact ties at k / k+1."""
    st = _stage(shape, {})
    try:
        for case, (lower, ways) in enumerate(TIE_CASES):
            fx, res = W.make_hidden(shape, 21, 0, case)
            router, tied, n_sel = _tie(orc, shape, W.make_router(shape, 21, case), fx, lower, ways)
            sel_o, w_o = _expect_tie_rule(orc, shape, router, fx, tied, n_sel)
            hl = W.make_layer(shape, 21, case, experts=sorted(set(sel_o.tolist()) | set(tied)))
            hl.router[:] = router
            st.set_layer(0, hl)
            print(f"route tie {shape.name} {TIE_IDS[case]} tied={tied} taken={n_sel}", flush=True)
            sel, w = st.route(0, fx)
            assert np.array_equal(sel, sel_o), (sel, sel_o)
            assert np.allclose(w, w_o, rtol=1e-6, atol=0)
            out, sel2, _ = st.layer(0, fx, res)
            assert np.array_equal(sel2, sel_o)
            ref, _, _ = orc.moe_layer(hl, fx, res)
            parity.assert_parity(out, ref, f"tie layer {shape.name} {TIE_IDS[case]}")
    finally:
        st.close()


def _decode_tie(orc, shape, kernel):
    """One-launch decode (kernel 1: expert per XCD, 2: rows spread) of a layer with
    an exact tie at the boundary: the output must be the oracle's for the lower
    index, and the oracle's output for the higher index must fail the bar (so a
    wrongly broken tie cannot pass)."""
    st = _stage(shape, {})
    try:
        st.set_option(H.OPT_DECODE_KERNEL, kernel)
        st.set_option(H.OPT_PERSISTENT_DECODE, 2)
        for case, (lower, ways) in enumerate(TIE_CASES):
            _, x = W.make_hidden(shape, 22, 0, case)
            fx = orc.rms_norm(x, W.RMS_EPS)
            router, tied, n_sel = _tie(orc, shape, W.make_router(shape, 22, case), fx, lower, ways)
            sel_o, w_o = _expect_tie_rule(orc, shape, router, fx, tied, n_sel)
            hl = W.make_layer(shape, 22, case, experts=sorted(set(sel_o.tolist()) | set(tied)))
            hl.router[:] = router
            st.set_layer(0, hl)
            print(f"decode tie {shape.name} kernel {kernel} {TIE_IDS[case]} tied={tied} taken={n_sel}", flush=True)
            y = st.decode(x, 0, 1, W.RMS_EPS)
            st.sync_check()
            ref, _, _ = orc.moe_layer(hl, fx, x)
            parity.assert_parity(y, ref, f"decode tie {TIE_IDS[case]}")
            wrong = sel_o.copy()  # the last taken member of the group swapped for the first left out
            wrong[wrong == tied[n_sel - 1]] = tied[n_sel]
            alt = orc.moe_ffn_combine(hl, fx, wrong, w_o, x)
            m = parity.metrics(alt, ref)
            assert m["max_rel"] > parity.MAX_REL, ("the tie would not be detected", m)
    finally:
        st.close()


def test_decode_xcd_tie_at_boundary(orc):
    _decode_tie(orc, W.QWEN3_30B, 1)


@pytest.mark.parametrize("shape", [W.QWEN3_30B, W.QWEN3_NEXT], ids=lambda s: s.name)
def test_decode_spread_tie_at_boundary(orc, shape):
    _decode_tie(orc, shape, 2)


def test_batched_route_tie_at_boundary(orc):
    """Six tokens routed together on a router with a boundary tie for each token
    (rows copied one token after another onto experts no earlier tie touched): the
    batched router's selection is the oracle's, and at least half of the ties still
    straddle their token's boundary once all rows are in place."""
    shape = W.QWEN3_30B
    M = 6
    toks = [W.make_hidden(shape, 23, 0, t) for t in range(M)]
    r = W.make_router(shape, 23, 0).reshape(shape.n_expert, shape.n_embd).copy()
    used, ties = set(), []
    for t, (fx, _) in enumerate(toks):
        order = _order(orc, shape, r.reshape(-1), fx)
        a = int(order[shape.n_used - 1])
        b = next(int(e) for e in order[shape.n_used:] if int(e) not in used and (int(e) < a) == (t % 2 == 0))
        r[b] = r[a]
        used |= {a, b}
        ties.append(sorted([a, b]))
    router = r.reshape(-1)
    sel_o = []
    straddling = 0
    for (fx, _), tied in zip(toks, ties):
        s_o, _, p = orc.route(router, fx, shape.n_expert, shape.n_used, shape.renorm)
        assert p[tied[0]] == p[tied[1]]
        if tied[0] in s_o.tolist() and tied[1] not in s_o.tolist():
            straddling += 1
        assert not (tied[1] in s_o.tolist() and tied[0] not in s_o.tolist()), "lower index first"
        sel_o.append(s_o)
    assert straddling >= M // 2, straddling
    hl = W.make_layer(shape, 23, 0)
    hl.router[:] = router
    st = _stage(shape, {0: hl}, max_tokens=16)
    try:
        fx = np.stack([f for f, _ in toks])
        res = np.stack([x for _, x in toks])
        print("batched tie", ties, f"straddling {straddling}", flush=True)
        out, sel, _ = st.forward_batched(0, fx, res)
        assert np.array_equal(sel, np.stack(sel_o)), (sel, sel_o)
        ref, _, _ = orc.moe_layer_batched(hl, fx, res)
        for t in range(M):
            parity.assert_parity(out[t], ref[t], f"batched tie token {t}")
    finally:
        st.close()


# ---- special values ----------------------------------------------------------

def _zero_d(hl, which: str, expert: int, rows, blocks=None):
    """Set d (and dmin, for Q4_K) of the given rows' super-blocks of one expert to +0."""
    s = hl.shape
    qtype = {"gate": s.gate_type, "up": s.up_type, "down": s.down_type}[which]
    cols = s.n_ff if which == "down" else s.n_embd
    nb = cols // 256
    bb = H.BLOCK_BYTES[qtype]
    buf = getattr(hl, which)
    base = expert * hl.stride(which)
    for r in rows:
        for b in (range(nb) if blocks is None else blocks):
            o = base + (r * nb + b) * bb
            if qtype in (H.TYPE_Q4_K, H.TYPE_Q5_K):
                buf[o:o + 4] = 0          # fp16 d, fp16 dmin
            elif qtype == H.TYPE_Q6_K:
                buf[o + 208:o + 210] = 0  # fp16 d (last)
            else:
                buf[o + 108:o + 110] = 0  # Q3_K d (last)


@pytest.mark.parametrize("shape", [W.QWEN3_30B, W.OLMOE], ids=lambda s: s.name)
def test_zero_blocks_and_zero_scales(orc, shape):
    """fx with an all-zero 256-block (Q8_K d = 0), selected experts with d = dmin = 0
    super-blocks in gate, up and down, and one selected expert whose gate and up rows
    are all zero, so that every block of its h is zero."""
    fx, res = W.make_hidden(shape, 24, 0, 0)
    fx = fx.copy()
    fx[256:512] = 0.0
    hl = W.make_layer(shape, 24, 0)
    sel_o, w_o, _ = orc.route(hl.router, fx, shape.n_expert, shape.n_used, shape.renorm)
    e0, e1, e2 = (int(e) for e in sel_o[:3])
    _zero_d(hl, "gate", e0, range(0, 16), blocks=[0, 3])
    _zero_d(hl, "up", e0, range(8, 40))
    _zero_d(hl, "down", e1, range(0, 64))
    _zero_d(hl, "gate", e2, range(shape.n_ff))
    _zero_d(hl, "up", e2, range(shape.n_ff))
    st = _stage(shape, {0: hl})
    try:
        print(f"special values {shape.name}: zero fx block, zero-scale blocks in {e0} {e1}, zero h of {e2}",
              flush=True)
        ref, sel_r, _ = orc.moe_layer(hl, fx, res)
        assert np.array_equal(sel_r, sel_o)
        out, sel, w_dev = st.layer(0, fx, res)
        assert np.array_equal(sel, sel_o)
        m = parity.assert_parity(out, ref, f"special values {shape.name}")
        print("  ", m, flush=True)
        out2 = st.ffn_combine(0, fx, sel, w_dev, res)  # the device's own weights: the same bits
        assert np.array_equal(out2.view(np.uint32), out.view(np.uint32))
        # the expert with zero gate/up rows contributes nothing: dropping it from the
        # selection (weight 0) changes no bit of the combine of the others
        w0 = w_o.copy()
        w0[2] = 0.0
        a = st.ffn_combine(0, fx, sel_o, w0, res)
        parity.assert_parity(a, orc.moe_ffn_combine(hl, fx, sel_o, w0, res), "zero-h expert")
    finally:
        st.close()


@pytest.mark.parametrize("kernel", ["xcd", "spread", "launches"])
def test_decode_zero_block_and_zero_scales(orc, kernel):
    """The same special values through the decode paths: x with an all-zero block
    (so fx has one), and zero-scale blocks in the experts of every layer's selection."""
    shape = W.QWEN3_30B
    nl = 3
    _, x = W.make_hidden(shape, 25, 0, 0)
    x = x.copy()
    x[512:768] = 0.0
    layers = {}
    xs = [x]
    for l in range(nl):
        hl = W.make_layer(shape, 25, l)
        fx = orc.rms_norm(xs[-1], W.RMS_EPS)
        sel_o, _, _ = orc.route(hl.router, fx, shape.n_expert, shape.n_used, shape.renorm)
        _zero_d(hl, "gate", int(sel_o[0]), range(0, 32), blocks=[1])
        _zero_d(hl, "down", int(sel_o[1]), range(100, 300))
        _zero_d(hl, "up", int(sel_o[3]), range(shape.n_ff))
        layers[l] = hl
        ref, _, _ = orc.moe_layer(hl, fx, xs[-1])
        xs.append(ref)
    st = _stage(shape, layers)
    try:
        if kernel == "launches":
            st.set_option(H.OPT_PERSISTENT_DECODE, 0)
        else:
            st.set_option(H.OPT_DECODE_KERNEL, 1 if kernel == "xcd" else 2)
            st.set_option(H.OPT_PERSISTENT_DECODE, 2)
        print(f"decode special values, {kernel}", flush=True)
        ys = [x]
        for l in range(nl):
            ys.append(st.decode(ys[-1], l, l + 1, W.RMS_EPS))
            st.sync_check()
            ref, _, _ = orc.moe_layer(layers[l], orc.rms_norm(ys[l], W.RMS_EPS), ys[l])
            parity.assert_parity(ys[-1], ref, f"decode special values {kernel} layer {l}")
        whole = st.decode(x, 0, nl, W.RMS_EPS)
        st.sync_check()
        parity.assert_parity(whole, ys[-1], f"decode special values {kernel} whole")
    finally:
        st.close()


def test_nan_in_fx_of_expert_products_matches_oracle(orc):
    """hoard_moe_ffn_combine with the caller's ids: a NaN element of fx quantises to 0."""
    shape = W.QWEN3_30B
    hl = W.make_layer(shape, 26, 0)
    st = _stage(shape, {0: hl})
    try:
        fx, res = W.make_hidden(shape, 26, 0, 0)
        sel_o, w_o, _ = orc.route(hl.router, fx, shape.n_expert, shape.n_used, shape.renorm)
        fx = fx.copy()
        fx[[5, 700, 2047]] = np.nan
        print("NaN in fx, caller's ids", flush=True)
        out = st.ffn_combine(0, fx, sel_o, w_o, res)
        ref = orc.moe_ffn_combine(hl, fx, sel_o, w_o, res)
        assert np.all(np.isfinite(ref))
        parity.assert_parity(out, ref, "NaN in fx")
        # an infinite element: Q8_K gives its block scale 1/(-127/inf) = -inf and every
        # quant 0, so every gate/up row is inf * 0 = NaN; Q8_K of an all-NaN h block is
        # the zero block (NaN never sets the scale), so every expert output is 0 and the
        # combine returns the residual, as ggml's quantize_row_q8_K makes it
        fx[5] = np.inf
        out = st.ffn_combine(0, fx, sel_o, w_o, res)
        ref = orc.moe_ffn_combine(hl, fx, sel_o, w_o, res)
        assert np.array_equal(ref.view(np.uint32), res.view(np.uint32))
        assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
    finally:
        st.close()


@pytest.mark.parametrize("bad", [np.nan, np.inf, -np.inf], ids=["nan", "inf", "-inf"])
def test_non_finite_router_input(orc, bad):
    """The rule for a non-finite router input on every routed path, and that the
    handle keeps working afterwards."""
    shape = W.QWEN3_30B
    nl = 2
    layers = {l: W.make_layer(shape, 27, l) for l in range(nl)}
    st = _stage(shape, layers, max_tokens=4)
    try:
        fx, res = W.make_hidden(shape, 27, 0, 0)
        good, _, _ = st.layer(0, fx, res)
        badfx = fx.copy()
        badfx[300] = bad
        print(f"non-finite router input {bad}: route / layer / batched", flush=True)
        sel, w = st.route(0, badfx)
        assert np.all(sel == INT32_MAX) and np.all(np.isnan(w)), (sel, w)
        out, lsel, lw = st.layer(0, badfx, res)
        assert np.all(np.isnan(out))
        assert np.all(lsel == INT32_MAX) and np.all(np.isnan(lw)), (lsel, lw)
        bfx = np.stack([fx, badfx, fx])
        bres = np.stack([res, res, res])
        bout, bsel, _ = st.forward_batched(0, bfx, bres)
        assert np.all(np.isnan(bout[1])) and np.all(bsel[1] == INT32_MAX)
        assert np.array_equal(bout[0].view(np.uint32), good.view(np.uint32))
        assert np.array_equal(bout[2].view(np.uint32), good.view(np.uint32))
        _, x = W.make_hidden(shape, 27, 0, 1)
        ref_whole = st.decode(x, 0, nl, W.RMS_EPS)
        badx = x.copy()
        badx[1000] = bad
        for mode, kernel in ((0, 0), (2, 1), (2, 2)):
            st.set_option(H.OPT_PERSISTENT_DECODE, mode)
            if mode:
                st.set_option(H.OPT_DECODE_KERNEL, kernel)
            print(f"  decode mode {mode} kernel {kernel}", flush=True)
            y = st.decode(badx, 0, nl, W.RMS_EPS)
            st.sync_check()  # no wait ran out: the NaN travelled through the exchanges
            assert np.all(np.isnan(y))
            y = st.decode(x, 0, nl, W.RMS_EPS)
            st.sync_check()
            parity.assert_parity(y, ref_whole, f"after non-finite input, mode {mode} kernel {kernel}")
        out, _, _ = st.layer(0, fx, res)
        assert np.array_equal(out.view(np.uint32), good.view(np.uint32))
    finally:
        st.close()


# ---- failure paths forced from the host ---------------------------------------

@pytest.mark.parametrize("shape,kernel", [(W.QWEN3_30B, 1), (W.QWEN3_30B, 2), (W.QWEN3_NEXT, 2)],
                         ids=["qwen3_30b-xcd", "qwen3_30b-spread", "qwen3_next-spread"])
def test_wait_limit_zero_gives_up_cleanly(orc, shape, kernel):
    """A wait limit of 0: the first wait that finds its data missing raises the
    error flag, every workgroup leaves, the failed rows are NaN and
    hoard_moe_sync_check reports HOARD_ERR_HIP; with the limit restored the same
    handle decodes the oracle's result again."""
    nl = 3
    layers = {l: W.make_layer(shape, 28, l) for l in range(nl)}
    st = _stage(shape, layers)
    try:
        st.set_option(H.OPT_DECODE_KERNEL, kernel)
        st.set_option(H.OPT_PERSISTENT_DECODE, 2)
        _, x = W.make_hidden(shape, 28, 0, 0)
        good = st.decode(x, 0, nl, W.RMS_EPS)
        st.sync_check()
        assert st.get_option(H.OPT_WAIT_LIMIT_US) == 200000
        st.set_option(H.OPT_WAIT_LIMIT_US, 0)
        print(f"wait limit 0, {shape.name} kernel {kernel}", flush=True)
        y = st.decode(x, 0, nl, W.RMS_EPS)
        with pytest.raises(H.HoardError) as ei:
            st.sync_check()
        assert ei.value.code == H.ERR_HIP
        assert np.isnan(y).any()
        st.sync_check()  # the flag was cleared by the report
        st.set_option(H.OPT_WAIT_LIMIT_US, 200000)
        y = st.decode(x, 0, nl, W.RMS_EPS)
        st.sync_check()
        assert np.array_equal(y.view(np.uint32), good.view(np.uint32))
        ref = x
        for l in range(nl):
            ref, _, _ = orc.moe_layer(layers[l], orc.rms_norm(ref, W.RMS_EPS), ref)
        parity.assert_parity(y, ref, "after the forced failure")
    finally:
        st.close()


def test_failed_slot_upload_leaves_pool_consistent():
    """HOARD_OPT_FAIL_UPLOAD makes a chosen upload fail: the call returns
    HOARD_ERR_HIP, the layer's residency is forgotten (the next call uploads every
    selected expert), and the output is then the resident handle's bit for bit."""
    shape = W.QWEN3_30B
    layers = {0: W.make_layer(shape, 29, 0)}
    res_st = _stage(shape, layers)
    pool = _stage(shape, layers, pool_k=12)
    try:
        fx, res = W.make_hidden(shape, 29, 0, 0)
        s1 = np.arange(8, dtype=np.int32)
        s2 = np.array([0, 1, 20, 21, 22, 23, 24, 25], np.int32)
        pool.pool_ensure(0, s1)
        pool.reset_stats()
        pool.set_option(H.OPT_FAIL_UPLOAD, 3)  # the third upload of s2's six misses fails
        print("failed slot upload", flush=True)
        with pytest.raises(H.HoardError) as ei:
            pool.pool_ensure(0, s2)
        assert ei.value.code == H.ERR_HIP
        assert pool.get_option(H.OPT_FAIL_UPLOAD) == 0
        torch.cuda.synchronize()
        pool.reset_stats()
        slots_h, slots_d = pool.pool_ensure(0, s2)
        st = pool.stats()
        assert st.misses == 8 and st.hits == 0, (st.hits, st.misses)  # residency was forgotten
        w = np.full(8, 0.125, np.float32)
        out = torch.empty(shape.n_embd, device="cuda")
        pool.ffn_combine_dev(0, pool.dev(fx), slots_d, pool.dev(w), pool.dev(res), out)
        torch.cuda.synchronize()
        ref = res_st.ffn_combine(0, fx, s2, w, res)
        assert np.array_equal(out.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    finally:
        pool.close()
        res_st.close()


@pytest.mark.parametrize("shape", [W.QWEN3_NEXT, W.QWEN35], ids=lambda s: s.name)
def test_non_finite_router_input_fused_many_experts(orc, shape):
    """The one-launch layer above 128 experts (two-step rank) and with a shared
    expert: a NaN router input gives no expert (INT32_MAX), weight NaN and a NaN
    row, as the three launches do; the next good token is exact."""
    layers = {0: W.make_layer(shape, 28, 0)}
    st = _stage(shape, layers)
    try:
        assert st.get_option(H.OPT_LAYER_FUSED) == 1
        fx, res = W.make_hidden(shape, 28, 0, 0)
        good, gsel, _ = st.layer(0, fx, res)
        badfx = fx.copy()
        badfx[77] = np.nan
        print(f"non-finite router input, one-launch layer {shape.name}", flush=True)
        out, sel, w = st.layer(0, badfx, res)
        st.sync_check()
        assert np.all(sel == INT32_MAX) and np.all(np.isnan(w)), (sel, w)
        assert np.all(np.isnan(out))
        st.set_option(H.OPT_LAYER_FUSED, 0)
        out0, sel0, w0 = st.layer(0, badfx, res)
        assert np.array_equal(sel0, sel) and np.all(np.isnan(w0)) and np.all(np.isnan(out0))
        st.set_option(H.OPT_LAYER_FUSED, 1)
        again, asel, _ = st.layer(0, fx, res)
        st.sync_check()
        assert np.array_equal(asel, gsel) and np.array_equal(again.view(np.uint32), good.view(np.uint32))
        ref, sel_o, _ = orc.moe_layer(layers[0], fx, res)
        assert np.array_equal(gsel, sel_o)
        parity.assert_parity(good, ref, f"one-launch layer {shape.name}")
    finally:
        st.set_option(H.OPT_LAYER_FUSED, 1)
        st.close()


def test_fused_layer_wait_limit_zero_gives_up_cleanly(orc):
    """The one-launch layer's waits with a limit of 0: its gate/up and down
    workgroups give up at the first missing count, the output is NaN and
    hoard_moe_sync_check reports HOARD_ERR_HIP; restored, the next calls are exact
    (the counters stayed in step through the failed launch)."""
    shape = W.QWEN3_30B
    layers = {l: W.make_layer(shape, 30, l) for l in range(2)}
    st = _stage(shape, layers)
    try:
        assert st.get_option(H.OPT_LAYER_FUSED) == 1
        fx, res = W.make_hidden(shape, 30, 0, 0)
        good, _, _ = st.layer(0, fx, res)
        st.sync_check()
        st.set_option(H.OPT_WAIT_LIMIT_US, 0)
        print("fused layer, wait limit 0", flush=True)
        out, _, _ = st.layer(0, fx, res)
        with pytest.raises(H.HoardError) as ei:
            st.sync_check()
        assert ei.value.code == H.ERR_HIP
        assert np.isnan(out).any()
        st.set_option(H.OPT_WAIT_LIMIT_US, 200000)
        for _ in range(2):
            out, _, _ = st.layer(0, fx, res)
            st.sync_check()
            assert np.array_equal(out.view(np.uint32), good.view(np.uint32))
        ref, _, _ = orc.moe_layer(layers[0], fx, res)
        parity.assert_parity(out, ref, "fused layer after the forced failure")
    finally:
        st.close()
