"""hoard_moe_forward_batched_noalloc: the batched forward with its scratch in the
library's fixed device array, so that the call allocates nothing.  Its results
must be hoard_moe_forward_batched's bit for bit (and so at the parity bar against
the oracle) on two calls in a row, the second with fewer tokens on another
layer; sizes past the array's limit are refused with HOARD_ERR_INVALID."""
import ctypes

import numpy as np
import pytest

import hoard_amd as H
import parity
from hoard_amd import workloads as W

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _tokens(shape, M, base):
    fx, res = zip(*(W.make_hidden(shape, 13, 0, base + t) for t in range(M)))
    return np.stack(fx), np.stack(res)


def _noalloc(st, layer, fx, res):
    fx_d, res_d = st.dev(fx), st.dev(res)
    M = fx_d.shape[0]
    out = torch.empty_like(res_d)
    sel = torch.empty((M, st.shape.n_used), dtype=torch.int32, device="cuda")
    w = torch.empty((M, st.shape.n_used), dtype=torch.float32, device="cuda")
    rc = st.lib.hoard_moe_forward_batched_noalloc(st.h, layer, M, st.ptr(fx_d), st.ptr(res_d), st.ptr(out),
                                                  st.ptr(sel), st.ptr(w), st.stream())
    return rc, (fx_d, res_d, out, sel, w)


@pytest.mark.parametrize("shape", [W.QWEN3_30B, W.QWEN3_NEXT], ids=lambda s: s.name)
def test_noalloc_matches_forward_batched(orc, shape):
    """Qwen3-Next adds the shared expert's group and output slot to the layout."""
    from hoard_amd.runtime import MoEStage
    layers = {l: W.make_layer(shape, 13, l) for l in range(2)}
    st = MoEStage(shape, n_layer=2, layers=layers, max_tokens=16)
    try:
        calls = [(0, _tokens(shape, 16, 0)), (1, _tokens(shape, 5, 100))]
        refs = [st.forward_batched(l, fx, res) for l, (fx, res) in calls]
        print(f"no-alloc {shape.name}: two calls in a row, M = 16 then M = 5", flush=True)
        got = []
        for l, (fx, res) in calls:
            rc, bufs = _noalloc(st, l, fx, res)
            H.check(rc)
            got.append(bufs)
        torch.cuda.synchronize()
        for (l, (fx, res)), (ro, rs, rw), (_, _, out, sel, w) in zip(calls, refs, got):
            out, sel, w = out.cpu().numpy(), sel.cpu().numpy(), w.cpu().numpy()
            assert np.array_equal(sel, rs), l
            assert np.array_equal(w.view(np.uint32), rw.view(np.uint32)), l
            assert np.array_equal(out.view(np.uint32), ro.view(np.uint32)), l
            ref, sel_o, _ = orc.moe_layer_batched(layers[l], fx, res)
            assert np.array_equal(sel, sel_o)
            for t in range(fx.shape[0]):
                parity.assert_parity(out[t], ref[t], f"no-alloc layer {l} token {t}")
        stats = st.stats()  # the histogram of the last call (5 tokens on layer 1)
        counts = np.bincount(refs[1][1].ravel(), minlength=shape.n_expert)
        assert np.array_equal(np.array(stats.expert_hist[:shape.n_expert]), counts)
    finally:
        st.close()


def test_noalloc_refuses_sizes_past_its_limit():
    from hoard_amd.runtime import MoEStage
    shape = W.QWEN3_30B
    st = MoEStage(shape, n_layer=1, layers={0: W.make_layer(shape, 13, 0, experts=[])}, max_tokens=32)
    try:
        rc, _ = _noalloc(st, 0, *_tokens(shape, 17, 0))  # more tokens than the fixed scratch is laid out for
        assert rc == H.ERR_INVALID, rc
        rc, bufs = _noalloc(st, 0, *_tokens(shape, 3, 0))  # and the handle still works
        H.check(rc)
        torch.cuda.synchronize()
        assert torch.isfinite(bufs[2]).all().item()
    finally:
        st.close()
    big = W.Shape("e256k16", 6, 2048, 256, 16, 1024, 1, H.TYPE_Q4_K, H.TYPE_Q4_K, H.TYPE_Q6_K, 1)
    st = MoEStage(big, n_layer=1, layers={0: W.make_layer(big, 13, 0, experts=[])}, max_tokens=16)
    try:
        rc, _ = _noalloc(st, 0, *_tokens(big, 16, 0))  # 16 tokens of this shape need more than the array
        assert rc == H.ERR_INVALID, rc
        assert b"fixed array" in st.lib.hoard_last_error()
    finally:
        st.close()


def test_noalloc_stats_belong_to_the_handle():
    """Two handles on one GPU share the fixed array: each handle's statistics
    still report its own last call after the other handle's call."""
    from hoard_amd.runtime import MoEStage
    shape = W.QWEN3_30B
    mk = lambda: MoEStage(shape, n_layer=1, layers={0: W.make_layer(shape, 13, 0, experts=[])},  # noqa: E731
                          max_tokens=16)
    sa, sb = mk(), mk()
    try:
        rc, ba = _noalloc(sa, 0, *_tokens(shape, 16, 0))
        H.check(rc)
        rc, bb = _noalloc(sb, 0, *_tokens(shape, 5, 100))
        H.check(rc)
        torch.cuda.synchronize()
        for st, bufs, M in ((sa, ba, 16), (sb, bb, 5)):
            sel = bufs[3].cpu().numpy()
            counts = np.bincount(sel.ravel(), minlength=shape.n_expert)
            stats = st.stats()
            assert np.array_equal(np.array(stats.expert_hist[:shape.n_expert]), counts), M
            assert stats.last_unique == len(np.unique(sel)), M
    finally:
        sa.close()
        sb.close()
