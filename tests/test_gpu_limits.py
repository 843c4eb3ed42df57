"""Shapes at the edges of what the stage takes (hoard_moe_create: n_expert
1..1024, n_used 1..16, n_embd / n_ff any multiple of 256): the most experts with
the largest top-k, a single expert, and hidden sizes other than 2048 (which the
shape-generic kernels serve), each against the oracle to the parity bar with
identical top-k.  Only the selected experts' weights are generated."""
import numpy as np
import pytest

import hoard_amd as H
import parity
from hoard_amd import workloads as W

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

CASES = [
    W.Shape("e1024_k16", 5, 2048, 1024, 16, 256, 1, H.TYPE_Q4_K, H.TYPE_Q4_K, H.TYPE_Q6_K, 1),
    W.Shape("e1_k1", 6, 2048, 1, 1, 256, 1, H.TYPE_Q4_K, H.TYPE_Q4_K, H.TYPE_Q6_K, 1),
    W.Shape("d1024_e8_k2_norenorm", 7, 1024, 8, 2, 512, 0, H.TYPE_Q4_K, H.TYPE_Q4_K, H.TYPE_Q4_K, 1),
    W.Shape("d4096_e32_k4_shared", 8, 4096, 32, 4, 256, 1, H.TYPE_Q4_K, H.TYPE_Q4_K, H.TYPE_Q6_K, 1,
            n_ff_shexp=512),
    # an odd expert count (router workgroups partly filled), and 60 experts top-4 with a
    # shared expert, the routing of Qwen1.5-MoE
    W.Shape("e61_k7", 9, 2048, 61, 7, 768, 1, H.TYPE_Q4_K, H.TYPE_Q4_K, H.TYPE_Q6_K, 1),
    W.Shape("e60_k4_shared", 10, 2048, 60, 4, 1536, 1, H.TYPE_Q4_K, H.TYPE_Q4_K, H.TYPE_Q6_K, 1,
            n_ff_shexp=1024),
    # more than 128 experts without a shared expert: the one-launch layer's gate/up
    # and down workgroups run the one-wave router tail instead of the rank
    W.Shape("e256_k8", 11, 2048, 256, 8, 512, 1, H.TYPE_Q4_K, H.TYPE_Q4_K, H.TYPE_Q6_K, 1),
]


@pytest.mark.parametrize("shape", CASES, ids=lambda s: s.name)
def test_edge_shapes_match_oracle(orc, shape):
    from hoard_amd.runtime import MoEStage
    router = W.make_router(shape, 0, 0)
    toks = [W.make_hidden(shape, 0, 0, t) for t in range(4)]
    sels = [orc.route(router, fx, shape.n_expert, shape.n_used, shape.renorm)[0] for fx, _ in toks]
    hl = W.make_layer(shape, 0, 0, experts=sorted(set(np.concatenate(sels).tolist())))
    st = MoEStage(shape, n_layer=1, layers={0: hl})
    try:
        for t, (fx, res) in enumerate(toks):
            print(f"edge {shape.name} token {t}", flush=True)
            sel_d, w_d = st.route(0, fx)
            assert np.array_equal(sel_d, sels[t]), (sel_d, sels[t])
            out, sel, w = st.layer(0, fx, res)
            ref, sel_o, w_o = orc.moe_layer(hl, fx, res)
            assert np.array_equal(sel, sel_o)
            assert np.allclose(w, w_o, rtol=1e-6, atol=0)
            m = parity.assert_parity(out, ref, f"{shape.name} token {t}")
            print("  ", m, flush=True)
        if shape.n_embd == 2048:  # the stacked decode over the one layer
            _, x = toks[0]
            y = st.decode(x, 0, 1, W.RMS_EPS)
            st.sync_check()
            ref, _, _ = orc.moe_layer(hl, orc.rms_norm(x, W.RMS_EPS), x)
            parity.assert_parity(y, ref, f"{shape.name} decode")
    finally:
        st.close()


def test_create_rejects_out_of_range_shapes():
    import ctypes
    lib = H.load_library()
    base = dict(n_embd=2048, n_expert=64, n_used=8, n_ff=1024, n_ff_shexp=0, n_layer=1, renorm=1, pool_k=0,
                max_tokens=1)
    for field, bad in (("n_expert", 1025), ("n_used", 17), ("n_used", 0), ("n_embd", 2000), ("n_ff", 100),
                       ("n_ff_shexp", 300), ("pool_k", 4), ("pool_k", 65), ("max_tokens", 0)):
        cfg = H.MoeCfg(**{**base, field: bad})
        h = ctypes.c_void_p()
        rc = lib.hoard_moe_create(ctypes.byref(cfg), ctypes.byref(h))
        assert rc == H.ERR_INVALID, (field, bad, rc)
