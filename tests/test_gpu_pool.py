"""Device slot pool (pool_k > 0) through the C ABI.

The reference's own invariant (bench/results/qwen/parity.csv:3) is that the
output does not depend on the cache: naive recopy and the LRU pool give
bit-identical tokens.  Here the pool is checked against the all-resident
handle on the same inputs, and its hit/miss/byte counters against the host
replay of the same LRU bookkeeping.
"""
import ctypes

import numpy as np
import pytest

import hoard_amd as H
from hoard_amd import workloads as W

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

SHAPE = W.QWEN3_30B
NL = 2


@pytest.fixture(scope="module")
def handles():
    from hoard_amd.runtime import MoEStage
    layers = {l: W.make_layer(SHAPE, 2, l) for l in range(NL)}
    res = MoEStage(SHAPE, n_layer=NL, layers=layers)
    pool = MoEStage(SHAPE, n_layer=NL, layers=layers, pool_k=12)
    yield layers, res, pool
    pool.close()
    res.close()


def _host_replay(trace, k, naive=False):
    lib = H.load_library()
    p = ctypes.c_void_p()
    H.check(lib.hoard_slot_lru_create(NL, SHAPE.n_expert, k, int(naive), ctypes.byref(p)))
    misses = 0
    try:
        for t in range(trace.sel.shape[0]):
            for l in range(NL):
                sel = np.ascontiguousarray(trace.sel[t, l])
                slots = np.zeros(SHAPE.n_used, np.int32)
                miss = np.zeros(SHAPE.n_used, np.uint8)
                H.check(lib.hoard_slot_lru_access(p, l, sel.ctypes.data, SHAPE.n_used, slots.ctypes.data,
                                                  miss.ctypes.data))
                misses += int(miss.sum())
    finally:
        lib.hoard_slot_lru_destroy(p)
    return misses


@pytest.mark.parametrize("naive", [False, True], ids=["lru", "naive"])
def test_pool_ffn_is_bit_identical_to_resident(handles, naive):
    layers, res_st, pool_st = handles
    pool_st.set_option(H.OPT_POOL_NAIVE, int(naive))
    pool_st.reset_stats()
    trace = W.routing_trace(SHAPE, seed=3, tokens=20, n_layer=NL)
    copy_stream = torch.cuda.Stream()
    try:
        for t in range(trace.sel.shape[0]):
            for l in range(NL):
                sel, w = trace.sel[t, l], trace.w[t, l]
                fx, res = W.make_hidden(SHAPE, 2, l, t)
                print(f"pool naive={naive} token {t} layer {l} sel {sel.tolist()}", flush=True)
                slots, slots_d = pool_st.pool_ensure(l, sel, copy_stream=copy_stream)
                fx_d, w_d, res_d = pool_st.dev(fx), pool_st.dev(w), pool_st.dev(res)
                out_d = torch.empty_like(res_d)
                pool_st.ffn_combine_dev(l, fx_d, slots_d, w_d, res_d, out_d)
                torch.cuda.synchronize()
                got = out_d.cpu().numpy()
                ref = res_st.ffn_combine(l, fx, sel, w, res)
                assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (t, l)
                if naive:
                    assert slots.tolist() == list(range(SHAPE.n_used))
        st = pool_st.stats()
        reqs = trace.sel.size
        misses = reqs if naive else _host_replay(trace, 12)
        assert st.reqs == reqs and st.misses == misses and st.hits == reqs - misses
        assert st.bytes_h2d == misses * SHAPE.expert_bytes()
        print(f"   reqs {st.reqs} hits {st.hits} misses {st.misses} bytes {st.bytes_h2d}", flush=True)
    finally:
        pool_st.set_option(H.OPT_POOL_NAIVE, 0)


def test_pool_on_demand_layer_and_decode_match_resident(handles):
    layers, res_st, pool_st = handles
    for t in range(4):
        for l in range(NL):
            fx, res = W.make_hidden(SHAPE, 2, l, 100 + t)
            print(f"pool on-demand layer token {t} layer {l}", flush=True)
            out_p, sel_p, w_p = pool_st.layer(l, fx, res)
            out_r, sel_r, w_r = res_st.layer(l, fx, res)
            assert np.array_equal(sel_p, sel_r)
            assert np.array_equal(w_p.view(np.uint32), w_r.view(np.uint32))
            assert np.array_equal(out_p.view(np.uint32), out_r.view(np.uint32))
    res_st.set_option(H.OPT_PERSISTENT_DECODE, 0)  # the same per-layer kernels on both handles
    try:
        for t in range(3):
            _, x = W.make_hidden(SHAPE, 2, 0, 200 + t)
            print(f"pool on-demand decode token {t}", flush=True)
            a = pool_st.decode(x, 0, NL, W.RMS_EPS)
            b = res_st.decode(x, 0, NL, W.RMS_EPS)
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    finally:
        res_st.set_option(H.OPT_PERSISTENT_DECODE, 1)


def test_pool_rejects_bad_ids(handles):
    _, _, pool_st = handles
    bad = np.full(SHAPE.n_used, SHAPE.n_expert, dtype=np.int32)
    with pytest.raises(H.HoardError):
        pool_st.pool_ensure(0, bad)
