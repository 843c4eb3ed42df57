"""Slot pool served by the storage tier (include/hoard_store.h): experts
streamed from a GGUF file through the RAM tier into HBM slots give the
all-resident stage's outputs bit for bit, in LRU and naive pool modes, with the
reference's three-tier accounting (src/run_qwen35.cpp:596-638): every slot miss
is one RAM-tier request, and each request is a RAM hit or a file read."""
import numpy as np
import pytest

import hoard_amd as H
from gguf_writer import write_layers
from hoard_amd import workloads as W

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", params=[W.QWEN3_30B, W.QWEN35], ids=lambda s: s.name)
def model(tmp_path_factory, request):
    """Two layers in a GGUF; Qwen3.5's add a shared expert and Q5_K down rows."""
    shape, nl = request.param, 2
    layers = {l: W.make_layer(shape, 6, l) for l in range(nl)}
    path = tmp_path_factory.mktemp("store") / f"{shape.name}_2l.gguf"
    write_layers(path, shape, layers, "qwen3moe")
    return shape, nl, path


# 24 requests per token (two decode layers and one more layer-1 call); a RAM hit
# needs an expert gone from the slots but still in the RAM tier, so the tier holds
# more than two tokens' requests
@pytest.mark.parametrize("naive,k,ram", [(0, 12, 64), (1, 8, 56)], ids=["lru", "naive"])
def test_streamed_pool_matches_resident(model, naive, k, ram):
    from hoard_amd.runtime import MoEStage
    from hoard_amd.store import ExpertStore
    shape, nl, path = model
    ref = MoEStage.from_gguf(path)
    store = ExpertStore.from_gguf(path, readers=8, ram_experts=ram, direct=True, pinned=True)
    st = MoEStage.from_gguf(path, pool_k=k, store=store)
    try:
        st.set_option(H.OPT_POOL_NAIVE, naive)
        eps = st.rms_eps
        for tok, src in enumerate([0, 1, 0, 2, 3, 0, 1, 4]):  # repeats give slot and RAM hits
            _, x = W.make_hidden(shape, 6, 0, src)
            print(f"streamed pool naive={naive} token {tok}", flush=True)
            want = ref.decode(x, 0, nl, eps)
            got = st.decode(x, 0, nl, eps)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), tok
            fx, res = W.make_hidden(shape, 6, 1, src)
            o1, s1, _ = st.layer(1, fx, res)
            o0, s0, _ = ref.layer(1, fx, res)
            assert np.array_equal(s1, s0) and np.array_equal(o1.view(np.uint32), o0.view(np.uint32))
        ps, ss = st.stats(), store.stats()
        print(f"  pool reqs {ps.reqs} hits {ps.hits} misses {ps.misses}; store requests {ss.requests} "
              f"ram hits {ss.ram_hits} file reads {ss.file_reads} direct {ss.direct}", flush=True)
        assert ss.requests == ps.misses and ss.ram_hits + ss.file_reads == ss.requests
        assert ss.file_reads > 0 and ss.ram_hits > 0
        assert ss.bytes_read == ss.file_reads * shape.expert_bytes()
    finally:
        st.close()
        ref.close()
        store.close()


def test_attach_rules(model):
    import ctypes

    from hoard_amd.runtime import MoEStage
    from hoard_amd.store import ExpertStore
    shape, nl, path = model
    store = ExpertStore.from_gguf(path, ram_experts=4, pinned=True)
    resident = MoEStage(shape, n_layer=nl)
    pooled = MoEStage(shape, n_layer=nl, pool_k=8)
    try:
        with pytest.raises(H.HoardError) as ei:  # no slot pool
            H.check(resident.lib.hoard_moe_attach_store(resident.h, store.h))
        assert ei.value.code == H.ERR_STATE
        with pytest.raises(H.HoardError) as ei:  # RAM tier smaller than n_used
            H.check(pooled.lib.hoard_moe_attach_store(pooled.h, store.h))
        assert ei.value.code == H.ERR_INVALID
        big = ExpertStore.from_gguf(path, ram_experts=64, pinned=True)
        wrong = MoEStage(shape, n_layer=nl + 1, pool_k=8)
        with pytest.raises(H.HoardError) as ei:  # layer count differs
            H.check(wrong.lib.hoard_moe_attach_store(wrong.h, big.h))
        assert ei.value.code == H.ERR_INVALID
        wrong.close()
        pooled.set_layer(0, W.make_layer(shape, 6, 0, experts=[]))
        with pytest.raises(H.HoardError) as ei:  # after weights were set
            H.check(pooled.lib.hoard_moe_attach_store(pooled.h, big.h))
        assert ei.value.code == H.ERR_STATE
        fresh = MoEStage(shape, n_layer=nl, pool_k=8)
        H.check(fresh.lib.hoard_moe_attach_store(fresh.h, big.h))
        hl = W.make_layer(shape, 6, 0, experts=[])  # held: w points into its arrays
        w = hl.weights()
        w.gate_type = H.TYPE_Q6_K  # not the file's type: the store's strides disagree
        with pytest.raises(H.HoardError) as ei:
            H.check(fresh.lib.hoard_moe_set_layer_weights(fresh.h, 0, ctypes.byref(w)))
        assert ei.value.code == H.ERR_INVALID
        fresh.close()
        big.close()
    finally:
        resident.close()
        pooled.close()
        store.close()
