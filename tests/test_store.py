"""Storage tier (include/hoard_store.h) on the host: the bytes a fetch hands
out are the file's, from O_DIRECT and from buffered reads, and the RAM tier's
hits and reads follow the reference's RamTier policy (src/run_qwen35.cpp:
603-607: one LRU over all layers keyed layer * n_expert + e; a hit moves to
the front, a miss evicts the back).  pinned=0 keeps the RAM tier in pageable
memory, so no device is touched."""
import ctypes
import os

import numpy as np
import pytest

import hoard_amd as H
from hoard_amd.store import ExpertStore

N_LAYER, N_EXPERT = 3, 10
STRIDES = [(1000, 1000, 2100), (1234, 1234, 777), (4096, 4096, 5000)]


@pytest.fixture(scope="module")
def model_file(tmp_path_factory):
    """Random bytes with each layer's three expert tensors at unaligned offsets."""
    rng = np.random.default_rng(0)
    layers, off = [], 100
    for l in range(N_LAYER):
        offs = []
        for i in range(3):
            off += int(rng.integers(1, 5000))
            offs.append(off)
            off += STRIDES[l][i] * N_EXPERT
        layers.append((tuple(offs), STRIDES[l]))
    data = rng.integers(0, 256, off + 777, dtype=np.uint8).tobytes()
    p = tmp_path_factory.mktemp("store") / "experts.bin"
    p.write_bytes(data)
    return p, layers, data


def expert_bytes(data, layers, l, e):
    return [data[layers[l][0][i] + e * layers[l][1][i]:][:layers[l][1][i]] for i in range(3)]


def replay_ram_tier(requests, cap):
    """The reference's RamTier, request by request: True for a hit."""
    lru, out = [], []  # front = most recent
    for key in requests:
        if key in lru:
            lru.remove(key)
            out.append(True)
        else:
            if len(lru) == cap:
                lru.pop()
            out.append(False)
        lru.insert(0, key)
    return out


@pytest.mark.parametrize("direct,readers", [(1, 8), (0, 8), (1, 1)], ids=["direct8", "buffered8", "direct1"])
def test_fetch_returns_the_file_bytes(model_file, direct, readers):
    path, layers, data = model_file
    with ExpertStore(path, layers, N_EXPERT, readers=readers, ram_experts=7, direct=bool(direct), pinned=False) as st:
        rng = np.random.default_rng(1)
        for _ in range(60):
            l = int(rng.integers(0, N_LAYER))
            ids = rng.choice(N_EXPERT, size=int(rng.integers(1, 6)), replace=False)
            parts, _ = st.fetch(l, ids)
            for e, p in zip(ids, parts):
                want = expert_bytes(data, layers, l, int(e))
                for i in range(3):
                    assert ctypes.string_at(p[i], len(want[i])) == want[i], (l, e, i)
        s = st.stats()
        assert s.ram_hits + s.file_reads == s.requests
        assert s.ram_experts == 7
        if not direct:
            assert s.direct == 0


@pytest.mark.parametrize("cap", [4, 9, 30])
def test_hits_follow_the_reference_ram_tier(model_file, cap):
    path, layers, _ = model_file
    rng = np.random.default_rng(cap)
    batches = []
    for _ in range(200):
        l = int(rng.integers(0, N_LAYER))
        # skewed choice so that hits happen at every capacity
        ids = np.unique(np.minimum(rng.zipf(1.6, size=int(rng.integers(1, 5))) - 1, N_EXPERT - 1))[:cap]
        batches.append((l, ids))
    want = replay_ram_tier([l * N_EXPERT + int(e) for l, ids in batches for e in ids], cap)
    with ExpertStore(path, layers, N_EXPERT, readers=4, ram_experts=cap, direct=True, pinned=False) as st:
        got = []
        for l, ids in batches:
            _, hit = st.fetch(l, ids)
            got += list(hit)
        s = st.stats()
    assert got == want
    assert s.ram_hits == sum(want) and s.file_reads == len(want) - sum(want)
    assert s.bytes_read == sum(sum(layers[l][1]) for (l, ids) in batches for e in ids) - \
        sum(sum(layers[l][1]) for (l, e), h in zip([(l, e) for l, ids in batches for e in ids], want) if h)


def test_every_expert_fits_by_default(model_file):
    path, layers, _ = model_file
    with ExpertStore(path, layers, N_EXPERT, ram_experts=0, pinned=False) as st:
        for rep in range(2):
            for l in range(N_LAYER):
                st.fetch(l, np.arange(N_EXPERT))
        s = st.stats()
        assert s.ram_experts == N_LAYER * N_EXPERT
        assert s.file_reads == N_LAYER * N_EXPERT and s.ram_hits == N_LAYER * N_EXPERT


def test_argument_errors(model_file):
    path, layers, _ = model_file
    with ExpertStore(path, layers, N_EXPERT, ram_experts=3, pinned=False) as st:
        for l, ids in ((N_LAYER, [0]), (-1, [0]), (0, [N_EXPERT]), (0, [-1]), (0, [0, 1, 2, 3])):
            with pytest.raises(H.HoardError) as ei:
                st.fetch(l, ids)
            assert ei.value.code == H.ERR_INVALID
    bad = [(layers[0][0], (layers[0][1][0] * 1000, 1, 1))] + layers[1:]
    with pytest.raises(H.HoardError) as ei:
        ExpertStore(path, bad, N_EXPERT, pinned=False)
    assert ei.value.code == H.ERR_INVALID
    with pytest.raises(H.HoardError) as ei:
        ExpertStore(path.parent / "absent.bin", layers, N_EXPERT, pinned=False)
    assert ei.value.code == H.ERR_IO


def test_read_failure_drops_the_entries(model_file, tmp_path):
    """A file cut short after opening: the read fails with ERR_IO, the entries it
    was filling are dropped, and once the file is whole again they are read."""
    path, layers, data = model_file
    p = tmp_path / "cut.bin"
    p.write_bytes(data)
    with ExpertStore(p, layers, N_EXPERT, ram_experts=5, pinned=False) as st:
        os.truncate(p, layers[2][0][0])  # layer 2's tensors are gone
        with pytest.raises(H.HoardError) as ei:
            st.fetch(2, [1, 2])
        assert ei.value.code == H.ERR_IO
        p.write_bytes(data)
        parts, hit = st.fetch(2, [1, 2])
        assert not hit.any()
        for e, pp in zip((1, 2), parts):
            for i, w in enumerate(expert_bytes(data, layers, 2, e)):
                assert ctypes.string_at(pp[i], len(w)) == w


def test_gguf_extents_point_at_the_expert_tensors(tmp_path):
    from gguf_writer import write_layers
    from hoard_amd import workloads as W
    from hoard_amd.gguf import GGUFWeights
    shape = W.Shape("tiny", 0, 512, 4, 2, 256, 1, H.TYPE_Q4_K, H.TYPE_Q4_K, H.TYPE_Q6_K, 2)
    layers = {l: W.make_layer(shape, 7, l) for l in range(2)}
    p = tmp_path / "m.gguf"
    write_layers(p, shape, layers, "qwen3moe")
    with ExpertStore.from_gguf(p, ram_experts=3, pinned=False) as st, GGUFWeights(p) as g:
        assert (st.n_layer, st.n_expert) == (2, 4)
        for l, hl in layers.items():
            w = g.layer_weights(l)
            assert st.layers[l][1] == (hl.stride("gate"), hl.stride("up"), hl.stride("down"))
            parts, _ = st.fetch(l, [3, 0])
            for e, pp in zip((3, 0), parts):
                for i, name in enumerate(("gate", "up", "down")):
                    sb = hl.stride(name)
                    assert ctypes.string_at(pp[i], sb) == getattr(hl, name)[e * sb:(e + 1) * sb].tobytes()
            assert w.gate  # the reader's own view of the same file
