"""Expert-slot LRU bookkeeping (host replay through the C ABI, no device).

Pinned by a hand-traced known answer, by the pool's invariants, and by a
restatement of the engine's fetch step (src/run_moe_stream.cpp:385-419:
hits first, then each miss takes the back of the LRU list).
"""
import ctypes

import numpy as np
import pytest

import hoard_amd as H


def _replay(lib, n_layer, n_expert, k, naive, trace):
    """trace: list of (layer, sel list).  Returns per-call (slots, misses)."""
    p = ctypes.c_void_p()
    H.check(lib.hoard_slot_lru_create(n_layer, n_expert, k, int(naive), ctypes.byref(p)))
    out = []
    try:
        for layer, sel in trace:
            s = np.asarray(sel, dtype=np.int32)
            slots = np.zeros(len(s), dtype=np.int32)
            miss = np.zeros(len(s), dtype=np.uint8)
            rc = lib.hoard_slot_lru_access(p, layer, s.ctypes.data, len(s), slots.ctypes.data, miss.ctypes.data)
            assert rc == 0
            out.append((slots.tolist(), miss.tolist()))
    finally:
        lib.hoard_slot_lru_destroy(p)
    return out


def _engine_restatement(n_layer, n_expert, k, naive, trace):
    """The reference engine's Slots update, restated with plain lists and dicts."""
    slot_expert = [[-1] * k for _ in range(n_layer)]
    expert_slot = [dict() for _ in range(n_layer)]
    lru = [list(range(k)) for _ in range(n_layer)]  # index 0 = front = most recent
    out = []
    for layer, sel in trace:
        n = len(sel)
        slots, hit = [0] * n, [False] * n
        if not naive:
            for j, e in enumerate(sel):
                if e in expert_slot[layer]:
                    s = expert_slot[layer][e]
                    lru[layer].remove(s)
                    lru[layer].insert(0, s)
                    slots[j], hit[j] = s, True
        for j, e in enumerate(sel):
            if hit[j]:
                continue
            if naive:
                slots[j] = j
                continue
            s = lru[layer].pop()
            old = slot_expert[layer][s]
            if old >= 0:
                expert_slot[layer].pop(old, None)
            slot_expert[layer][s] = e
            expert_slot[layer][e] = s
            lru[layer].insert(0, s)
            slots[j] = s
        out.append((slots, [0 if h else 1 for h in hit]))
    return out


def test_known_answer(hlib):
    # K=3, two experts per token; slots start as LRU list [0, 1, 2] (front first)
    trace = [(0, [0, 1]), (0, [1, 2]), (0, [3, 0])]
    got = _replay(hlib, 1, 8, 3, False, trace)
    # t0: both miss -> back slots 2 then 1; t1: 1 hits slot 1, 2 takes slot 0;
    # t2: 0 hits (slot 2 moves to front) before 3's miss evicts expert 1 from slot 1
    assert got == [([2, 1], [1, 1]), ([1, 0], [0, 1]), ([1, 2], [1, 0])]


def test_naive_mode_places_request_j_in_slot_j(hlib):
    trace = [(0, [5, 6, 7]), (0, [5, 6, 7]), (1, [1, 2, 3])]
    got = _replay(hlib, 2, 16, 4, True, trace)
    assert all(s == [0, 1, 2] and m == [1, 1, 1] for s, m in got)


def _zipf_trace(rng, n_layer, n_expert, n_used, tokens):
    p = 1.0 / np.arange(1, n_expert + 1) ** 0.8
    p /= p.sum()
    trace = []
    for _ in range(tokens):
        for layer in range(n_layer):
            trace.append((layer, rng.choice(n_expert, n_used, replace=False, p=p).tolist()))
    return trace


@pytest.mark.parametrize("k,naive", [(8, False), (12, False), (32, False), (8, True)])
def test_matches_engine_restatement(hlib, k, naive):
    rng = np.random.default_rng(k)
    trace = _zipf_trace(rng, 3, 128, 8, 200)
    assert _replay(hlib, 3, 128, k, naive, trace) == _engine_restatement(3, 128, k, naive, trace)


def test_invariants(hlib):
    rng = np.random.default_rng(7)
    n_layer, n_expert, k, n_used = 2, 64, 10, 8
    trace = _zipf_trace(rng, n_layer, n_expert, n_used, 300)
    got = _replay(hlib, n_layer, n_expert, k, False, trace)
    resident = [dict() for _ in range(n_layer)]  # slot -> expert, from the replay's own answers
    for (layer, sel), (slots, miss) in zip(trace, got):
        assert len(set(slots)) == len(slots), "one slot per request"
        assert all(0 <= s < k for s in slots)
        for e, s, m in zip(sel, slots, miss):
            if not m:  # a hit must name the slot that holds the expert
                assert resident[layer].get(s) == e
            assert m == (e not in resident[layer].values())
        for e, s in zip(sel, slots):
            resident[layer][s] = e
        # with K >= n_used every expert of the token is resident after the call
        assert set(sel) <= set(resident[layer].values())


def test_bad_arguments(hlib):
    p = ctypes.c_void_p()
    assert hlib.hoard_slot_lru_create(1, 8, 9, 0, ctypes.byref(p)) != 0  # K > n_expert
    H.check(hlib.hoard_slot_lru_create(1, 8, 4, 0, ctypes.byref(p)))
    try:
        sel = np.array([0, 8], dtype=np.int32)
        slots = np.zeros(2, dtype=np.int32)
        assert hlib.hoard_slot_lru_access(p, 0, sel.ctypes.data, 2, slots.ctypes.data, None) != 0
        assert hlib.hoard_slot_lru_access(p, 1, sel.ctypes.data, 1, slots.ctypes.data, None) != 0
    finally:
        hlib.hoard_slot_lru_destroy(p)


def _verify_loop_restatement(n_layer, n_expert, k, trace):
    """The verify loop's ensure (src/run_specloop.cpp:59-67), id after id: a hit
    moves its slot to the front; a miss pops the back slot, drops its expert,
    takes the id and goes to the front."""
    slot_expert = [[-1] * k for _ in range(n_layer)]
    expert_slot = [dict() for _ in range(n_layer)]
    lru = [list(range(k)) for _ in range(n_layer)]
    out = []
    for layer, sel in trace:
        slots, miss = [], []
        for e in sel:
            if e in expert_slot[layer]:
                s = expert_slot[layer][e]
                lru[layer].remove(s)
                miss.append(0)
            else:
                s = lru[layer].pop()
                old = slot_expert[layer][s]
                if old >= 0:
                    del expert_slot[layer][old]
                slot_expert[layer][s] = e
                expert_slot[layer][e] = s
                miss.append(1)
            lru[layer].insert(0, s)
            slots.append(s)
        out.append((slots, miss))
    return out


def test_sequential_order_matches_verify_loop(hlib):
    """Batches of several tokens' ids (repeats included) against the restatement;
    with a batch whose distinct ids exceed K the two orders part ways, which the
    engine order would hide."""
    rng = np.random.default_rng(21)
    n_layer, n_expert, k = 3, 40, 12
    trace = []
    for _ in range(300):
        m = int(rng.integers(1, 5))
        sel = []
        for _ in range(m):  # m tokens of 4 distinct experts each, Zipf-ish
            sel += list(rng.choice(n_expert, 4, replace=False, p=np.arange(n_expert, 0, -1) / np.arange(n_expert, 0, -1).sum()))
        trace.append((int(rng.integers(0, n_layer)), [int(e) for e in sel]))
    got = _replay(hlib, n_layer, n_expert, k, 2, trace)
    want = _verify_loop_restatement(n_layer, n_expert, k, trace)
    assert got == want
    # a repeated id in one call is a hit on the slot it just took
    g = _replay(hlib, 1, 8, 4, 2, [(0, [5, 5, 1, 5])])
    assert g == [([3, 3, 2, 3], [1, 0, 1, 0])]
