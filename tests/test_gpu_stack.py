"""The measured workloads at their full size, against the oracle and the host replay.

* The headline stack: 48 Qwen3-30B-shaped layers decoded in one launch must be
  bit-identical to the same kernel run one layer per launch, and every layer of
  that chain must match the oracle applied to the device's own input of the
  layer (top-k indices identical, output within the bar).  The per-layer launch
  path (hoard_moe_layer's kernels) over the same 48 layers is held to the bar.
  The same for 48 Qwen3-Next-shaped layers through the rows-spread kernel.
* The slot-pool workload as measured: K = 32 slots per layer over all 48 layers,
  routing from the seeded 512-token trace (Zipf(0.8) popularity per layer, 40 %
  reuse of the last 4 tokens' experts).  Every token's chained hidden through the
  48 layers must be the all-resident handle's bit for bit (the reference's own
  losslessness invariant, bench/results/qwen/parity.csv:3), and the slots,
  hits, misses and uploaded bytes must equal the host replay of the same LRU
  (src/run_moe_stream.cpp:379-420).
"""
import ctypes

import numpy as np
import pytest

import hoard_amd as H
import parity
from hoard_amd import workloads as W

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

SHAPE = W.QWEN3_30B
NL = 48


def _fill(st_list, seed, shape=SHAPE):
    hl = W.make_layer(shape, seed, 0)
    for l in range(NL):
        if l:
            W.fill_layer(hl, seed, l)
        for st in st_list:
            st.set_layer(l, hl)
    del hl


def _stack_against_oracle(orc, shape, seed, kernel):
    """48 layers of `shape` decoded in one launch of the one-launch kernel
    `kernel` (1 expert per XCD, 2 rows spread), for 2 tokens: bit-identical to
    the same kernel run one layer per launch, every layer of that chain against
    the oracle applied to the device's own input of the layer (top-k identical,
    output within the bar), and the per-layer launches within the bar."""
    from hoard_amd.runtime import MoEStage
    st = MoEStage(shape, n_layer=NL)
    try:
        print(f"stack {shape.name}: uploading 48 layers", flush=True)
        _fill([st], seed, shape)
        st.set_option(H.OPT_PERSISTENT_DECODE, 2)
        st.set_option(H.OPT_DECODE_KERNEL, kernel)
        for tok in range(2):
            _, x = W.make_hidden(shape, seed, 0, tok)
            print(f"stack {shape.name} token {tok}: one launch over 48 layers", flush=True)
            whole = st.decode(x, 0, NL, W.RMS_EPS)
            st.sync_check()
            xs = [x]
            for l in range(NL):
                xs.append(st.decode(xs[-1], l, l + 1, W.RMS_EPS))
            st.sync_check()
            assert np.array_equal(whole.view(np.uint32), xs[-1].view(np.uint32)), "one launch vs layer by layer"
            worst = {"max_rel": 0.0, "cos": 1.0, "bit_identical": 1.0}
            for l in range(NL):
                fx = orc.rms_norm(xs[l], W.RMS_EPS)
                router = W.make_router(shape, seed, l)
                sel_o, _, _ = orc.route(router, fx, shape.n_expert, shape.n_used, shape.renorm)
                hl = W.make_layer(shape, seed, l, experts=sel_o)
                ref, sel_r, _ = orc.moe_layer(hl, fx, xs[l])
                assert np.array_equal(sel_r, sel_o)
                m = parity.assert_parity(xs[l + 1], ref, f"stack {shape.name} token {tok} layer {l}")
                worst = {"max_rel": max(worst["max_rel"], m["max_rel"]), "cos": min(worst["cos"], m["cos"]),
                         "bit_identical": min(worst["bit_identical"], m["bit_identical"])}
            print(f"   48 layers against the oracle, worst {worst}", flush=True)
            st.set_option(H.OPT_PERSISTENT_DECODE, 0)
            launched = st.decode(x, 0, NL, W.RMS_EPS)
            st.set_option(H.OPT_PERSISTENT_DECODE, 2)
            m = parity.assert_parity(launched, whole, f"stack {shape.name} token {tok}: per-layer launches vs one launch")
            print(f"   per-layer launches vs one launch {m}", flush=True)
    finally:
        st.close()


def test_headline_stack_48_layers(orc):
    _stack_against_oracle(orc, SHAPE, 31, H.DECODE_XCD)


def test_qwen3_next_stack_48_layers(orc):
    """The Qwen3-Next-shaped decode at its stated depth: 48 layers of 512
    experts, top-10 and the sigmoid-gated shared expert (50 GB resident),
    through the rows-spread one-launch kernel, whose exchange tags and
    mailboxes are carried across all 48 layers."""
    _stack_against_oracle(orc, W.QWEN3_NEXT, 37, H.DECODE_SPREAD)


def _replay(trace, k):
    """Slots and misses of the host LRU replay, per (token, layer)."""
    lib = H.load_library()
    p = ctypes.c_void_p()
    T = trace.sel.shape[0]
    slots = np.zeros((T, NL, SHAPE.n_used), np.int32)
    miss = np.zeros((T, NL, SHAPE.n_used), np.uint8)
    H.check(lib.hoard_slot_lru_create(NL, SHAPE.n_expert, k, 0, ctypes.byref(p)))
    try:
        for t in range(T):
            for l in range(NL):
                sel = np.ascontiguousarray(trace.sel[t, l])
                H.check(lib.hoard_slot_lru_access(p, l, sel.ctypes.data, SHAPE.n_used, slots[t, l].ctypes.data,
                                                  miss[t, l].ctypes.data))
    finally:
        lib.hoard_slot_lru_destroy(p)
    return slots, miss


def test_pool_workload_512_tokens_48_layers():
    from hoard_amd.runtime import MoEStage
    seed, K, T = 0, 32, 512
    trace = W.routing_trace(SHAPE, seed, tokens=T, n_layer=NL)
    slots_ref, miss_ref = _replay(trace, K)
    res = MoEStage(SHAPE, n_layer=NL)
    pool = MoEStage(SHAPE, n_layer=NL, pool_k=K)
    try:
        print("pool workload: uploading 48 layers (resident) and pinned masters (pool)", flush=True)
        _fill([res, pool], seed)
        dev = torch.device("cuda")
        n_hid = 16
        hid = [W.make_hidden(SHAPE, seed, 0, t) for t in range(n_hid)]
        fx_d = torch.stack([torch.from_numpy(f) for f, _ in hid]).to(dev)
        x0_d = torch.stack([torch.from_numpy(r) for _, r in hid]).to(dev)
        sel_d = torch.from_numpy(trace.sel).to(dev)
        w_d = torch.from_numpy(trace.w).to(dev)
        xp = torch.empty((T, SHAPE.n_embd), device=dev)
        xr = torch.empty((T, SHAPE.n_embd), device=dev)
        slots_d = torch.empty((NL, SHAPE.n_used), dtype=torch.int32, device=dev)
        slots_h = np.zeros((T, NL, SHAPE.n_used), np.int32)
        copy_stream = torch.cuda.Stream()
        sp = pool.stream()
        cp = ctypes.c_void_p(copy_stream.cuda_stream)
        pool.reset_stats()
        for t in range(T):
            if t % 128 == 0:
                print(f"pool workload: token {t}", flush=True)
            xp[t].copy_(x0_d[t % n_hid])
            xr[t].copy_(x0_d[t % n_hid])
            fx = fx_d[t % n_hid]
            for l in range(NL):
                sel_h = np.ascontiguousarray(trace.sel[t, l])
                H.check(pool.lib.hoard_moe_pool_ensure(pool.h, l, sel_h.ctypes.data, slots_h[t, l].ctypes.data,
                                                       pool.ptr(slots_d[l]), sp, cp))
                pool.ffn_combine_dev(l, fx, slots_d[l], w_d[t, l], xp[t], xp[t])
                res.ffn_combine_dev(l, fx, sel_d[t, l], w_d[t, l], xr[t], xr[t])
        torch.cuda.synchronize()
        st = pool.stats()
        n_req = T * NL * SHAPE.n_used
        misses = int(miss_ref.sum())
        print(f"pool workload: hit rate {1 - misses / n_req:.4f}, {misses} misses", flush=True)
        assert np.array_equal(slots_h, slots_ref)
        assert (st.reqs, st.misses, st.hits) == (n_req, misses, n_req - misses)
        assert st.bytes_h2d == misses * SHAPE.expert_bytes()
        a, b = xp.cpu().numpy(), xr.cpu().numpy()
        assert np.all(np.isfinite(a))
        diff = np.nonzero(np.any(a.view(np.uint32) != b.view(np.uint32), axis=1))[0]
        assert diff.size == 0, f"tokens differing from the resident handle: {diff[:10]}"
    finally:
        pool.close()
        res.close()
