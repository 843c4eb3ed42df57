"""Device parity: the HIP path through the C ABI against the CPU oracle.

Bar: top-k indices identical; layer outputs max|d| <= 2e-3*||y||_inf and
cosine >= 0.9999.  The kernels reproduce the CPU path's Q8_K activation
quantisation and integer super-block sums, and the router logits in the CPU
dot's fma order, so in practice most outputs are bit-identical; the printed
bit_identical fraction tracks that.
"""
import ctypes

import numpy as np
import pytest

import parity
from hoard_amd import workloads as W

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _stage(shape, layers, **kw):
    from hoard_amd.runtime import MoEStage
    return MoEStage(shape, n_layer=max(layers, default=0) + 1, layers=layers, **kw)


@pytest.fixture(scope="module", params=[W.QWEN3_30B, W.QWEN3_NEXT, W.OLMOE, W.QWEN35, W.OLMOE_Q3],
                ids=lambda s: s.name)
def resident(request):
    shape = request.param
    nl = 1 if shape in (W.OLMOE, W.OLMOE_Q3) else 2
    layers = {l: W.make_layer(shape, 0, l) for l in range(nl)}
    st = _stage(shape, layers)
    yield shape, layers, st
    st.close()


def test_route_matches_oracle(orc, resident):
    shape, layers, st = resident
    for l, hl in layers.items():
        for t in range(6):
            fx, _ = W.make_hidden(shape, 0, l, t)
            print(f"route {shape.name} layer {l} token {t}", flush=True)
            sel, w = st.route(l, fx)
            sel_o, w_o, p = orc.route(hl.router, fx, shape.n_expert, shape.n_used, shape.renorm)
            assert np.array_equal(sel, sel_o), (sel, sel_o)
            assert np.allclose(w, w_o, rtol=1e-6, atol=0), (w, w_o)


def test_ffn_combine_matches_oracle(orc, resident):
    shape, layers, st = resident
    for l, hl in layers.items():
        for t in range(3):
            fx, res = W.make_hidden(shape, 0, l, t)
            sel_o, w_o, _ = orc.route(hl.router, fx, shape.n_expert, shape.n_used, shape.renorm)
            print(f"ffn_combine {shape.name} layer {l} token {t} sel {list(sel_o)}", flush=True)
            out = st.ffn_combine(l, fx, sel_o, w_o, res)
            ref = orc.moe_ffn_combine(hl, fx, sel_o, w_o, res)
            m = parity.assert_parity(out, ref, f"{shape.name} l{l} t{t}")
            print("  ", m, flush=True)


def test_layer_matches_oracle(orc, resident):
    shape, layers, st = resident
    for l, hl in layers.items():
        fx, res = W.make_hidden(shape, 0, l, 99)
        print(f"layer {shape.name} layer {l}", flush=True)
        out, sel, w = st.layer(l, fx, res)
        ref, sel_o, w_o = orc.moe_layer(hl, fx, res)
        assert np.array_equal(sel, sel_o)
        parity.assert_parity(out, ref, f"{shape.name} layer {l}")


def test_arbitrary_ids_and_repeats(orc, resident):
    """ffn_combine over caller-chosen ids, duplicates included (graph B takes any slot list)."""
    shape, layers, st = resident
    hl = layers[0]
    fx, res = W.make_hidden(shape, 0, 0, 5)
    ids = np.array([shape.n_expert - 1, 0, 3, 3] + list(range(7, 7 + shape.n_used - 4)), np.int32)
    w = np.linspace(0.3, -0.2, shape.n_used).astype(np.float32)
    print(f"arbitrary ids {shape.name} {list(ids)}", flush=True)
    out = st.ffn_combine(0, fx, ids, w, res)
    ref = orc.moe_ffn_combine(hl, fx, ids, w, res)
    parity.assert_parity(out, ref, "arbitrary ids")


def test_out_of_range_ids_poison_not_fault(resident):
    shape, layers, st = resident
    fx, res = W.make_hidden(shape, 0, 0, 6)
    ids = np.arange(shape.n_used, dtype=np.int32)
    ids[2] = shape.n_expert + 3
    w = np.full(shape.n_used, 0.1, np.float32)
    print(f"poison ids {shape.name}", flush=True)
    out = st.ffn_combine(0, fx, ids, w, res)
    assert np.all(np.isnan(out))
    ids[2] = -1
    out = st.ffn_combine(0, fx, ids, w, res)
    assert np.all(np.isnan(out))
    ids[2] = 2  # the handle still works afterwards
    assert np.all(np.isfinite(st.ffn_combine(0, fx, ids, w, res)))


def test_deterministic(resident):
    shape, layers, st = resident
    fx, res = W.make_hidden(shape, 0, 0, 7)
    a = st.layer(0, fx, res)[0]
    b = st.layer(0, fx, res)[0]
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_layer_kernels_match_generic(resident):
    """hoard_moe_layer through the kernels compiled for the shape gives the
    shape-generic kernels' bits: output, selected experts and weights."""
    import hoard_amd as H
    shape, layers, st = resident
    try:
        for l in layers:
            for t in range(4):
                fx, res = W.make_hidden(shape, 3, l, t)
                print(f"layer kernels {shape.name} layer {l} token {t}", flush=True)
                st.set_option(H.OPT_LAYER_KERNELS, 1)
                o1, s1, w1 = st.layer(l, fx, res)
                st.set_option(H.OPT_LAYER_KERNELS, 0)
                o0, s0, w0 = st.layer(l, fx, res)
                assert np.array_equal(s1, s0), (s1, s0)
                assert np.array_equal(w1.view(np.uint32), w0.view(np.uint32))
                assert np.array_equal(o1.view(np.uint32), o0.view(np.uint32))
    finally:
        st.set_option(H.OPT_LAYER_KERNELS, 1)


def test_olmoe_seeds_0_to_63(orc):
    """OLMoE-shaped layer, seeds 0..63, one token each (each seed its own weights)."""
    shape = W.OLMOE
    st = _stage(shape, {})
    worst = {"max_rel": 0.0, "cos": 1.0}
    try:
        for seed in range(64):
            router = W.make_router(shape, seed, 0)
            fx, res = W.make_hidden(shape, seed, 0, 0)
            sel_o, w_o, _ = orc.route(router, fx, shape.n_expert, shape.n_used, shape.renorm)
            hl = W.make_layer(shape, seed, 0, experts=sel_o)
            st.set_layer(0, hl)
            print(f"olmoe seed {seed}", flush=True)
            out, sel, w = st.layer(0, fx, res)
            assert np.array_equal(sel, sel_o), (seed, sel, sel_o)
            ref, _, _ = orc.moe_layer(hl, fx, res)
            m = parity.assert_parity(out, ref, f"olmoe seed {seed}")
            worst["max_rel"] = max(worst["max_rel"], m["max_rel"])
            worst["cos"] = min(worst["cos"], m["cos"])
    finally:
        st.close()
    print("olmoe 64 seeds worst", worst, flush=True)


def test_decode_chain_per_layer(orc):
    """Stacked decode on device (fx = rms_norm(x) fused into the router) against the
    oracle applied layer by layer to the device's own input of each layer; one call
    per layer runs the per-layer launches, the whole range one cooperative launch."""
    import hoard_amd as H
    shape = W.QWEN3_30B
    nl = 3
    layers = {l: W.make_layer(shape, 0, l) for l in range(nl)}
    st = _stage(shape, layers)
    try:
        assert st.get_option(H.OPT_PERSISTENT_DECODE) == 1
        _, x = W.make_hidden(shape, 0, 0, 0)
        xs = [x]
        for l in range(nl):
            print(f"decode layer {l}", flush=True)
            xs.append(st.decode(xs[-1], l, l + 1, W.RMS_EPS))
        for l in range(nl):
            fx = orc.rms_norm(xs[l], W.RMS_EPS)
            ref, _, _ = orc.moe_layer(layers[l], fx, xs[l])
            parity.assert_parity(xs[l + 1], ref, f"decode layer {l}")
        whole = st.decode(xs[0], 0, nl, W.RMS_EPS)
        st.sync_check()
        parity.assert_parity(whole, xs[-1], "one launch vs per-layer launches")
    finally:
        st.close()


@pytest.mark.parametrize("shape", [W.QWEN3_30B, W.OLMOE, W.OLMOE_Q3], ids=lambda s: s.name)
def test_persistent_decode_matches_oracle_and_launch_path(orc, shape):
    """One-launch stacked decode (router, experts per XCD, combine, rms_norm) against the
    oracle layer by layer, and against the per-layer launch path on the same input."""
    import hoard_amd as H
    nl = 4
    layers = {l: W.make_layer(shape, 1, l) for l in range(nl)}
    st = _stage(shape, layers)
    try:
        assert st.get_option(H.OPT_PERSISTENT_AVAILABLE) == 1
        st.set_option(H.OPT_PERSISTENT_DECODE, 2)
        for tok in range(3):
            _, x = W.make_hidden(shape, 1, 0, tok)
            xs = [x]
            for l in range(nl):
                print(f"persistent {shape.name} token {tok} layer {l}", flush=True)
                xs.append(st.decode(xs[-1], l, l + 1, W.RMS_EPS))
                st.sync_check()
            for l in range(nl):
                fx = orc.rms_norm(xs[l], W.RMS_EPS)
                ref, _, _ = orc.moe_layer(layers[l], fx, xs[l])
                m = parity.assert_parity(xs[l + 1], ref, f"persistent {shape.name} tok {tok} layer {l}")
                print("  ", m, flush=True)
            print(f"persistent {shape.name} token {tok} all layers", flush=True)
            whole = st.decode(xs[0], 0, nl, W.RMS_EPS)
            st.sync_check()
            assert np.array_equal(whole.view(np.uint32), xs[-1].view(np.uint32))
            st.set_option(H.OPT_PERSISTENT_DECODE, 0)
            launched = st.decode(xs[0], 0, nl, W.RMS_EPS)
            st.set_option(H.OPT_PERSISTENT_DECODE, 2)
            parity.assert_parity(whole, launched, "persistent vs per-layer launches")
            st.set_option(H.OPT_DECODE_LAUNCH, 1)  # plain launch of the same kernel: the same bits
            plain = st.decode(xs[0], 0, nl, W.RMS_EPS)
            st.sync_check()
            st.set_option(H.OPT_DECODE_LAUNCH, 0)
            assert np.array_equal(plain.view(np.uint32), whole.view(np.uint32))
    finally:
        st.close()


@pytest.mark.parametrize("shape,kernel", [(W.QWEN3_NEXT, 0), (W.QWEN3_30B, 2), (W.QWEN35, 0)],
                         ids=["qwen3_next-auto", "qwen3_30b-spread", "qwen35-auto"])
def test_spread_decode_matches_oracle_and_launch_path(orc, shape, kernel):
    """One-launch decode with every expert's rows spread over all CUs (router over all
    E, top-k of up to 512, shared expert, combine, rms_norm) against the oracle layer by
    layer, the whole range in one launch against the layer-by-layer chain, and both
    against the per-layer launch path."""
    import hoard_amd as H
    nl = 3
    layers = {l: W.make_layer(shape, 1, l) for l in range(nl)}
    st = _stage(shape, layers)
    try:
        assert st.get_option(H.OPT_PERSISTENT_AVAILABLE) == 1
        assert st.get_option(H.OPT_DECODE_KERNELS_AVAILABLE) & 2
        st.set_option(H.OPT_DECODE_KERNEL, kernel)
        st.set_option(H.OPT_PERSISTENT_DECODE, 2)
        for tok in range(3):
            _, x = W.make_hidden(shape, 1, 0, tok)
            xs = [x]
            for l in range(nl):
                print(f"spread {shape.name} token {tok} layer {l}", flush=True)
                xs.append(st.decode(xs[-1], l, l + 1, W.RMS_EPS))
                st.sync_check()
            for l in range(nl):
                fx = orc.rms_norm(xs[l], W.RMS_EPS)
                ref, _, _ = orc.moe_layer(layers[l], fx, xs[l])
                m = parity.assert_parity(xs[l + 1], ref, f"spread {shape.name} tok {tok} layer {l}")
                print("  ", m, flush=True)
            print(f"spread {shape.name} token {tok} all layers", flush=True)
            whole = st.decode(xs[0], 0, nl, W.RMS_EPS)
            st.sync_check()
            assert np.array_equal(whole.view(np.uint32), xs[-1].view(np.uint32))
            st.set_option(H.OPT_PERSISTENT_DECODE, 0)
            launched = st.decode(xs[0], 0, nl, W.RMS_EPS)
            st.set_option(H.OPT_PERSISTENT_DECODE, 2)
            parity.assert_parity(whole, launched, "spread vs per-layer launches")
            st.set_option(H.OPT_DECODE_LAUNCH, 1)
            plain = st.decode(xs[0], 0, nl, W.RMS_EPS)
            st.sync_check()
            st.set_option(H.OPT_DECODE_LAUNCH, 0)
            assert np.array_equal(plain.view(np.uint32), whole.view(np.uint32))
            if shape is W.QWEN3_30B:
                st.set_option(H.OPT_DECODE_KERNEL, 1)
                per_xcd = st.decode(xs[0], 0, nl, W.RMS_EPS)
                st.sync_check()
                st.set_option(H.OPT_DECODE_KERNEL, kernel)
                parity.assert_parity(whole, per_xcd, "spread vs expert-per-XCD kernel")
    finally:
        st.close()


def test_persistent_decode_unavailable_shape_falls_back():
    import dataclasses

    import hoard_amd as H
    shape = dataclasses.replace(W.QWEN3_NEXT, n_used=6)  # top-6 of 512: no one-launch kernel
    st = _stage(shape, {0: W.make_layer(shape, 0, 0, experts=[])})
    try:
        assert st.get_option(H.OPT_PERSISTENT_AVAILABLE) == 0
        assert st.get_option(H.OPT_DECODE_KERNELS_AVAILABLE) == 0
        with pytest.raises(H.HoardError):
            st.set_option(H.OPT_PERSISTENT_DECODE, 2)
        with pytest.raises(H.HoardError):
            st.set_option(H.OPT_DECODE_KERNEL, 2)
    finally:
        st.close()


def test_decode_splits_the_range_where_layer_types_change(orc):
    """Layers 0-2 with Q6_K down experts and layer 3 with Q4_K (a Q4_K_M file's mix):
    automatic mode decodes layers 0-2 in one launch and layer 3 with the per-layer
    kernels, and the result matches the oracle layer by layer and the all-launches path."""
    import ctypes
    import dataclasses

    import hoard_amd as H
    shape = W.QWEN3_30B
    shapes = [shape] * 3 + [dataclasses.replace(shape, down_type=H.TYPE_Q4_K)]
    layers = {l: W.make_layer(shapes[l], 5, l) for l in range(4)}
    st = _stage(shape, layers)
    try:
        assert st.get_option(H.OPT_PERSISTENT_DECODE) == 1
        _, x = W.make_hidden(shape, 5, 0, 0)
        H.check(st.lib.hoard_moe_profile(st.h, 1))
        print("mixed-type decode of 4 layers", flush=True)
        y = st.decode(x, 0, 4, W.RMS_EPS)
        st.sync_check()
        kt = H.KernelTimes()
        H.check(st.lib.hoard_moe_profile_read(st.h, ctypes.byref(kt)))
        H.check(st.lib.hoard_moe_profile(st.h, 0))
        assert kt.launches[H.KERNEL_DECODE] == 1 and kt.launches[H.KERNEL_ROUTER] == 1, list(kt.launches)
        xs = [x]
        for l in range(4):  # the per-layer path, layer by layer, each checked against the oracle
            xs.append(st.decode(xs[-1], l, l + 1, W.RMS_EPS))
            ref, _, _ = orc.moe_layer(layers[l], orc.rms_norm(xs[l], W.RMS_EPS), xs[l])
            parity.assert_parity(xs[-1], ref, f"mixed types layer {l}")
        parity.assert_parity(y, xs[-1], "split range vs layer by layer")
        st.set_option(H.OPT_PERSISTENT_DECODE, 0)
        launched = st.decode(x, 0, 4, W.RMS_EPS)
        assert np.array_equal(launched.view(np.uint32), xs[-1].view(np.uint32))
        st.set_option(H.OPT_PERSISTENT_DECODE, 2)  # one launch over mixed types: refused before any launch
        with pytest.raises(H.HoardError) as ei:
            st.decode(x, 0, 4, W.RMS_EPS)
        assert ei.value.code == H.ERR_UNSUPPORTED
    finally:
        st.close()


# more than 128 experts: the one-launch layer's waiting workgroups run the router tail
E256 = W.Shape("e256_k8", 11, 2048, 256, 8, 512, 1, W.TYPE_Q4_K, W.TYPE_Q4_K, W.TYPE_Q6_K, 1)
# more than 8 experts per token without a shared expert: more than 64 down rows
# per workgroup, Q6_K rows (pairs of rows per 8-lane group) and Q4_K rows
E128_K10 = W.Shape("e128_k10", 12, 2048, 128, 10, 768, 1, W.TYPE_Q4_K, W.TYPE_Q4_K, W.TYPE_Q6_K, 1)
E64_K10_Q4 = W.Shape("e64_k10_q4", 13, 2048, 64, 10, 1024, 0, W.TYPE_Q4_K, W.TYPE_Q4_K, W.TYPE_Q4_K, 1)


def _kernel_launches(st):
    import hoard_amd as H
    kt = H.KernelTimes()
    H.check(st.lib.hoard_moe_profile_read(st.h, ctypes.byref(kt)))
    return list(kt.launches)


@pytest.mark.parametrize("shape", [W.QWEN3_30B, W.OLMOE, E256, E128_K10, E64_K10_Q4, W.QWEN3_NEXT, W.QWEN35,
                                   W.OLMOE_Q3], ids=lambda s: s.name)
def test_fused_layer_matches_three_launches(orc, shape):
    """hoard_moe_layer in one launch (router, gate/up and down workgroups in the
    order they start; the shared expert's workgroups first) against the three
    launches per layer: the same output, selection and weights bit for bit, for
    several tokens and layers in a row (the launches' counters carry over), and
    the per-layer decode the same way."""
    import hoard_amd as H
    nl = 3
    layers = {l: W.make_layer(shape, 14, l) for l in range(nl)}
    st = _stage(shape, layers)
    try:
        assert st.get_option(H.OPT_LAYER_FUSED) == 1
        for t in range(4):
            for l in range(nl):
                fx, res = W.make_hidden(shape, 14, l, t)
                print(f"fused layer {shape.name} token {t} layer {l}", flush=True)
                st.set_option(H.OPT_LAYER_FUSED, 1)
                H.check(st.lib.hoard_moe_profile(st.h, 1))
                o1, s1, w1 = st.layer(l, fx, res)
                launches = _kernel_launches(st)
                H.check(st.lib.hoard_moe_profile(st.h, 0))
                assert launches[H.KERNEL_LAYER] == 1 and launches[H.KERNEL_GATEUP] == 0, launches
                st.set_option(H.OPT_LAYER_FUSED, 0)
                o0, s0, w0 = st.layer(l, fx, res)
                assert np.array_equal(s1, s0) and np.array_equal(w1.view(np.uint32), w0.view(np.uint32))
                assert np.array_equal(o1.view(np.uint32), o0.view(np.uint32))
                if t == 0:
                    ref, sel_o, _ = orc.moe_layer(layers[l], fx, res)
                    assert np.array_equal(s1, sel_o)
                    parity.assert_parity(o1, ref, f"fused {shape.name} layer {l}")
        st.set_option(H.OPT_PERSISTENT_DECODE, 0)
        _, x = W.make_hidden(shape, 14, 0, 9)
        st.set_option(H.OPT_LAYER_FUSED, 1)
        y1 = st.decode(x, 0, nl, W.RMS_EPS)
        st.sync_check()
        st.set_option(H.OPT_LAYER_FUSED, 0)
        y0 = st.decode(x, 0, nl, W.RMS_EPS)
        assert np.array_equal(y1.view(np.uint32), y0.view(np.uint32))
    finally:
        st.set_option(H.OPT_LAYER_FUSED, 1)
        st.close()
