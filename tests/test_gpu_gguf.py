"""A stage loaded from a GGUF file (include/hoard_gguf.h -> hoard_moe_set_layer_weights)
against the oracle on the same weights: Qwen3-Next-shaped layers with an f32, a
bf16 and an f16 router and the bf16 shared-expert gate the reference
upconverts (src/run_qwen35.cpp:219, :250-253), and Qwen3-30B-shaped layers
whose down experts are Q6_K in one layer and Q4_K in the next, and an OLMoE
layer in its Q3_K_M form (Q3_K gate/up, Q5_K down, no renormalisation).  Same bar as the other parity
tests: identical top-k, max|d| <= 2e-3*||y||_inf, cosine >= 0.9999."""
import dataclasses

import numpy as np
import pytest

import parity
from gguf_writer import GGML_BF16, GGML_F16, GGML_F32, write_layers
import hoard_amd as H
from hoard_amd import workloads as W

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.mark.parametrize("shape,arch,routers", [(W.QWEN3_NEXT, "qwen3next", (GGML_BF16, GGML_F16)),
                                                (W.QWEN3_30B, "qwen3moe", (GGML_F32, GGML_BF16)),
                                                (W.OLMOE_Q3, "olmoe", (GGML_F32,))],
                         ids=["qwen3_next", "qwen3_30b", "olmoe_q3"])
def test_layers_from_gguf_match_oracle(orc, tmp_path, shape, arch, routers):
    from hoard_amd.runtime import MoEStage
    nl = len(routers)
    # layer 1 of the Qwen3-30B file has Q4_K down experts (mixed types per layer, as Q4_K_M files have)
    layer_shapes = [shape, dataclasses.replace(shape, down_type=H.TYPE_Q4_K) if shape is W.QWEN3_30B else shape]
    layers = {l: W.make_layer(layer_shapes[l], 4, l) for l in range(nl)}
    path = tmp_path / "model.gguf"
    held = write_layers(path, shape, layers, arch, dict(enumerate(routers)))
    # the oracle's view of each layer: the router and shared gate as the file holds them
    ref_layers = {l: dataclasses.replace(hl, router=held[l][0], sh_gate_inp=held[l][1]) for l, hl in layers.items()}
    print(f"gguf {shape.name}: {path.stat().st_size} bytes", flush=True)
    st = MoEStage.from_gguf(path)
    try:
        assert st.cfg.n_layer == nl and st.cfg.n_ff_shexp == shape.n_ff_shexp
        assert st.rms_eps == pytest.approx(1e-6)
        for l in range(nl):
            for t in range(2):
                fx, res = W.make_hidden(shape, 4, l, t)
                print(f"gguf {shape.name} layer {l} token {t}", flush=True)
                out, sel, w = st.layer(l, fx, res)
                ref, sel_o, w_o = orc.moe_layer(ref_layers[l], fx, res)
                assert np.array_equal(sel, sel_o), (sel, sel_o)
                m = parity.assert_parity(out, ref, f"gguf {shape.name} layer {l} token {t}")
                print("  ", m, flush=True)
        _, x = W.make_hidden(shape, 4, 0, 7)
        print(f"gguf {shape.name} decode of {nl} layers", flush=True)
        y = st.decode(x, 0, nl, st.rms_eps)
        st.sync_check()
        xr = x
        for l in range(nl):
            xr, _, _ = orc.moe_layer(ref_layers[l], orc.rms_norm(xr, st.rms_eps), xr)
        parity.assert_parity(y, xr, f"gguf {shape.name} decode")
    finally:
        st.close()
