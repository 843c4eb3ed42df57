"""GGUF reader (include/hoard_gguf.h): metadata, tensor lookup and the per-layer
weights the stage takes, on synthetic files written from the format's spec.
Host only: the reader makes no device calls."""
import ctypes

import numpy as np
import pytest

import hoard_amd as H
from gguf_writer import (ARRAY, BOOL, F32, F64, GGML_BF16, GGML_F16, GGML_F32, GGML_Q4_K, GGML_Q6_K, GGML_Q8_0,
                         I32, STRING, U8, U32, bf16, write_gguf)
from hoard_amd.gguf import GGUFWeights

EMBD, FF, E, K, FF_SH = 512, 256, 4, 2, 256


def q4k(rows, cols, rng):
    return rng.integers(0, 256, rows * (cols // 256) * 144, dtype=np.uint8).tobytes()


def q6k(rows, cols, rng):
    return rng.integers(0, 256, rows * (cols // 256) * 210, dtype=np.uint8).tobytes()


def model(arch="qwen3moe", n_layer=2, shared=False, router_type=GGML_F32, seed=0):
    """(kv, tensors, expected) of a small MoE model with distractor keys and tensors."""
    rng = np.random.default_rng(seed)
    kv = [("general.architecture", STRING, arch),
          ("general.alignment", U32, 32),
          ("general.name", STRING, "synthetic"),
          ("tokenizer.ggml.tokens", ARRAY, (STRING, ["a", "bb", "ccc"])),
          ("tokenizer.ggml.scores", ARRAY, (F32, [0.5, 1.5, 2.5])),
          ("general.nested", ARRAY, (ARRAY, [(U32, [1, 2]), (STRING, ["x"]), (ARRAY, [(I32, [-1])])])),
          ("general.flag", BOOL, True),
          ("general.small", U8, 7),
          ("general.signed", I32, -3),
          ("general.double", F64, 2.25),
          (f"{arch}.block_count", U32, n_layer),
          (f"{arch}.embedding_length", U32, EMBD),
          (f"{arch}.feed_forward_length", U32, 3 * EMBD),
          (f"{arch}.expert_feed_forward_length", U32, FF),
          (f"{arch}.expert_count", U32, E),
          (f"{arch}.expert_used_count", U32, K),
          (f"{arch}.attention.layer_norm_rms_epsilon", F32, 1e-6)]
    if shared:
        kv.append((f"{arch}.expert_shared_feed_forward_length", U32, FF_SH))
    tensors = [("token_embd.weight", GGML_Q4_K, [EMBD, 10], q4k(10, EMBD, rng))]
    exp = {}
    for l in range(n_layer):
        router = rng.normal(0, 0.02, (E, EMBD)).astype(np.float32)
        if router_type == GGML_F32:
            rbytes, rf32 = router.tobytes(), router
        elif router_type == GGML_F16:
            h = router.astype(np.float16)
            rbytes, rf32 = h.tobytes(), h.astype(np.float32)
        else:
            rbytes = bf16(router)
            rf32 = (np.frombuffer(rbytes, np.uint16).astype(np.uint32) << 16).view(np.float32).reshape(E, EMBD)
        g, u, d = q4k(E * FF, EMBD, rng), q4k(E * FF, EMBD, rng), q6k(E * EMBD, FF, rng)
        tensors += [(f"blk.{l}.attn_norm.weight", GGML_F32, [EMBD], np.ones(EMBD, np.float32).tobytes()),
                    (f"blk.{l}.ffn_gate_inp.weight", router_type, [EMBD, E], rbytes),
                    (f"blk.{l}.ffn_gate_exps.weight", GGML_Q4_K, [EMBD, FF, E], g),
                    (f"blk.{l}.ffn_up_exps.weight", GGML_Q4_K, [EMBD, FF, E], u),
                    (f"blk.{l}.ffn_down_exps.weight", GGML_Q6_K, [FF, EMBD, E], d)]
        exp[l] = {"router": rf32, "gate": g, "up": u, "down": d}
        if shared:
            sg, su, sd = q4k(FF_SH, EMBD, rng), q4k(FF_SH, EMBD, rng), q6k(EMBD, FF_SH, rng)
            gi = rng.normal(0, 0.02, EMBD).astype(np.float32)
            gb = bf16(gi)
            tensors += [(f"blk.{l}.ffn_gate_shexp.weight", GGML_Q4_K, [EMBD, FF_SH], sg),
                        (f"blk.{l}.ffn_up_shexp.weight", GGML_Q4_K, [EMBD, FF_SH], su),
                        (f"blk.{l}.ffn_down_shexp.weight", GGML_Q6_K, [FF_SH, EMBD], sd),
                        (f"blk.{l}.ffn_gate_inp_shexp.weight", GGML_BF16, [EMBD], gb)]
            exp[l].update(sh_gate=sg, sh_up=su, sh_down=sd,
                          sh_gate_inp=(np.frombuffer(gb, np.uint16).astype(np.uint32) << 16).view(np.float32))
    return kv, tensors, exp


def read(ptr, n):
    return ctypes.string_at(ptr, n)


def f32_at(ptr, n):
    return np.frombuffer(read(ptr, 4 * n), np.float32)


def test_metadata_and_layers(tmp_path):
    kv, tensors, exp = model()
    p = tmp_path / "m.gguf"
    write_gguf(p, kv, tensors)
    with GGUFWeights(p) as g:
        assert g.arch() == "qwen3moe"
        c = g.cfg()
        assert (c.n_embd, c.n_expert, c.n_used, c.n_ff, c.n_ff_shexp, c.n_layer, c.renorm, c.pool_k, c.max_tokens) == \
            (EMBD, E, K, FF, 0, 2, 1, 0, 1)
        assert g.rms_eps() == pytest.approx(1e-6)
        for l in range(2):
            w = g.layer_weights(l)
            assert (w.gate_type, w.up_type, w.down_type) == (H.TYPE_Q4_K, H.TYPE_Q4_K, H.TYPE_Q6_K)
            assert read(w.gate, len(exp[l]["gate"])) == exp[l]["gate"]
            assert read(w.up, len(exp[l]["up"])) == exp[l]["up"]
            assert read(w.down, len(exp[l]["down"])) == exp[l]["down"]
            assert np.array_equal(f32_at(w.router, E * EMBD), exp[l]["router"].ravel())
            assert not w.sh_gate and not w.sh_gate_inp
        t, ne, nb, addr = g.tensor("blk.1.ffn_down_exps.weight")
        assert (t, ne, nb) == (GGML_Q6_K, [FF, EMBD, E, 1], E * EMBD * (FF // 256) * 210)
        assert read(addr, nb) == exp[1]["down"]


@pytest.mark.parametrize("rt", [GGML_F16, GGML_BF16], ids=["f16", "bf16"])
def test_router_upconverted_to_f32(tmp_path, rt):
    kv, tensors, exp = model(router_type=rt, n_layer=1)
    p = tmp_path / "m.gguf"
    write_gguf(p, kv, tensors)
    with GGUFWeights(p) as g:
        w = g.layer_weights(0)
        got = f32_at(w.router, E * EMBD)
        assert np.array_equal(got.view(np.uint32), exp[0]["router"].ravel().view(np.uint32))
        assert g.layer_weights(0).router == w.router  # converted once, kept by the handle


def test_shared_expert_and_bf16_gate(tmp_path):
    """run_qwen35's gated shared expert (src/run_qwen35.cpp:659-665) with the bf16
    ffn_gate_inp_shexp it upconverts (:219, :250-253)."""
    kv, tensors, exp = model(arch="qwen3next", shared=True, n_layer=1)
    p = tmp_path / "m.gguf"
    write_gguf(p, kv, tensors)
    with GGUFWeights(p) as g:
        c = g.cfg()
        assert c.n_ff_shexp == FF_SH and c.renorm == 1
        w = g.layer_weights(0)
        assert (w.sh_gate_type, w.sh_up_type, w.sh_down_type) == (H.TYPE_Q4_K, H.TYPE_Q4_K, H.TYPE_Q6_K)
        assert read(w.sh_gate, len(exp[0]["sh_gate"])) == exp[0]["sh_gate"]
        assert read(w.sh_down, len(exp[0]["sh_down"])) == exp[0]["sh_down"]
        assert np.array_equal(f32_at(w.sh_gate_inp, EMBD).view(np.uint32), exp[0]["sh_gate_inp"].view(np.uint32))


def test_shared_ff_taken_from_the_tensor(tmp_path):
    kv, tensors, _ = model(arch="qwen3next", shared=True, n_layer=1)
    kv = [e for e in kv if not e[0].endswith("expert_shared_feed_forward_length")]
    p = tmp_path / "m.gguf"
    write_gguf(p, kv, tensors)
    with GGUFWeights(p) as g:
        assert g.cfg().n_ff_shexp == FF_SH


def test_olmoe_does_not_renormalise(tmp_path):
    kv, tensors, _ = model(arch="olmoe", n_layer=1)
    p = tmp_path / "m.gguf"
    write_gguf(p, kv, tensors)
    with GGUFWeights(p) as g:
        assert g.cfg().renorm == 0


def test_version_2_and_other_alignment(tmp_path):
    kv, tensors, exp = model(n_layer=1)
    kv = [(k, t, 64 if k == "general.alignment" else v) for k, t, v in kv]
    p = tmp_path / "m.gguf"
    write_gguf(p, kv, tensors, alignment=64, version=2)
    with GGUFWeights(p) as g:
        w = g.layer_weights(0)
        assert w.gate % 64 == 0
        assert read(w.gate, len(exp[0]["gate"])) == exp[0]["gate"]


def _expect_error(p, code):
    with pytest.raises(H.HoardError) as ei:
        GGUFWeights(p)
    assert ei.value.code == code, ei.value


def test_rejects_bad_files(tmp_path):
    kv, tensors, _ = model(n_layer=1)
    p = tmp_path / "bad_magic.gguf"
    write_gguf(p, kv, tensors, magic=b"GGML")
    _expect_error(p, H.ERR_INVALID)
    p = tmp_path / "v4.gguf"
    write_gguf(p, kv, tensors, version=4)
    _expect_error(p, H.ERR_UNSUPPORTED)
    good = tmp_path / "good.gguf"
    write_gguf(good, kv, tensors)
    data = good.read_bytes()
    for cut in (10, 40, len(data) // 3, len(data) - 100):
        p = tmp_path / f"cut{cut}.gguf"
        p.write_bytes(data[:cut])
        _expect_error(p, H.ERR_INVALID)
    _expect_error(tmp_path / "absent.gguf", H.ERR_INVALID)


def test_layer_errors(tmp_path):
    kv, tensors, _ = model(n_layer=2)
    # layer 1 lacks its down experts; layer 0's router has the wrong type
    tensors = [t for t in tensors if t[0] != "blk.1.ffn_down_exps.weight"]
    tensors = [(n, GGML_Q8_0, [EMBD, E], b"\0" * (EMBD // 32 * 34 * E)) if n == "blk.0.ffn_gate_inp.weight" else (n, ty, ne, d)
               for n, ty, ne, d in tensors]
    p = tmp_path / "m.gguf"
    write_gguf(p, kv, tensors)
    with GGUFWeights(p) as g:
        with pytest.raises(H.HoardError) as ei:
            g.layer_weights(1)
        assert "ffn_down_exps" in str(ei.value)
        with pytest.raises(H.HoardError):
            g.layer_weights(0)
        with pytest.raises(H.HoardError):
            g.layer_weights(2)
        with pytest.raises(H.HoardError):
            g.tensor("no.such.tensor")


def test_missing_hparams(tmp_path):
    kv, tensors, _ = model(n_layer=1)
    kv = [e for e in kv if not e[0].endswith("expert_count")]
    p = tmp_path / "m.gguf"
    write_gguf(p, kv, tensors)
    with GGUFWeights(p) as g:
        with pytest.raises(H.HoardError):
            g.cfg()


def test_f16_special_values(tmp_path):
    """Subnormals, signed zeros, infinities and NaN convert as numpy's f16 -> f32 does."""
    kv, tensors, _ = model(router_type=GGML_F16, n_layer=1)
    special = np.array([0.0, -0.0, 2 ** -24, -(2 ** -24), 2 ** -15, 1023 * 2 ** -24, 65504.0, -65504.0,
                        np.inf, -np.inf, 1.0, -2.5], np.float16)
    router = np.resize(special, E * EMBD).astype(np.float16)
    router[-3:] = np.frombuffer(np.array([0x7E00, 0x7C01, 0xFE00], np.uint16).tobytes(), np.float16)  # NaNs
    tensors = [(n, ty, ne, router.tobytes() if n == "blk.0.ffn_gate_inp.weight" else d) for n, ty, ne, d in tensors]
    p = tmp_path / "m.gguf"
    write_gguf(p, kv, tensors)
    with GGUFWeights(p) as g:
        got = f32_at(g.layer_weights(0).router, E * EMBD)
    want = router.astype(np.float32)
    fin = np.isfinite(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))
    assert np.array_equal(np.isnan(got), np.isnan(want)) and np.array_equal(np.isinf(got), np.isinf(want))
    assert np.array_equal(np.signbit(got), np.signbit(want))


def test_stage_layers_round_trip(tmp_path):
    """write_layers (the GPU test's file) holds the synthetic layer's bytes where the
    reader points, and shape() gives back the stage shape."""
    from gguf_writer import write_layers
    from hoard_amd import workloads as W
    shape = W.Shape("tiny", 0, 512, 4, 2, 256, 1, H.TYPE_Q4_K, H.TYPE_Q4_K, H.TYPE_Q6_K, 2, n_ff_shexp=256)
    layers = {l: W.make_layer(shape, 3, l) for l in range(2)}
    p = tmp_path / "m.gguf"
    held = write_layers(p, shape, layers, "qwen3next", {1: GGML_BF16})
    with GGUFWeights(p) as g:
        s = g.shape()
        assert (s.n_embd, s.n_expert, s.n_used, s.n_ff, s.n_ff_shexp, s.n_layer, s.renorm) == (512, 4, 2, 256, 256, 2, 1)
        assert (s.gate_type, s.down_type, s.sh_down_type) == (H.TYPE_Q4_K, H.TYPE_Q6_K, H.TYPE_Q6_K)
        for l, hl in layers.items():
            w = g.layer_weights(l)
            for name in ("gate", "up", "down", "sh_gate", "sh_up", "sh_down"):
                a = getattr(hl, name)
                assert read(getattr(w, name), a.nbytes) == a.tobytes(), name
            assert np.array_equal(f32_at(w.router, 4 * 512), held[l][0])
            assert np.array_equal(f32_at(w.sh_gate_inp, 512), held[l][1])
        assert np.array_equal(held[0][0], layers[0].router.ravel())


def test_streaming_writer_matches_layers(tmp_path):
    """The layer-by-layer writer bench.py uses for its storage-tier workload."""
    from gguf_writer import write_stage_streaming
    from hoard_amd import workloads as W
    shape = W.Shape("tiny", 0, 512, 4, 2, 256, 1, H.TYPE_Q4_K, H.TYPE_Q4_K, H.TYPE_Q6_K, 3, n_ff_shexp=256)
    layers = {l: W.make_layer(shape, 9, l) for l in range(3)}
    p = tmp_path / "s.gguf"
    write_stage_streaming(p, shape, 3, lambda l: layers[l], "qwen3next")
    with GGUFWeights(p) as g:
        c = g.cfg()
        assert (c.n_layer, c.n_ff_shexp, c.n_expert) == (3, 256, 4)
        for l, hl in layers.items():
            w = g.layer_weights(l)
            for name in ("gate", "up", "down", "sh_gate", "sh_up", "sh_down"):
                a = getattr(hl, name)
                assert read(getattr(w, name), a.nbytes) == a.tobytes(), (l, name)
            assert np.array_equal(f32_at(w.router, 4 * 512), hl.router.ravel())
