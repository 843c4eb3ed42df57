"""The C ABI from C++: tests/c_consumer/consumer.cpp includes include/*.h only,
links libhoard_moe.so and drives what hoard's loader and layer loop would
(GGUF reader, storage tier, slot LRU, one layer, the pooled verify step).  Its
results are checked here against the file and the oracle."""
import subprocess
from pathlib import Path

import numpy as np
import pytest

import hoard_amd as H
from gguf_writer import write_layers
from hoard_amd import workloads as W

HERE = Path(__file__).resolve().parent
BIN = HERE / "c_consumer" / "consumer"


def _binary(build_if_missing: bool) -> Path:
    if not BIN.exists():
        if not build_if_missing:
            pytest.fail(f"{BIN} is not built: run __graft_entry__.build()")
        import importlib.util
        spec = importlib.util.spec_from_file_location("c_consumer_build", HERE / "c_consumer" / "build.py")
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        mod.build()
    return BIN


def _run(*args) -> str:
    r = subprocess.run([str(BIN), *map(str, args)], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                       timeout=240)
    assert r.returncode == 0, r.stdout
    return r.stdout


def test_host_side_from_cpp(tmp_path):
    _binary(True)
    shape = W.Shape("tiny", 0, 512, 6, 2, 256, 1, H.TYPE_Q4_K, H.TYPE_Q4_K, H.TYPE_Q6_K, 2, n_ff_shexp=256)
    layers = {l: W.make_layer(shape, 5, l) for l in range(2)}
    p = tmp_path / "tiny.gguf"
    write_layers(p, shape, layers, "qwen3next", eps=1e-6)
    out = _run("host", p)
    print(out)
    f = dict(kv.split("=") for kv in out.split()[2:])
    assert (f["arch"], f["layers"], f["embd"], f["experts"], f["ff"], f["shexp"], f["renorm"]) == \
        ("qwen3next", "2", "512", "2/6", "256", "256", "1")
    assert float(f["eps"]) == pytest.approx(1e-6)
    assert f["checked"] == "18" and f["reads"] == "6"  # 3 experts x 3 tensors x 2 layers, all read once
    assert f["misses"] == "1010"  # the verify loop's order: 3 miss, 3 hit, 1 miss, 3 hit


@pytest.mark.gpu
def test_layer_and_verify_step_from_cpp(orc, tmp_path):
    _binary(False)
    shape = W.QWEN3_30B
    layers = {l: W.make_layer(shape, 8, l) for l in range(2)}
    p = tmp_path / "qwen3_30b_2l.gguf"
    write_layers(p, shape, layers, "qwen3moe")
    hl = layers[0]
    # one resident layer
    fx, res = W.make_hidden(shape, 8, 0, 0)
    np.concatenate([fx, res]).astype(np.float32).tofile(tmp_path / "in1.bin")
    print(_run("layer", p, tmp_path / "in1.bin", tmp_path / "out1.bin"), flush=True)
    raw = np.fromfile(tmp_path / "out1.bin", dtype=np.uint8)
    y = raw[:4 * shape.n_embd].view(np.float32)
    sel = raw[4 * shape.n_embd:4 * (shape.n_embd + shape.n_used)].view(np.int32)
    ref, sel_o, _ = orc.moe_layer(hl, fx, res)
    assert np.array_equal(sel, sel_o)
    import parity
    parity.assert_parity(y, ref, "C++ consumer, one layer")
    # the verify step: 4 tokens through a 32-slot pool streamed from the file
    M = 4
    toks = [W.make_hidden(shape, 8, 0, 10 + t) for t in range(M)]
    np.concatenate([np.concatenate(t) for t in toks]).astype(np.float32).tofile(tmp_path / "in4.bin")
    print(_run("verify", p, tmp_path / "in4.bin", tmp_path / "out4.bin", 32), flush=True)
    raw = np.fromfile(tmp_path / "out4.bin", dtype=np.uint8)
    per = 4 * (shape.n_embd + 2 * shape.n_used)
    for t, (fx_t, res_t) in enumerate(toks):
        r = raw[t * per:(t + 1) * per]
        y_t = r[:4 * shape.n_embd].view(np.float32)
        s_t = r[4 * shape.n_embd:4 * (shape.n_embd + shape.n_used)].view(np.int32)
        w_t = r[4 * (shape.n_embd + shape.n_used):].view(np.float32)
        sel_o, w_o, _ = orc.route(hl.router, fx_t, shape.n_expert, shape.n_used, shape.renorm)
        assert np.array_equal(s_t, sel_o), t
        ref = orc.moe_ffn_combine(hl, fx_t, s_t, w_t, res_t)
        parity.assert_parity(y_t, ref, f"C++ consumer, verify token {t}")
