"""Writes tests/golden/moe_layer_golden.npz: oracle outputs of one MoE layer
for a few seeded synthetic inputs, the regression fixture for the oracle, the
synthetic-weight generator and the device path.

Run from the repository root after building (python -m hoard_amd.build and the
oracle):  python tests/golden/make_fixtures.py
Cases: OLMoE-shaped layer 0 for seeds 0..3 (two tokens each) and the
Qwen3-30B-A3B-shaped layer 0 for seed 0 (four tokens).  Inputs are not stored:
they are regenerated from (shape, seed, layer, token); a digest of the first
expert's bytes is stored to pin the generator.
"""
import hashlib
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

import oracle  # noqa: E402
from hoard_amd import workloads as W  # noqa: E402

CASES = [("olmoe", s, 0, t) for s in range(4) for t in range(2)] + [("qwen3_30b", 0, 0, t) for t in range(4)]


def compute(cases=CASES):
    out = {}
    layers = {}
    for name, seed, layer, tok in cases:
        shape = W.SHAPES[name]
        key = (name, seed, layer)
        if key not in layers:
            layers[key] = W.make_layer(shape, seed, layer)
        hl = layers[key]
        fx, res = W.make_hidden(shape, seed, layer, tok)
        y, sel, w = oracle.moe_layer(hl, fx, res)
        tag = f"{name}_s{seed}_l{layer}_t{tok}"
        out[tag + "_sel"] = np.asarray(sel, np.int32)
        out[tag + "_w"] = np.asarray(w, np.float32)
        out[tag + "_y"] = np.asarray(y, np.float32)
        stride = hl.stride("gate")
        out[f"{name}_s{seed}_l{layer}_gate0_sha256"] = np.frombuffer(
            hashlib.sha256(hl.gate[:stride].tobytes()).digest(), dtype=np.uint8)
    return out


if __name__ == "__main__":
    data = compute()
    dst = Path(__file__).resolve().parent / "moe_layer_golden.npz"
    np.savez_compressed(dst, **data)
    print(f"wrote {dst} ({dst.stat().st_size} bytes, {len(data)} arrays)")
