"""Golden fixtures (tests/golden/moe_layer_golden.npz, written by
tests/golden/make_fixtures.py): the oracle and the seeded synthetic weights
must keep reproducing them bit for bit, and the device path must match them to
the parity bar with identical expert indices."""
from pathlib import Path

import numpy as np
import pytest

HERE = Path(__file__).resolve().parent
FIXTURE = HERE / "golden" / "moe_layer_golden.npz"


def _load():
    with np.load(FIXTURE) as f:  # allow_pickle stays False
        return {k: f[k] for k in f.files}


def test_oracle_and_generator_reproduce_fixture(orc):
    import sys
    sys.path.insert(0, str(HERE / "golden"))
    import make_fixtures
    gold = _load()
    now = make_fixtures.compute()
    assert set(now) == set(gold)
    for k in gold:
        assert np.array_equal(now[k], gold[k]), k


@pytest.mark.gpu
def test_device_matches_fixture():
    pytest.importorskip("torch")
    import sys
    sys.path.insert(0, str(HERE / "golden"))
    import make_fixtures
    import parity
    from hoard_amd import workloads as W
    from hoard_amd.runtime import MoEStage
    gold = _load()
    stages = {}
    try:
        for name, seed, layer, tok in make_fixtures.CASES:
            shape = W.SHAPES[name]
            key = (name, seed, layer)
            if key not in stages:
                stages[key] = MoEStage(shape, n_layer=1, layers={0: W.make_layer(shape, seed, layer)})
            fx, res = W.make_hidden(shape, seed, layer, tok)
            print(f"golden {name} seed {seed} token {tok}", flush=True)
            y, sel, w = stages[key].layer(0, fx, res)
            tag = f"{name}_s{seed}_l{layer}_t{tok}"
            assert np.array_equal(sel, gold[tag + "_sel"])
            assert np.allclose(w, gold[tag + "_w"], rtol=1e-6, atol=0)
            parity.assert_parity(y, gold[tag + "_y"], tag)
    finally:
        for st in stages.values():
            st.close()
