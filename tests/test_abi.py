"""The product library loads on a CPU-only host, exports every symbol the
public headers declare, and does not link the oracle (no compute calls)."""
import re
import subprocess
from pathlib import Path

import hoard_amd

ROOT = Path(__file__).resolve().parent.parent


def declared_symbols():
    names = set()
    for h in sorted((ROOT / "include").glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"^[A-Za-z_][\w \*]*?\b(hoard_\w+)\s*\(", text, flags=re.M))
    return names


def test_headers_declare_the_abi():
    names = declared_symbols()
    assert {"hoard_moe_create", "hoard_moe_route", "hoard_moe_ffn_combine", "hoard_moe_decode",
            "hoard_last_error", "hoard_synth_fill_experts"} <= names


def test_library_exports_every_declared_symbol(hlib):
    missing = [n for n in sorted(declared_symbols()) if not hasattr(hlib, n)]
    assert not missing, missing


def test_python_bindings_cover_the_headers():
    assert declared_symbols() == set(hoard_amd.ABI)


def test_product_does_not_link_the_oracle():
    out = subprocess.run(["nm", "-D", str(hoard_amd.LIB_PATH)], capture_output=True, text=True).stdout
    assert "orc_" not in out
    deps = subprocess.run(["ldd", str(hoard_amd.LIB_PATH)], capture_output=True, text=True).stdout
    assert "moe_oracle" not in deps


def test_missing_library_raises(tmp_path):
    import pytest
    with pytest.raises(hoard_amd.HoardError):
        hoard_amd.load_library(tmp_path / "absent.so")
