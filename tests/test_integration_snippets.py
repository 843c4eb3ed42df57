"""Every ```cpp snippet of INTEGRATION.md compiles against include/*.h.

Each snippet becomes the body of a function of its own, after a preamble that
declares the engine-side names the snippets use (hparams, device pointers,
streams, die()); #include lines move to the top.  g++ checks the syntax and
every call's argument count and types against the public headers.
"""
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent

PREAMBLE = """
#include <cstdint>
#include <vector>
#include "hoard_gguf.h"
#include "hoard_moe.h"
#include "hoard_store.h"
[[noreturn]] void die(const char *msg);
extern int n_embd, n_expert, n_used, n_ff_exp, n_layer, wnorm, il, M, m, n_use, ioqd, ram_cap;
extern const float *router_f32[];
struct Hparams { int gtype[64], utype[64], dtype[64]; uint64_t goff[64], uoff[64], doff[64]; };
extern Hparams H;
const void *host_bytes(uint64_t off);
extern const char *path;
extern hoard_moe *moe;
extern hoard_gguf *g;
extern hoard_moe_cfg cfg;
extern float *fx_dev, *res_dev, *x_dev, *out_dev, *w_dev, *wgt_dev, *ffninp_dev;
extern int32_t *sel_dev, *slots_dev;
extern int32_t sel[16], ids[256];
extern void *stream, *copy_stream;
extern float eps;
"""


def snippets():
    text = (ROOT / "INTEGRATION.md").read_text()
    return re.findall(r"```cpp\n(.*?)```", text, flags=re.S)


def test_snippets_exist():
    assert len(snippets()) >= 8


@pytest.mark.parametrize("i", range(len(snippets())))
def test_snippet_compiles(tmp_path, i):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("no g++")
    body = snippets()[i]
    includes = [l for l in body.splitlines() if l.startswith("#include")]
    code = "\n".join(l for l in body.splitlines() if not l.startswith("#include"))
    src = tmp_path / f"snippet{i}.cpp"
    src.write_text("\n".join(includes) + PREAMBLE + f"\nvoid snippet_{i}() {{\n{code}\n}}\n")
    r = subprocess.run([gxx, "-std=c++17", "-fsyntax-only", "-Wall", "-Wno-unused-variable",
                        "-Wno-unused-but-set-variable", f"-I{ROOT / 'include'}", str(src)],
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    assert r.returncode == 0, f"INTEGRATION.md snippet {i} does not compile:\n{body}\n{r.stdout}"
