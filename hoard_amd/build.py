"""Build recipe for libhoard_moe.so (gfx950) -- plain hipcc, in-tree.

    python -m hoard_amd.build        # or hoard_amd.build.build()

Compiles every C++/HIP source under hoard_amd/csrc into one shared library
next to this file.  Device code is built with contraction off (each fp32
operation rounds where written, which the bit-exact parity tests rely on) and
without packed-fp32 instructions.
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
INCLUDE = HERE.parent / "include"
LIB = HERE / "libhoard_moe.so"
ARCH = os.environ.get("HOARD_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-command-line-argument",
    f"-I{INCLUDE}", f"-I{CSRC}",
]


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))


def build(verbose: bool = False, jobs: int = 8) -> Path:
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    objdir = HERE / "_build"
    objdir.mkdir(exist_ok=True)
    procs = []
    objs = []
    for src in sources():
        obj = objdir / (src.name + ".o")
        objs.append(obj)
        cmd = [hipcc, *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
        if src.suffix == ".hip":
            cmd[1:1] = ["-x", "hip"]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
        if len(procs) >= jobs:
            _drain(procs)
    _drain(procs)
    tmp = LIB.with_suffix(".so.tmp")
    link = [hipcc, "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(link), flush=True)
    r = subprocess.run(link, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode:
        raise RuntimeError(f"link failed:\n{r.stdout}")
    os.replace(tmp, LIB)
    return LIB


def _drain(procs):
    errs = []
    for src, p in procs:
        out, _ = p.communicate()
        if p.returncode:
            errs.append(f"{src.name}:\n{out}")
        elif out.strip() and "warning" in out and "packed-fp32-ops" not in out:
            print(out, file=sys.stderr)
    procs.clear()
    if errs:
        raise RuntimeError("hipcc failed:\n" + "\n".join(errs))


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
