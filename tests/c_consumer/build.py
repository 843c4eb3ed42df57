"""Builds tests/c_consumer/consumer: a C++ program that includes include/*.h only
and links libhoard_moe.so (run from the test suite; found next to this file)."""
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
BIN = HERE / "consumer"


def build() -> Path:
    cmd = ["/opt/rocm/bin/hipcc", "-O2", "-std=c++17", "--offload-arch=gfx950", f"-I{ROOT / 'include'}",
           str(HERE / "consumer.cpp"), f"-L{ROOT / 'hoard_amd'}", "-lhoard_moe",
           "-Wl,-rpath,$ORIGIN/../../hoard_amd", "-o", str(BIN)]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode:
        raise RuntimeError(f"consumer build failed:\n{r.stdout}")
    return BIN


if __name__ == "__main__":
    print(build())
