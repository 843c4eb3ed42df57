"""The storage tier's reader pool (hoard_amd/csrc/store.cpp) under ThreadSanitizer
and AddressSanitizer + UndefinedBehaviorSanitizer.

The reference's DirectIO pool (src/run_qwen35.cpp:99-138) has no such check; the
pool here spawns its readers once and hands them batches through a generation
counter and two condition variables, which is what TSAN watches.  The driver
(tests/sanitize/store_race.cpp) fetches thousands of random batches through a
6-expert RAM tier with 8 readers and compares every expert's bytes with the
file.  A racy canary program must be flagged, so a sanitizer that silently does
nothing in this environment fails the test instead of passing it.
"""
import os
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
GXX = shutil.which("g++")
HIP_INC = Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / "include"

pytestmark = pytest.mark.skipif(GXX is None or not (HIP_INC / "hip" / "hip_runtime.h").exists(),
                                reason="needs g++ and the HIP headers")

CANARY = r"""
#include <thread>
int shared_value = 0;
int main() {
    std::thread t([] { for (int i = 0; i < 100000; ++i) ++shared_value; });
    for (int i = 0; i < 100000; ++i) ++shared_value;
    t.join();
    return 0;
}
"""


def _build(out: Path, sanitize: str, sources):
    cmd = [GXX, "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", f"-fsanitize={sanitize}",
           "-D__HIP_PLATFORM_AMD__", f"-I{HIP_INC}", f"-I{ROOT / 'include'}", f"-I{ROOT / 'hoard_amd' / 'csrc'}",
           *map(str, sources), "-o", str(out), "-lpthread"]
    subprocess.run(cmd, check=True, capture_output=True, text=True)


def _run(exe: Path, *args, env_extra=None):
    env = dict(os.environ)
    env.update(env_extra or {})
    return subprocess.run([str(exe), *map(str, args)], capture_output=True, text=True, timeout=300, env=env)


@pytest.mark.parametrize("sanitize,opts", [
    ("thread", {"TSAN_OPTIONS": "halt_on_error=1 exitcode=66"}),
    ("address,undefined", {"ASAN_OPTIONS": "detect_leaks=1 exitcode=66",
                           "UBSAN_OPTIONS": "halt_on_error=1 print_stacktrace=1 exitcode=66"}),
], ids=["tsan", "asan_ubsan"])
def test_reader_pool_clean_under_sanitizer(tmp_path, sanitize, opts):
    exe = tmp_path / "store_race"
    _build(exe, sanitize, [ROOT / "hoard_amd" / "csrc" / "store.cpp", ROOT / "tests" / "sanitize" / "store_race.cpp"])
    r = _run(exe, tmp_path / "experts.bin", 2000, 8, env_extra=opts)
    report = r.stdout + r.stderr
    assert r.returncode == 0, report[-4000:]
    assert "WARNING: ThreadSanitizer" not in report and "ERROR: AddressSanitizer" not in report, report[-4000:]
    assert "runtime error:" not in report, report[-4000:]
    assert report.startswith("bad 0 "), report[-2000:]


def test_thread_sanitizer_flags_a_race(tmp_path):
    """The canary: an unsynchronised counter shared by two threads is reported."""
    src = tmp_path / "canary.cpp"
    src.write_text(CANARY)
    exe = tmp_path / "canary"
    _build(exe, "thread", [src])
    r = _run(exe, env_extra={"TSAN_OPTIONS": "exitcode=66"})
    assert r.returncode == 66 and "data race" in r.stderr, (r.returncode, r.stderr[-2000:])
