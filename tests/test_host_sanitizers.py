"""libtsfa's host-only code (csrc/tsfa_plan.cpp: planners, validators,
workspace sizing, the host metadata builder) built with
-fsanitize=address,undefined and exercised two ways on the CPU: the
randomized invariant sweep of tests/sanitize/plan_sweep.cpp, and the
C-ABI tests (tests/test_capi.py) plus the host metadata tests
(tests/test_host_meta.py) loading the sanitized library."""

import os
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
CSRC = ROOT / "eagle3-tree-sparse-flashattn_amd" / "csrc"
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g", "-O1"]
GXX = shutil.which("g++")

pytestmark = pytest.mark.skipif(GXX is None, reason="needs g++")


def _sanitizer_failed(text: str) -> bool:
    return "runtime error:" in text or "ERROR: AddressSanitizer" in text or "ERROR: LeakSanitizer" in text


@pytest.fixture(scope="module")
def build_dir(tmp_path_factory):
    return tmp_path_factory.mktemp("asan")


def test_randomized_host_sweep_under_sanitizers(build_dir):
    exe = build_dir / "plan_sweep"
    cmd = [GXX, "-std=c++17", *SAN, f"-I{CSRC}", str(ROOT / "tests" / "sanitize" / "plan_sweep.cpp"),
           str(CSRC / "tsfa_plan.cpp"), "-o", str(exe)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300,
                         env={**os.environ, "ASAN_OPTIONS": "detect_leaks=1", "UBSAN_OPTIONS": "print_stacktrace=1"})
    out = res.stdout + res.stderr
    print(out[-2000:])
    assert res.returncode == 0 and not _sanitizer_failed(out), out[-4000:]
    assert "all invariants hold" in res.stdout


def test_capi_and_host_metadata_tests_on_the_sanitized_library(build_dir):
    lib = build_dir / "libtsfa_plan_asan.so"
    cmd = [GXX, "-std=c++17", *SAN, "-shared", "-fPIC", f"-I{CSRC}", str(CSRC / "tsfa_plan.cpp"), "-o", str(lib)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    libasan = subprocess.run([GXX, "-print-file-name=libasan.so"], capture_output=True, text=True).stdout.strip()
    assert Path(libasan).exists(), libasan
    env = {**os.environ, "LD_PRELOAD": libasan, "TSFA_LIB": str(lib), "TSFA_HOST_ONLY": "1",
           # the interpreter and torch are not instrumented: report errors in
           # the library under test, not leaks or allocator pairing elsewhere
           "ASAN_OPTIONS": "detect_leaks=0:alloc_dealloc_mismatch=0:detect_odr_violation=0"}
    res = subprocess.run([sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider", "-m", "not gpu",
                          str(ROOT / "tests" / "test_capi.py"), str(ROOT / "tests" / "test_host_meta.py")],
                         capture_output=True, text=True, timeout=600, env=env, cwd=str(ROOT))
    out = res.stdout + res.stderr
    print(out[-3000:])
    assert res.returncode == 0 and not _sanitizer_failed(out), out[-4000:]
    assert " passed" in res.stdout
