"""Build libtsfa.so for gfx950 in-tree.

Each ``csrc/*.hip`` file is compiled with ``hipcc -c``, each host-only
``csrc/*.cpp`` file with the system C++ compiler, and the objects are linked
with the system C++ compiler against the HIP runtime that PyTorch
loads (torch/lib/libamdhip64.so when torch is importable), so the library and
torch share one HIP runtime in the process and torch's stream handles are
valid for libtsfa.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent.parent
CSRC = PKG_DIR / "csrc"
BUILD_DIR = PKG_DIR / "_build"
LIB_PATH = PKG_DIR / "libtsfa.so"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-result",
    # no packed-fp32 instructions anywhere in this library
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hip_runtime_dir() -> Path:
    """Directory of the libamdhip64.so the host process uses (torch's, if present)."""
    env = os.environ.get("TSFA_HIP_RUNTIME_DIR")
    if env:
        return Path(env)
    try:
        import torch  # noqa: F401

        tdir = Path(torch.__file__).resolve().parent / "lib"
        if (tdir / "libamdhip64.so").exists():
            return tdir
    except Exception:  # pragma: no cover - torch absent
        pass
    return ROCM / "lib"


CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra", "-Wno-unused-parameter"]


def _compile(src: Path, obj: Path) -> None:
    if src.suffix == ".cpp":
        cmd = [shutil.which("g++") or "c++", *CXX_FLAGS, "-c", str(src), "-o", str(obj)]
    else:
        cmd = [str(ROCM / "bin" / "hipcc"), *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(
        line for line in (res.stdout + res.stderr).splitlines() if "packed-fp32-ops" not in line
    )
    if res.returncode != 0:
        raise RuntimeError(f"compile failed for {src.name}:\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def build(verbose: bool = True) -> Path:
    """Compile every csrc/*.hip and csrc/*.cpp and link libtsfa.so (always rebuilds)."""
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    objs = [BUILD_DIR / (s.stem + ".o") for s in sources]
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(sources))) as ex:
        list(ex.map(_compile, sources, objs))
    rt = hip_runtime_dir()
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cxx = shutil.which("g++") or "c++"
    cmd = [cxx, "-shared", "-o", str(tmp), *map(str, objs), f"-L{rt}", "-l:libamdhip64.so",
           f"-Wl,-rpath,{rt}", "-Wl,--no-undefined", "-Wl,--no-as-needed"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} (HIP runtime {rt})")
    return LIB_PATH


if __name__ == "__main__":
    build()
