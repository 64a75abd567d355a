"""Register budgets of the built kernels, read from the code object's metadata.

A kernel change can move scalars out of SGPRs into VGPR lanes (the compiler's
SGPR spills, reloaded with v_readlane) without any test seeing it: the results
stay bit-exact and only the time grows.  Code compiled into an instance that
never runs it, an equivalent rewrite of a ring-stage address, and one loop
shared by two paths each did so here (2 to 120 spilled SGPRs, 3 to 11 % per
call).  These checks read the metadata of the built device code (no GPU
needed) and hold the split-KV instances of the shipped paths to ceilings a few
SGPRs above their current counts, and every kernel to no scratch at all.
"""

import os
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
BUILD = ROOT / "eagle3-tree-sparse-flashattn_amd" / "_build"
LLVM = Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / "llvm" / "bin"
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"

# split_kernel<T, 128, S, PAGED, C32, FAST> -> most SGPR spills allowed.
# FAST: 0 checked steps, 1/2 unchecked (plain / non-temporal loads), +4 the
# one-slot kernel that writes O, +8 the paged page-id table.
SPLIT_CEILINGS = {
    # contiguous: 8B decode (2, FAST 2), batched decode (2, 6), wide tree
    # (1, 1), 70B (1, 5), and the checked steps
    (2, False, False, 2): 19, (2, False, False, 1): 19, (2, False, False, 6): 17, (2, False, False, 5): 17,
    (2, False, False, 0): 42, (1, False, False, 1): 17, (1, False, False, 5): 17, (1, False, False, 0): 55,
    # paged, 32-bit offsets (two streams) and 64-bit (two streams, one stream)
    (2, True, True, 9): 35, (2, True, True, 13): 36, (2, True, True, 1): 43, (2, True, True, 5): 39,
    (2, True, True, 0): 46, (2, True, False, 13): 34, (2, True, False, 1): 42, (2, True, False, 5): 38,
    (2, True, False, 0): 64, (1, True, False, 9): 43, (1, True, False, 13): 38, (1, True, False, 1): 56,
    (1, True, False, 5): 33, (1, True, False, 0): 33,
}
SPLIT_RE = re.compile(r"_ZN4tsfa3fwd12split_kernelI(DF16b|DF16_)Li128ELi(\d)ELb(\d)ELb(\d)ELi(\d+)EEEvNS0_9SplitArgsE")


def _kernels(obj: Path):
    """name -> {metadata key: int} for every kernel of the object's gfx950 code."""
    tools = [LLVM / t for t in ("llvm-objcopy", "clang-offload-bundler", "llvm-readelf")]
    if not all(t.exists() for t in tools):
        pytest.skip("ROCm LLVM tools not found")
    if not obj.exists():
        pytest.skip(f"{obj.name} not built (run __graft_entry__.build())")
    tmp = Path(os.environ.get("TMPDIR", "/tmp")) / f"tsfa_res_{os.getpid()}_{obj.stem}"
    tmp.mkdir(parents=True, exist_ok=True)
    try:
        fb, co = tmp / "fatbin", tmp / "device.co"
        subprocess.run([str(tools[0]), f"--dump-section=.hip_fatbin={fb}", str(obj), str(tmp / "host.o")],
                       check=True, capture_output=True)
        subprocess.run([str(tools[1]), "--unbundle", "--type=o", f"--targets={TARGET}", f"--input={fb}",
                        f"--output={co}"], check=True, capture_output=True)
        notes = subprocess.run([str(tools[2]), "--notes", str(co)], check=True, capture_output=True,
                               text=True).stdout
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    out = {}
    for blk in notes.split("  - .")[1:]:
        name = re.search(r"\.name:\s+(\S+)", blk)
        if not name:
            continue
        vals = {k: int(v) for k, v in re.findall(r"\.(sgpr_spill_count|vgpr_spill_count|"
                                                 r"private_segment_fixed_size|vgpr_count):\s+(\d+)", blk)}
        out[name.group(1)] = vals
    return out


@pytest.mark.parametrize("src", ["tsfa_fwd", "tsfa_bwd", "tsfa_meta"])
def test_no_scratch(src):
    kernels = _kernels(BUILD / f"{src}.o")
    assert kernels, f"no kernels found in {src}.o"
    for name, k in kernels.items():
        assert k.get("private_segment_fixed_size", 0) == 0, f"{name} uses scratch"
        assert k.get("vgpr_spill_count", 0) == 0, f"{name} spills VGPRs"


def test_split_kernel_sgpr_spill_ceilings():
    kernels = _kernels(BUILD / "tsfa_fwd.o")
    seen = set()
    over = []
    for name, k in kernels.items():
        m = SPLIT_RE.fullmatch(name)
        if not m:
            continue
        key = (int(m.group(2)), m.group(3) == "1", m.group(4) == "1", int(m.group(5)))
        if key not in SPLIT_CEILINGS:
            continue
        seen.add(key)
        if k["sgpr_spill_count"] > SPLIT_CEILINGS[key]:
            over.append(f"{name}: {k['sgpr_spill_count']} spilled SGPRs > {SPLIT_CEILINGS[key]}")
    assert seen == set(SPLIT_CEILINGS), f"instances missing: {sorted(set(SPLIT_CEILINGS) - seen)}"
    assert not over, "\n".join(over)
