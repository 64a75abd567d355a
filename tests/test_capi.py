"""The C-ABI library loads, exports every declared symbol, and validates
arguments on the host exactly as the reference rejects them (no GPU work)."""

import ctypes
import os
import re
from pathlib import Path

import pytest

from tsfa import _lib

HEADER = Path(__file__).resolve().parent.parent / "include" / "tsfa.h"

# TSFA_HOST_ONLY=1: the library under test is the host-only part alone (the
# sanitizer build of csrc/tsfa_plan.cpp); entry points of the HIP sources
# are absent there
needs_full_library = pytest.mark.skipif(os.environ.get("TSFA_HOST_ONLY") == "1",
                                        reason="entry point of the HIP sources (host-only library)")


def _declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tsfa_[a-z0-9_]+)\s*\(", text)))


@needs_full_library
def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = _declared()
    assert set(declared) == set(_lib.EXPORTS)
    for name in declared:
        assert hasattr(lib, name), name


def test_version_and_status_strings():
    lib = _lib.load()
    assert lib.tsfa_version() >= 1
    assert lib.tsfa_status_string(0) == b"ok"
    assert b"invalid" in lib.tsfa_status_string(1)


def test_meta_check_args():
    lib = _lib.load()
    assert lib.tsfa_meta_check_args(1, 64, 16, 64) == _lib.TSFA_OK
    assert lib.tsfa_meta_check_args(1, 0, 16, 64) == _lib.TSFA_OK        # empty mask is valid
    assert lib.tsfa_meta_check_args(1, 64, 0, 64) == _lib.TSFA_ERR_INVALID_ARGUMENT   # :87-88
    assert lib.tsfa_meta_check_args(1, 64, 16, -2) == _lib.TSFA_ERR_INVALID_ARGUMENT
    assert lib.tsfa_meta_workspace_bytes(2, 64, 16, 64) > 0


FWD_OK = dict(batch=1, num_heads=32, num_kv_heads=8, q_len=64, kv_len=4160, prefix_len=4096, n_q_blocks=4,
              n_tree_blocks=1, gqa_group_size=4, block_m=16, block_n=64, head_dim=128, dtype=_lib.TSFA_DTYPE_BF16)


def _fwd_check(**kw):
    args = dict(FWD_OK)
    args.update(kw)
    return _lib.load().tsfa_fwd_check_args(*args.values())


def test_fwd_check_args_ok():
    assert _fwd_check() == _lib.TSFA_OK


@pytest.mark.parametrize("kw,status", [
    (dict(block_m=0), _lib.TSFA_ERR_INVALID_ARGUMENT),
    (dict(prefix_len=-1), _lib.TSFA_ERR_INVALID_ARGUMENT),
    (dict(kv_len=100, prefix_len=200), _lib.TSFA_ERR_INVALID_ARGUMENT),   # eagle_tree_sparse_bridge.py:91-93
    (dict(gqa_group_size=3), _lib.TSFA_ERR_INVALID_ARGUMENT),
    (dict(n_q_blocks=5), _lib.TSFA_ERR_INVALID_ARGUMENT),
    (dict(head_dim=96), _lib.TSFA_ERR_UNSUPPORTED),
    (dict(block_n=24, n_tree_blocks=3), _lib.TSFA_ERR_UNSUPPORTED),
    (dict(dtype=7), _lib.TSFA_ERR_UNSUPPORTED),
])
def test_fwd_check_args_rejects(kw, status):
    assert _fwd_check(**kw) == status


@needs_full_library
def test_null_pointers_rejected_before_device_work():
    lib = _lib.load()
    strides = (ctypes.c_int64 * 16)(*([1] * 16))
    ms = (ctypes.c_int64 * 5)()
    st = lib.tsfa_fwd(None, None, None, None, None, None, None, None, None, ms, strides, ctypes.c_float(0.1),
                      *list(FWD_OK.values()), None, 0, None)
    assert st == _lib.TSFA_ERR_INVALID_ARGUMENT
    assert lib.tsfa_pack_bits(None, -1, None, None) == _lib.TSFA_ERR_INVALID_ARGUMENT


@needs_full_library
def test_kernel_mask_hook_validates_and_restores(monkeypatch):
    lib = _lib.load()
    for bad in (0, 4, -1):
        assert lib.tsfa_fwd_set_kernel_mask(bad) == _lib.TSFA_ERR_INVALID_ARGUMENT
    # locked unless the process opts in to measurement hooks
    monkeypatch.delenv("TSFA_BENCH_HOOKS", raising=False)
    for locked in (1, 2):
        assert lib.tsfa_fwd_set_kernel_mask(locked) == _lib.TSFA_ERR_UNSUPPORTED
    assert lib.tsfa_fwd_set_kernel_mask(3) == _lib.TSFA_OK
    monkeypatch.setenv("TSFA_BENCH_HOOKS", "1")
    for ok in (1, 2, 3):
        assert lib.tsfa_fwd_set_kernel_mask(ok) == _lib.TSFA_OK
    assert lib.tsfa_fwd_set_kernel_mask(3) == _lib.TSFA_OK  # back to computing O


def test_tree_limits_reported_unsupported():
    # tree keys beyond 32768 (1024 units of 32) and block-state tables larger
    # than the LDS ring are refused, not silently mis-computed
    assert _fwd_check(q_len=40000, kv_len=44096, n_q_blocks=2500, n_tree_blocks=625) == _lib.TSFA_ERR_UNSUPPORTED
    # a 256-row chunk of G = 4 spans 66 q-blocks of BM = 1: 66 x 512 tree blocks x 4 B > 128 KiB
    assert _fwd_check(q_len=8192, kv_len=12288, block_m=1, n_q_blocks=8192, block_n=16,
                      n_tree_blocks=512) == _lib.TSFA_ERR_UNSUPPORTED
    assert _fwd_check(q_len=8192, kv_len=12288, block_m=1, n_q_blocks=8192, block_n=32,
                      n_tree_blocks=256) == _lib.TSFA_OK


def _paged_call(page_size=16, n_pages=8, n_indices=16, pt_stride=4, indptr=None, cache=0x1000, **kw):
    """tsfa_fwd_paged with fake (aligned, never dereferenced) device pointers:
    every case here is refused on the host before any device work."""
    args = dict(FWD_OK)
    args.update(kw)
    fake = 0x2000
    ms = (ctypes.c_int64 * 5)()
    qs = (ctypes.c_int64 * 4)(4096 * 128 * 32, 64 * 128, 128, 1)
    cs = (ctypes.c_int64 * 5)(2 * page_size * 8 * 128, page_size * 8 * 128, 8 * 128, 128, 1)
    return _lib.load().tsfa_fwd_paged(fake, cache, indptr, fake, n_indices, pt_stride, n_pages, page_size, fake,
                                      None, fake, fake, fake, fake, fake, ms, qs, cs, qs, ctypes.c_float(0.1),
                                      *args.values(), fake, 1 << 30, None)


@needs_full_library
@pytest.mark.parametrize("kw,status", [
    (dict(page_size=8), _lib.TSFA_ERR_UNSUPPORTED),          # a wave's 16-key share would span 3 pages
    (dict(page_size=48), _lib.TSFA_ERR_UNSUPPORTED),         # not a power of two
    (dict(cache=None), _lib.TSFA_ERR_INVALID_ARGUMENT),
    (dict(n_pages=0), _lib.TSFA_ERR_INVALID_ARGUMENT),
    (dict(pt_stride=-1), _lib.TSFA_ERR_INVALID_ARGUMENT),
    # dense table: sequence 0 needs ceil(4160 / 16) = 260 ids, 16 are given
    (dict(), _lib.TSFA_ERR_INVALID_ARGUMENT),
    (dict(head_dim=96), _lib.TSFA_ERR_UNSUPPORTED),
])
def test_fwd_paged_rejects_on_host(kw, status):
    assert _paged_call(**kw) == status


@needs_full_library
def test_tree_attention_rejects_on_the_host():
    # kv_len < q_len is the reference's ValueError (eagle_tree_sparse_bridge.py:91-93),
    # refused before any device query; a null mask or strides likewise
    lib = _lib.load()
    strides = (ctypes.c_int64 * 16)(*([1] * 16))
    args = dict(batch=1, num_heads=8, num_kv_heads=2, q_len=40, kv_len=30, block_m=16, block_n=32, head_dim=128,
                dtype=_lib.TSFA_DTYPE_BF16)
    st = lib.tsfa_tree_attention(None, None, None, None, None, 0, 40, 1, strides, ctypes.c_float(0.1),
                                 *args.values(), None, 0, None)
    assert st == _lib.TSFA_ERR_INVALID_ARGUMENT
    assert lib.tsfa_tree_attention_workspace_bytes(1, 8, 2, 40, 30, 1, 16, 32, 128, 1) == 0
    assert lib.tsfa_tree_attention_workspace_bytes(2, 8, 2, 40, 100, 3, 16, 32, 128, 1) == 0  # n_masks not 1 or B
