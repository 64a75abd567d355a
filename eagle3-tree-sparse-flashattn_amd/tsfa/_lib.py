"""ctypes binding of libtsfa.so (declarations: include/tsfa.h).

The library is loaded after ``import torch`` so that it binds to the HIP
runtime torch already loaded (one runtime per process; torch's stream handles
are then valid for libtsfa).  There is no fallback: if the library is missing
or a call fails, an exception is raised.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  (must precede the CDLL load, see module docstring)

LIB_PATH = Path(__file__).resolve().parent.parent / "libtsfa.so"

TSFA_OK = 0
TSFA_ERR_INVALID_ARGUMENT = 1
TSFA_ERR_UNSUPPORTED = 2
TSFA_ERR_WORKSPACE = 3
TSFA_ERR_LAUNCH = 4
TSFA_ERR_DEVICE = 5

TSFA_DTYPE_FP16 = 0
TSFA_DTYPE_BF16 = 1
TSFA_DTYPE_FP32 = 2

EXPORTS = (
    "tsfa_version",
    "tsfa_status_string",
    "tsfa_meta_check_args",
    "tsfa_meta_workspace_bytes",
    "tsfa_meta_build",
    "tsfa_pack_bits",
    "tsfa_meta_build_host",
    "tsfa_pack_bits_host",
    "tsfa_config_reload",
    "tsfa_fwd_plan_for_device",
    "tsfa_fwd_workspace_bytes_for_device",
    "tsfa_device_limits",
    "tsfa_fwd_check_args",
    "tsfa_fwd_workspace_bytes",
    "tsfa_fwd_workspace_bytes_for_dtype",
    "tsfa_fwd",
    "tsfa_fwd_lse",
    "tsfa_fwd_noalloc",
    "tsfa_tree_attention",
    "tsfa_tree_attention_workspace_bytes",
    "tsfa_bwd",
    "tsfa_bwd_workspace_bytes",
    "tsfa_fwd_paged",
    "tsfa_fwd_plan",
    "tsfa_fwd_set_kernel_mask",
)

_c_int, _c_i64, _c_size, _c_vp, _c_float = ctypes.c_int, ctypes.c_int64, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_float

_SIGNATURES = {
    "tsfa_version": (_c_int, []),
    "tsfa_status_string": (ctypes.c_char_p, [_c_int]),
    "tsfa_meta_check_args": (_c_int, [_c_int] * 4),
    "tsfa_meta_workspace_bytes": (_c_size, [_c_int] * 4),
    "tsfa_meta_build": (_c_int, [_c_vp, _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_int,
                                 _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_size, _c_vp]),
    "tsfa_pack_bits": (_c_int, [_c_vp, _c_i64, _c_vp, _c_vp]),
    "tsfa_meta_build_host": (_c_int, [_c_vp, _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_int,
                                      _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp]),
    "tsfa_pack_bits_host": (_c_int, [_c_vp, _c_i64, _c_vp]),
    "tsfa_config_reload": (_c_int, []),
    "tsfa_fwd_plan_for_device": (_c_int, [_c_int] * 10 + [ctypes.POINTER(ctypes.c_int32)]),
    "tsfa_fwd_workspace_bytes_for_device": (_c_size, [_c_int] * 9),
    "tsfa_device_limits": (_c_int, [ctypes.POINTER(ctypes.c_int32)]),
    "tsfa_fwd_check_args": (_c_int, [_c_int] * 13),
    "tsfa_fwd_workspace_bytes": (_c_size, [_c_int] * 7),
    "tsfa_fwd_workspace_bytes_for_dtype": (_c_size, [_c_int] * 8),
    "tsfa_fwd": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp,
                          ctypes.POINTER(_c_i64), ctypes.POINTER(_c_i64), _c_float]
                 + [_c_int] * 13 + [_c_vp, _c_size, _c_vp]),
    "tsfa_fwd_lse": (_c_int, [_c_vp] * 10 + [ctypes.POINTER(_c_i64), ctypes.POINTER(_c_i64), _c_float]
                     + [_c_int] * 13 + [_c_vp, _c_size, _c_vp]),
    "tsfa_fwd_noalloc": (_c_int, [_c_vp] * 9 + [ctypes.POINTER(_c_i64), ctypes.POINTER(_c_i64), _c_float]
                         + [_c_int] * 13 + [_c_vp]),
    "tsfa_tree_attention": (_c_int, [_c_vp] * 5 + [_c_i64, _c_i64, _c_int, ctypes.POINTER(_c_i64), _c_float]
                            + [_c_int] * 9 + [_c_vp, _c_size, _c_vp]),
    "tsfa_tree_attention_workspace_bytes": (_c_size, [_c_int] * 10),
    "tsfa_bwd_workspace_bytes": (_c_size, [_c_int] * 10),
    "tsfa_bwd": (_c_int, [_c_vp] * 14 + [ctypes.POINTER(_c_i64), ctypes.POINTER(_c_i64), _c_float]
                 + [_c_int] * 13 + [_c_vp, _c_size, _c_vp]),
    "tsfa_fwd_paged": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_int, _c_int, _c_vp, _c_vp,
                                _c_vp, _c_vp, _c_vp, _c_vp, _c_vp]
                       + [ctypes.POINTER(_c_i64)] * 4 + [_c_float] + [_c_int] * 13 + [_c_vp, _c_size, _c_vp]),
    "tsfa_fwd_plan": (_c_int, [_c_int] * 7 + [ctypes.POINTER(ctypes.c_int32)]),
    "tsfa_fwd_set_kernel_mask": (_c_int, [_c_int]),
}

_lib = None


class TsfaError(RuntimeError):
    def __init__(self, fn: str, status: int):
        self.status = status
        super().__init__(f"{fn} failed: {status_string(status)} (status {status})")


def load() -> ctypes.CDLL:
    """Load libtsfa.so (built by ``tsfa.build``); raise if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    path = Path(os.environ.get("TSFA_LIB", LIB_PATH))
    if not path.exists():
        raise RuntimeError(
            f"libtsfa.so not found at {path}: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
            "(the HIP path has no CPU fallback)"
        )
    lib = ctypes.CDLL(str(path))
    # TSFA_HOST_ONLY=1: a build of the host-only part (tsfa_plan.cpp), as
    # the sanitizer test loads it; its entry points are a subset
    host_only = os.environ.get("TSFA_HOST_ONLY") == "1"
    for name, (res, args) in _SIGNATURES.items():
        if host_only and not hasattr(lib, name):
            continue
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def status_string(status: int) -> str:
    try:
        return load().tsfa_status_string(status).decode()
    except Exception:  # pragma: no cover
        return f"status {status}"


def check(fn: str, status: int) -> None:
    """Map a tsfa status to the reference's exception types."""
    if status == TSFA_OK:
        return
    if status == TSFA_ERR_INVALID_ARGUMENT:
        raise ValueError(f"{fn}: {status_string(status)}")
    if status == TSFA_ERR_UNSUPPORTED:
        raise NotImplementedError(f"{fn}: {status_string(status)}")
    raise TsfaError(fn, status)


def ptr(t) -> int:
    return 0 if t is None else t.data_ptr()


# torch's raw current-stream accessor (an int, no Stream object: ~0.2 us
# against ~1.8 us for current_stream(dev).cuda_stream per eager call)
_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device) -> int:
    """The hipStream_t of torch's current stream on `device` (the capture
    stream under graph capture)."""
    if _RAW_STREAM is not None:
        idx = device.index if isinstance(device, torch.device) else device
        return _RAW_STREAM(torch.cuda.current_device() if idx is None else idx)
    return torch.cuda.current_stream(device).cuda_stream


def i64_array(values):
    arr = (ctypes.c_int64 * len(values))(*[int(v) for v in values])
    return arr


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float16:
        return TSFA_DTYPE_FP16
    if dtype == torch.bfloat16:
        return TSFA_DTYPE_BF16
    if dtype == torch.float32:
        return TSFA_DTYPE_FP32
    raise NotImplementedError(f"dtype {dtype} is not supported by the HIP kernels (fp16/bf16/fp32)")


def fwd_plan(batch, num_heads, num_kv_heads, q_len, kv_len, prefix_len, head_dim) -> dict:
    out = (ctypes.c_int32 * 6)()
    check("tsfa_fwd_plan", load().tsfa_fwd_plan(batch, num_heads, num_kv_heads, q_len, kv_len, prefix_len,
                                                 head_dim, out))
    keys = ("prefix_splits", "units_per_split", "rows_per_chunk", "row_chunks", "workgroups", "ring_stages")
    plan = dict(zip(keys, list(out)))
    # the partial slots per row chunk and the folded tree, planned for this device
    lim = (ctypes.c_int32 * 2)()
    check("tsfa_device_limits", load().tsfa_device_limits(lim))
    out8 = (ctypes.c_int32 * 8)()
    check("tsfa_fwd_plan_for_device", load().tsfa_fwd_plan_for_device(
        lim[0], lim[1], batch, num_heads, num_kv_heads, q_len, kv_len, prefix_len, head_dim, 0, out8))
    plan["slots"] = int(out8[6])
    plan["fold_tree"] = int(out8[7])
    return plan
