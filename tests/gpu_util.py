"""Helpers shared by the GPU parity tests (oracle comparison, tolerances)."""

from __future__ import annotations

import numpy as np
import torch

from oracle import meta_oracle as mo
from oracle.attn_oracle import dense_mask_attention

# max_abs_err bars against the fp32 oracle (the named workloads use these alone).
TOL = {torch.bfloat16: 8e-3, torch.float16: 2e-3, torch.float32: 1e-4}
# fp32 inputs (fp32 MFMA, P not rounded): the stated bars cover 16-bit
# inputs only; fp32 is held to 1e-4, well inside what the reference's fp32
# tl.dot (TF32 by default on its own hardware, tree_sparse_flashattn.py:269)
# could meet.
# Edge cases with few visible keys have |O| up to ~4, where rounding O once to
# the output dtype already costs up to half an ulp of O: 2^-7 = 7.8e-3 at |O|
# in [2, 4) for bf16, so no bf16-output kernel can meet 8e-3 absolute there
# once the reference's own rounding (P to the input dtype before P.V,
# tree_sparse_flashattn.py:278) adds its share.  Those tests allow the
# storage roundings of the call beyond the bar: |got - ref| <= TOL + n *
# ulp(got) / 2, ulp in the output dtype (MANT significand bits), n = 1 when
# the split kernel writes O (a one-slot plan) and n = 2 when the combine
# merges split-KV partials stored in the input dtype (one rounding of the
# partial, one of O; the reference has no partials).  Measured on the GPU
# suite's worst case (P = 1, G = 4, bf16, |O| up to 3.9): the reference's own
# P rounding moves O by up to 4.4e-3 from the fp32 oracle; the kernel is
# 1.34e-2 off with one slot (0.69 half-ulps beyond TOL) and 1.37e-2 with two
# (0.72 to 1.05).  Every such comparison prints its max_abs_err and how many
# half-ulps of |got| it used beyond TOL.
MANT = {torch.bfloat16: 8, torch.float16: 11, torch.float32: 24}


def storage_roundings(q, k, prefix_len) -> int:
    """Roundings of O to its dtype in one forward call of this shape: 1 when
    the plan has one slot (the kernel writes O, or a one-slot merge returns
    the partial), else 2 (partial in the input dtype, then O).  fp32 inputs:
    1 (fp32 partials).  The plan is read under the current TSFA_* switches."""
    from tsfa import _lib

    b, hq, t, d = q.shape
    if q.dtype == torch.float32:
        return 1
    if d > 128:
        return 1 if generic_slots(q, k, prefix_len) == 1 else 2
    width = 64 if d <= 64 else 128  # narrower head dims run zero-padded
    plan = _lib.fwd_plan(b, hq, k.shape[1], t, k.shape[2], prefix_len, width)
    return 1 if plan["slots"] == 1 else 2


def generic_slots(q, k, prefix_len) -> int:
    """Key splits of the generic kernel's plan for this 16-bit shape, read
    back from the library's workspace size (partials of rows x slots x D in
    the input dtype plus fp32 (m, l), each 256-byte aligned)."""
    from tsfa import _lib

    b, hq, t, d = q.shape
    rows = b * hq * t
    ws = int(_lib.load().tsfa_fwd_workspace_bytes_for_dtype(b, hq, k.shape[1], t, k.shape[2], prefix_len, d,
                                                            _lib.dtype_code(q.dtype)))

    def a256(x):
        return (x + 255) // 256 * 256

    for ns in range(1, (k.shape[2] + 31) // 32 + 1):
        if a256(rows * ns * d * 2) + a256(rows * ns * 8) == ws:
            return ns
    raise AssertionError(f"no slot count gives a workspace of {ws} bytes")


def half_ulp(x: torch.Tensor, dtype) -> torch.Tensor:
    """Half an ulp of each element of x (values of `dtype` held as fp32), in `dtype`."""
    _, e = torch.frexp(x.nan_to_num(0.0))  # x = m * 2^e, 0.5 <= |m| < 1
    return torch.where(x == 0, torch.zeros_like(x), torch.ldexp(torch.ones_like(x), e - MANT[dtype] - 1))


def assert_meta_equal(meta, ref: mo.OracleMetadata):
    """Bit-exact comparison of a TreeSparseMetadata with the oracle's record."""
    for field, dtype in (("row_ptr", torch.int32), ("col_idx", torch.int32), ("blk_type", torch.int8),
                         ("mixed_mask_payload", torch.int32), ("mixed_mask_offset", torch.int32)):
        got = getattr(meta, field)
        assert got.dtype == dtype, (field, got.dtype)
        exp = getattr(ref, field)
        np.testing.assert_array_equal(got.cpu().numpy(), exp, err_msg=field)
        assert tuple(got.shape) == exp.shape, (field, tuple(got.shape), exp.shape)
    for field in ("n_q_blocks", "n_tree_blocks", "block_m", "block_n", "prefix_len"):
        assert getattr(meta, field) == getattr(ref, field), field


def oracle_out(q, k, v, mask, prefix_len, heads=None, head_chunk=8):
    """fp32 oracle output; `heads` restricts it to a subset of query heads."""
    if heads is None:
        return dense_mask_attention(q, k, v, mask, prefix_len, head_chunk=head_chunk)
    group = q.shape[1] // k.shape[1]
    outs = []
    for h in heads:
        kv = h // group
        outs.append(dense_mask_attention(q[:, h:h + 1], k[:, kv:kv + 1], v[:, kv:kv + 1], mask, prefix_len))
    return torch.cat(outs, dim=1)


def assert_close_to_oracle(out, ref, dtype, heads=None, atol=None, half_ulps=0):
    """max |out - ref| <= TOL[dtype] (+ half_ulps halves of an ulp of out in
    `dtype`: the storage roundings of the call); NaN exactly where ref is NaN."""
    got = out.float().cpu()
    if heads is not None:
        got = got[:, list(heads)]
    tol = TOL[dtype] if atol is None else atol
    nan_got, nan_ref = torch.isnan(got), torch.isnan(ref)
    assert torch.equal(nan_got, nan_ref), f"NaN pattern differs: got {int(nan_got.sum())}, ref {int(nan_ref.sum())}"
    diff = (got - ref).abs()
    diff[nan_ref] = 0
    err = float(diff.max()) if diff.numel() else 0.0
    if half_ulps > 0:
        hu = half_ulp(got, dtype)
        excess = float((diff - tol - half_ulps * hu).max()) if diff.numel() else 0.0
        # the storage roundings the worst element used beyond the absolute bar
        used = ((diff - tol).clamp(min=0) / hu.clamp(min=1e-30))
        need = float(used.max()) if diff.numel() else 0.0
        print(f"[err] max_abs_err {err:.3e} (absolute bar {tol:.0e}); beyond it {need:.2f} half-ulp of |got| "
              f"(allowed {half_ulps})", flush=True)
        assert excess <= 0, (f"max_abs_err {err:.3e} exceeds {tol:.1e} + {half_ulps} * ulp(got)/2 "
                             f"(used {need:.2f} half-ulps)")
    else:
        print(f"[err] max_abs_err {err:.3e} (bar {tol:.0e})", flush=True)
        assert err <= tol, f"max_abs_err {err:.3e} > {tol:.1e}"
    return err
