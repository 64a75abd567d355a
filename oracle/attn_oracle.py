"""fp32 dense+mask attention oracle for tree verification.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).  Also the timed CPU
baseline of ``bench.py`` (``cpu_baseline.kind == "port"``).

``dense_mask_attention`` restates ``torch_baseline_tree_attention``
(benchmark.py:8-35) in float32 on the CPU:
  * GQA by ``repeat_interleave(G, dim=1)`` on K and V   (benchmark.py:17-18)
  * scores = Q K^T / sqrt(D)                             (benchmark.py:21)
  * mask [T, KV]: prefix columns visible, tree columns   (benchmark.py:25-27)
    from the tree mask
  * masked_fill(-inf), softmax, @ V                      (benchmark.py:30-34)
It extends the reference in one way: ``tree_mask`` may be ``[B, T, T]`` (one
tree per sequence); ``[T, T]`` is shared by the batch as in the reference.

``brute_force_attention`` is an independent float64 formulation for tiny
shapes: per (b, h, t) it gathers the visible keys explicitly, so it pins the
torch restatement (a dropped GQA mapping, a wrong mask column offset or a
transposed operand all fail it).  Special cases that reduce to textbook
routines are checked in tests/test_oracle_attn.py (all-ones tree == plain
softmax attention; prefix 0 with identity tree == V; chain tree ==
causal-with-prefix SDPA; prefix 0 and an empty row == NaN).
"""

from __future__ import annotations

import math

import numpy as np
import torch


def _full_mask(tree_mask: torch.Tensor, batch: int, q_len: int, kv_len: int, prefix_len: int) -> torch.Tensor:
    """[B|1, 1, T, KV] bool: prefix visible, tree part from the mask (benchmark.py:25-27)."""
    tm = tree_mask.to(torch.bool).cpu()
    if tm.ndim == 2:
        tm = tm.unsqueeze(0)
    full = torch.zeros((tm.shape[0], q_len, kv_len), dtype=torch.bool)
    full[:, :, :prefix_len] = True
    full[:, :, prefix_len:] = tm
    return full.unsqueeze(1)


def dense_mask_attention(q, k, v, tree_mask, prefix_len: int, *, head_chunk: int | None = None,
                         p_dtype: torch.dtype | None = None) -> torch.Tensor:
    """fp32 CPU restatement of benchmark.py:8-35.  Returns [B, Hq, T, D] float32.

    ``head_chunk`` bounds memory by processing that many query heads at a time
    (the scores tensor is [B, chunk, T, KV] fp32); the result does not depend
    on it.  ``p_dtype`` (default None: plain fp32 softmax) restates the
    reference kernel's own rounding instead: the probabilities
    exp(s - rowmax) are rounded to that dtype before the product with V while
    the row sum takes them unrounded (tree_sparse_flashattn.py:273-278,
    :321-326: ``l_i += tl.sum(p)`` in fp32, ``tl.dot(p.to(v.dtype), v)``).
    """
    q = q.detach().to("cpu", torch.float32)
    k = k.detach().to("cpu", torch.float32)
    v = v.detach().to("cpu", torch.float32)
    bsz, n_heads, q_len, head_dim = q.shape
    _, n_kv_heads, kv_len, _ = k.shape
    group = n_heads // n_kv_heads
    mask = _full_mask(tree_mask, bsz, q_len, kv_len, prefix_len)
    scale = 1.0 / math.sqrt(head_dim)
    chunk = n_heads if head_chunk is None else max(1, int(head_chunk))
    out = torch.empty((bsz, n_heads, q_len, head_dim), dtype=torch.float32)
    for h0 in range(0, n_heads, chunk):
        h1 = min(n_heads, h0 + chunk)
        kv_idx = torch.arange(h0, h1) // group            # repeat_interleave(G, dim=1)
        ke = k[:, kv_idx]
        ve = v[:, kv_idx]
        scores = torch.matmul(q[:, h0:h1], ke.transpose(-2, -1)) * scale
        scores = scores.masked_fill(~mask, float("-inf"))
        if p_dtype is None:
            out[:, h0:h1] = torch.matmul(torch.softmax(scores, dim=-1), ve)
        else:
            p = torch.exp(scores - scores.amax(dim=-1, keepdim=True))  # NaN rows stay NaN (no visible key)
            out[:, h0:h1] = torch.matmul(p.to(p_dtype).float(), ve) / p.sum(dim=-1, keepdim=True)
    return out


def brute_force_attention(q, k, v, tree_mask, prefix_len: int) -> np.ndarray:
    """float64 per-row loop: visible keys gathered explicitly.  Tiny shapes only."""
    qn = np.asarray(q.detach().cpu().double().numpy() if hasattr(q, "detach") else q, dtype=np.float64)
    kn = np.asarray(k.detach().cpu().double().numpy() if hasattr(k, "detach") else k, dtype=np.float64)
    vn = np.asarray(v.detach().cpu().double().numpy() if hasattr(v, "detach") else v, dtype=np.float64)
    tm = tree_mask.detach().cpu().numpy() if hasattr(tree_mask, "detach") else np.asarray(tree_mask)
    tm = tm != 0
    bsz, n_heads, q_len, head_dim = qn.shape
    n_kv_heads = kn.shape[1]
    group = n_heads // n_kv_heads
    out = np.empty_like(qn)
    for b in range(bsz):
        tmb = tm if tm.ndim == 2 else tm[b]
        for h in range(n_heads):
            kvh = h // group
            for t in range(q_len):
                keys = list(range(prefix_len)) + [prefix_len + j for j in range(q_len) if tmb[t, j]]
                if not keys:
                    out[b, h, t] = np.nan
                    continue
                s = np.array([np.dot(qn[b, h, t], kn[b, kvh, j]) for j in keys]) / math.sqrt(head_dim)
                w = np.exp(s - s.max())
                w /= w.sum()
                out[b, h, t] = sum(wi * vn[b, kvh, j] for wi, j in zip(w, keys))
    return out
