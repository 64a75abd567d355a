"""EAGLE verification entry points for the MI355X tree-sparse attention.

Drop-in for the reference's ``eagle_tree_sparse_bridge.py`` launch path:
  extract_tree_mask_from_attention_mask   eagle_tree_sparse_bridge.py:24-70
  run_tree_sparse_kernel                   eagle_tree_sparse_bridge.py:76-159

Differences from the reference, all in the caller's favour:
  * the metadata is built on the GPU from the device mask (no ``.cpu()``
    sync and no host->device copies, eagle_tree_sparse_bridge.py:95-106);
  * ``tree_mask`` may also be [B, Q, Q] (one tree per sequence); the
    reference accepts one [Q, Q] tree for the whole batch;
  * O is written in the input dtype (the reference stores through fp16,
    tree_sparse_flashattn.py:339).
"""

from __future__ import annotations

from typing import Optional

import torch

from tree_sparse_flashattn import (
    prepare_tree_sparse_metadata,
    prepare_tree_sparse_metadata_batched,
    tree_sparse_attention_fwd,
)


def extract_tree_mask_from_attention_mask(
    attention_mask: Optional[torch.Tensor],
    q_len: int,
    kv_len: int,
    *,
    batch_idx: int = 0,
) -> Optional[torch.Tensor]:
    """Tree-only [Q, Q] bool mask from a HF/EAGLE [B, 1, Q, KV] attention mask.

    Semantics of eagle_tree_sparse_bridge.py:24-70: 0 = visible, -inf =
    masked for float masks (visible iff finite and >= 0), nonzero = visible
    for bool/int masks; tree columns are the last Q of KV.  Returns None (the
    caller falls back) when the mask is None, q_len <= 1, not 4-D, too small,
    or kv_len < q_len.
    """
    if attention_mask is None:
        return None
    if q_len <= 1:
        return None
    if attention_mask.ndim != 4:
        return None
    if attention_mask.shape[2] < q_len or attention_mask.shape[3] < kv_len:
        return None
    prefix_len = kv_len - q_len
    if prefix_len < 0:
        return None
    tree_slice = attention_mask[batch_idx, 0, :q_len, prefix_len:prefix_len + q_len]
    if tree_slice.shape != (q_len, q_len):
        return None
    if torch.is_floating_point(tree_slice):
        tree_mask = torch.isfinite(tree_slice) & (tree_slice >= 0)
    else:
        tree_mask = tree_slice.to(torch.bool)
    return tree_mask.contiguous()


def run_tree_sparse_kernel(
    query_states: torch.Tensor,  # [B, Hq, Q, D]
    key_states: torch.Tensor,    # [B, Hkv, KV, D]
    value_states: torch.Tensor,  # [B, Hkv, KV, D]
    tree_mask: torch.Tensor,     # [Q, Q] (or [B, Q, Q]) bool
    *,
    block_m: int,
    block_n: int,
) -> torch.Tensor:
    """Tree-sparse verification attention (eagle_tree_sparse_bridge.py:76-159)."""
    assert query_states.is_cuda and key_states.is_cuda and value_states.is_cuda
    bsz, num_heads, q_len, head_dim = query_states.shape
    b2, num_kv_heads, kv_len, d2 = key_states.shape
    assert bsz == b2 and head_dim == d2
    assert value_states.shape == key_states.shape

    prefix_len = kv_len - q_len
    if prefix_len < 0:
        raise ValueError(f"Invalid lengths: kv_len={kv_len}, q_len={q_len}")

    mask = tree_mask.to(device=query_states.device)
    if mask.ndim == 3:
        meta = prepare_tree_sparse_metadata_batched(mask, prefix_len, block_m, block_n)
    else:
        meta = prepare_tree_sparse_metadata(mask, prefix_len, block_m, block_n)
    return tree_sparse_attention_fwd(query_states, key_states, value_states, meta)
