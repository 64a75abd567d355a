"""EAGLE verification entry points for the MI355X tree-sparse attention.

Drop-in for the reference's ``eagle_tree_sparse_bridge.py``:
  extract_tree_mask_from_attention_mask   eagle_tree_sparse_bridge.py:24-70
  run_tree_sparse_kernel                   eagle_tree_sparse_bridge.py:76-159
  patch_llama_flex_attention               eagle_tree_sparse_bridge.py:166-287
  patch_llama_attention                    eagle_tree_sparse_bridge.py:290-415
  inject_tree_sparse_bridge                eagle_tree_sparse_bridge.py:418-421

Differences from the reference, all in the caller's favour:
  * the metadata is built on the GPU from the device mask, with no host
    synchronisation at all (the reference does ``.cpu()`` and five
    host->device copies per call, eagle_tree_sparse_bridge.py:95-106), so a
    whole verification call can be captured in a HIP graph;
  * one metadata build can serve every layer: ``run_tree_sparse_kernel``
    takes an optional prebuilt ``metadata``, and ``TreeSparseMetadataCache``
    keys builds on the source mask tensor;
  * ``tree_mask`` may also be [B, Q, Q] (one tree per sequence); the
    reference accepts one [Q, Q] tree for the whole batch;
  * O is written in the input dtype (the reference stores through fp16,
    tree_sparse_flashattn.py:339).
"""

from __future__ import annotations

import math
from collections import OrderedDict
from typing import Callable, Optional, Tuple

import torch

from tree_sparse_flashattn import (
    BatchedTreeSparseMetadata,
    _check_qkv,
    _layout_ok,
    prepare_tree_sparse_metadata_batched,
    tree_sparse_attention_fwd,
)
from tsfa import _lib


def build_tree_metadata(tree_mask: torch.Tensor, prefix_len: int, block_m: int,
                        block_n: int) -> BatchedTreeSparseMetadata:
    """Device metadata for a [Q, Q] tree (shared by the batch) or [B, Q, Q]
    trees, built on the mask's HIP device without a host synchronisation."""
    return prepare_tree_sparse_metadata_batched(tree_mask, prefix_len, block_m, block_n)


class TreeSparseMetadataCache:
    """Reuses tree metadata across the layers of one verification step.

    A model calls the attention once per layer with the same attention-mask
    tensor; the first call builds the tree mask and its metadata, the others
    reuse them.  The key is the source tensor's identity -- storage pointer,
    shape, strides, dtype, device and its in-place version counter (an
    in-place write to the mask forces a rebuild) -- plus the geometry
    (prefix_len, q_len, block sizes, batch index).  Entries keep their source
    tensor alive, so a pointer cannot be reused by another tensor while its
    entry exists.  At most ``capacity`` entries, least recently used first out.
    """

    def __init__(self, capacity: int = 4):
        if capacity <= 0:
            raise ValueError("capacity must be positive")
        self.capacity = capacity
        self._entries: "OrderedDict[Tuple, Tuple[torch.Tensor, object]]" = OrderedDict()
        self.builds = 0
        self.hits = 0

    @staticmethod
    def key(source: torch.Tensor, *geometry) -> Tuple:
        return (source.data_ptr(), tuple(source.shape), tuple(source.stride()), source.dtype, source.device,
                source._version, *geometry)

    def get(self, source: torch.Tensor, geometry: Tuple, build: Callable[[], object]):
        k = self.key(source, *geometry)
        hit = self._entries.get(k)
        if hit is not None:
            self._entries.move_to_end(k)
            self.hits += 1
            return hit[1]
        value = build()
        self.builds += 1
        self._entries[k] = (source, value)
        while len(self._entries) > self.capacity:
            self._entries.popitem(last=False)
        return value

    def clear(self) -> None:
        self._entries.clear()


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
    tree_mask: Optional[torch.Tensor],  # [Q, Q] (or [B, Q, Q]) bool; unused with ``metadata``
    *,
    block_m: int,
    block_n: int,
    metadata=None,
) -> torch.Tensor:
    """Tree-sparse verification attention (eagle_tree_sparse_bridge.py:76-159).

    ``metadata`` (extension): a record from ``build_tree_metadata`` or
    ``prepare_tree_sparse_metadata[_batched]`` to reuse instead of building
    one from ``tree_mask``; its geometry must match this call.
    """
    assert query_states.is_cuda and key_states.is_cuda and value_states.is_cuda
    bsz, num_heads, q_len, head_dim = query_states.shape
    b2, num_kv_heads, kv_len, d2 = key_states.shape
    assert bsz == b2 and head_dim == d2
    assert value_states.shape == key_states.shape

    prefix_len = kv_len - q_len
    if prefix_len < 0:
        raise ValueError(f"Invalid lengths: kv_len={kv_len}, q_len={q_len}")

    if metadata is None:
        if tree_mask is None:
            raise ValueError("run_tree_sparse_kernel needs a tree_mask or prebuilt metadata")
        out = _tree_call(query_states, key_states, value_states, tree_mask, block_m, block_n)
        if out is not None:
            return out
        metadata = build_tree_metadata(tree_mask.to(device=query_states.device), prefix_len, block_m, block_n)
    else:
        nqb = (q_len + block_m - 1) // block_m
        ntb = (q_len + block_n - 1) // block_n
        if (metadata.prefix_len, metadata.block_m, metadata.block_n, metadata.n_q_blocks,
                metadata.n_tree_blocks) != (prefix_len, block_m, block_n, nqb, ntb):
            raise ValueError("metadata was built for another prefix_len, q_len or block size")
    return tree_sparse_attention_fwd(query_states, key_states, value_states, metadata)


# Launch arguments of the one-call path (tsfa_tree_attention: the metadata
# built from the device mask, then the forward, in one C call) per geometry;
# False marks a geometry that takes the general path.
_TREE_CALLS: dict = {}


def _tree_call_plan(q, k, v, mask, block_m, block_n):
    """Launch arguments of tsfa_tree_attention for this geometry, or False when
    the call needs the general path (a mask that is not a bool device tensor
    with unit column stride, head dims the kernels pad, layouts they copy)."""
    _check_qkv(q, k, v)
    bsz, n_heads, q_len, head_dim = q.shape
    _, n_kv_heads, kv_len, _ = k.shape
    if head_dim not in (64, 128) or not all(_layout_ok(t) for t in (q, k, v)):
        return False
    if mask.dim() == 2:
        n_masks, seq_stride = 1, 0
    elif mask.dim() == 3 and mask.shape[0] in (1, bsz):
        n_masks, seq_stride = mask.shape[0], mask.stride(0)
    else:
        return False
    if tuple(mask.shape[-2:]) != (q_len, q_len) or mask.stride(-1) != 1 or mask.stride(-2) < 1:
        return False
    probe = torch.empty_like(q)  # the strides empty_like gives O for this q layout
    if not _layout_ok(probe):
        return False
    lib = _lib.load()
    ws_bytes = lib.tsfa_tree_attention_workspace_bytes(bsz, n_heads, n_kv_heads, q_len, kv_len, n_masks, block_m,
                                                        block_n, head_dim, _lib.dtype_code(q.dtype))
    if ws_bytes == 0:
        return False
    strides = _lib.i64_array((*q.stride(), *k.stride(), *v.stride(), *probe.stride()))
    ints = (bsz, n_heads, n_kv_heads, q_len, kv_len, block_m, block_n, head_dim, _lib.dtype_code(q.dtype))
    return (strides, ints, ws_bytes, 1.0 / math.sqrt(head_dim), n_masks, seq_stride, mask.stride(-2))


def _tree_call(q, k, v, mask, block_m, block_n):
    """run_tree_sparse_kernel on a device mask in one C call, or None."""
    if mask.dtype != torch.bool or mask.device != q.device or q.dtype != k.dtype or q.dtype != v.dtype:
        return None
    key = (q.shape, q.stride(), k.shape, k.stride(), v.stride(), q.dtype, mask.shape, mask.stride(), block_m,
           block_n, q.device, (q.data_ptr() | k.data_ptr() | v.data_ptr()) & 15)
    entry = _TREE_CALLS.get(key)
    if entry is None:
        if q.dtype not in (torch.float16, torch.bfloat16):
            entry = False
        else:
            entry = _tree_call_plan(q, k, v, mask, block_m, block_n)
        if len(_TREE_CALLS) >= 64:
            _TREE_CALLS.clear()
        _TREE_CALLS[key] = entry
    if entry is False:
        return None
    strides, ints, ws_bytes, scale, n_masks, seq_stride, row_stride = entry
    dev = q.device
    out = torch.empty_like(q)
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=dev)
    lib = _lib.load()
    args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), mask.data_ptr(), seq_stride, row_stride, n_masks,
            strides, scale, *ints, ws.data_ptr(), ws_bytes)
    if dev.index == torch.cuda.current_device():
        st = lib.tsfa_tree_attention(*args, _lib.stream_handle(dev))
    else:
        with torch.cuda.device(dev):
            st = lib.tsfa_tree_attention(*args, _lib.stream_handle(dev))
    _lib.check("run_tree_sparse_kernel", st)
    return out


# ------------------------------------------------------------ model shims
# Monkey patches for an EAGLE llama module (eagle_tree_sparse_bridge.py:162-421).
# They need these symbols of the module: LlamaFlexAttention, LlamaAttention,
# LlamaMutiRotaryEmbedding, apply_rotary_pos_emb, apply_multimodal_rotary_pos_emb,
# repeat_kv, create_block_mask, flex_attention, compile_friendly_create_block_mask,
# compile_friendly_flex_attention, generate_eagle3_mask.  The verify condition
# and every fallback follow the reference; the tree branch differs only where
# the caller gains: one metadata build per attention mask serves every layer
# (TreeSparseMetadataCache), and the cache_hidden branch hands the kernel the
# un-expanded K/V heads (GQA) instead of the repeat_kv copies.

_MARK = "_orig_forward_tree_sparse_bridge"


def _rope(llama_module, module, query_states, key_states, position_ids, lck, q_len):
    """RoPE as the reference applies it (eagle_tree_sparse_bridge.py:205-219, :340-354)."""
    if isinstance(module.rotary_emb, llama_module.LlamaMutiRotaryEmbedding):
        cos, sin = module.rotary_emb(query_states, position_ids + lck)
        cos, sin = cos.to(query_states.device), sin.to(query_states.device)
        return llama_module.apply_multimodal_rotary_pos_emb(query_states, key_states, cos, sin,
                                                            module.config.rope_scaling["mrope_section"]) + (cos, sin)
    cos, sin = module.rotary_emb(query_states, seq_len=q_len + lck)
    cos, sin = cos.to(query_states.device), sin.to(query_states.device)
    q, k = llama_module.apply_rotary_pos_emb(query_states, key_states, cos, sin, position_ids + lck)
    return q, k, cos, sin


def _project(module, hidden_states):
    bsz, q_len, _ = hidden_states.size()
    q = module.q_proj(hidden_states).view(bsz, q_len, module.num_heads, module.head_dim).transpose(1, 2)
    k = module.k_proj(hidden_states).view(bsz, q_len, module.num_key_value_heads, module.head_dim).transpose(1, 2)
    v = module.v_proj(hidden_states).view(bsz, q_len, module.num_key_value_heads, module.head_dim).transpose(1, 2)
    return q, k, v


def _tree_metadata(cls, attention_mask, q_len, kv_len, block_m, block_n, device):
    """The tree metadata of this attention mask, built on its first use by any
    layer of the patched class (None when the mask does not describe a tree)."""
    if attention_mask is None or q_len <= 1:
        return None
    cache = cls._tree_sparse_metadata_cache

    def build():
        tree_mask = extract_tree_mask_from_attention_mask(attention_mask, q_len, kv_len)
        if tree_mask is None:
            return None
        return build_tree_metadata(tree_mask.to(device=device), kv_len - q_len, block_m, block_n)

    return cache.get(attention_mask, (q_len, kv_len, block_m, block_n, 0), build)


def patch_llama_flex_attention(llama_module, *, block_m: int = 64, block_n: int = 64):
    """Route LlamaFlexAttention's verify calls to the tree-sparse kernel
    (eagle_tree_sparse_bridge.py:166-287); idempotent."""
    cls = llama_module.LlamaFlexAttention
    if hasattr(cls, _MARK):
        return
    setattr(cls, _MARK, cls.forward)
    cls._tree_sparse_metadata_cache = TreeSparseMetadataCache()

    def _forward(self, hidden_states, cache_hidden=None, attention_mask=None, position_ids=None,
                 past_key_values=None, output_attentions=False, use_cache=False):
        bsz, q_len, _ = hidden_states.size()
        past_seen_tokens = past_key_values.get_seq_length() if past_key_values is not None else 0
        query_states, key_states, value_states = _project(self, hidden_states)
        lck = past_seen_tokens // q_len
        query_states, key_states, cos, sin = _rope(llama_module, self, query_states, key_states, position_ids, lck,
                                                   q_len)
        cache_position = torch.arange(past_seen_tokens, past_seen_tokens + q_len, device=hidden_states.device)
        key_cache, value_cache = past_key_values.update(
            key_states, value_states, layer_idx=0,
            cache_kwargs={"sin": sin, "cos": cos, "cache_position": cache_position})
        key_cache = key_cache.contiguous()
        value_cache = value_cache.contiguous()
        kv_len = key_cache.shape[-2]

        meta = _tree_metadata(cls, attention_mask, q_len, kv_len, block_m, block_n, query_states.device)
        if meta is not None:
            attn_output = run_tree_sparse_kernel(query_states.contiguous(), key_cache, value_cache, None,
                                                 block_m=block_m, block_n=block_n, metadata=meta)
        else:  # the flex-attention path (eagle_tree_sparse_bridge.py:248-280)
            seq_lengths = attention_mask.sum(dim=-1)
            seq_lengths -= lck
            if q_len <= 128:
                create_block_mask, flex = llama_module.create_block_mask, llama_module.flex_attention
            else:
                create_block_mask = llama_module.compile_friendly_create_block_mask
                flex = llama_module.compile_friendly_flex_attention
            block_mask = create_block_mask(
                mask_mod=llama_module.generate_eagle3_mask(seq_lengths=seq_lengths, Q_LEN=q_len, KV_LEN=kv_len,
                                                           lck=lck),
                B=bsz, H=1, Q_LEN=q_len, KV_LEN=kv_len, device=query_states.device)
            attn_output = flex(query=query_states, key=key_cache, value=value_cache, block_mask=block_mask,
                               enable_gqa=True)
        attn_output = attn_output.transpose(1, 2).contiguous().reshape(bsz, q_len, self.head_dim * self.num_heads)
        return self.o_proj(attn_output)

    cls.forward = _forward


def patch_llama_attention(llama_module, *, block_m: int = 64, block_n: int = 64):
    """Route LlamaAttention's cache_hidden (EAGLE3 TTT) verify calls to the
    tree-sparse kernel (eagle_tree_sparse_bridge.py:290-415); idempotent."""
    cls = llama_module.LlamaAttention
    if hasattr(cls, _MARK):
        return
    setattr(cls, _MARK, cls.forward)
    cls._tree_sparse_metadata_cache = TreeSparseMetadataCache()

    def _forward(self, hidden_states, cache_hidden=None, attention_mask=None, position_ids=None,
                 past_key_values=None, output_attentions=False, use_cache=False):
        if cache_hidden is None:  # prefill / plain decode: the original forward
            return getattr(cls, _MARK)(self, hidden_states=hidden_states, cache_hidden=cache_hidden,
                                       attention_mask=attention_mask, position_ids=position_ids,
                                       past_key_values=past_key_values, output_attentions=output_attentions,
                                       use_cache=use_cache)
        bsz, q_len, _ = hidden_states.size()
        query_states, key_states, value_states = _project(self, hidden_states)
        lck = len(cache_hidden[0])
        query_states, key_states, _, _ = _rope(llama_module, self, query_states, key_states, position_ids, lck,
                                               q_len)
        # the cache keeps repeat_kv copies, as the original forward stores them
        n_rep = self.num_key_value_groups
        key_states = llama_module.repeat_kv(key_states, n_rep)
        value_states = llama_module.repeat_kv(value_states, n_rep)
        cache_hidden[0] = cache_hidden[0] + [key_states]
        cache_hidden[1] = cache_hidden[1] + [value_states]
        kv_len = sum(t.shape[2] for t in cache_hidden[0])

        meta = _tree_metadata(cls, attention_mask, q_len, kv_len, block_m, block_n, query_states.device)
        if meta is not None:
            # head h of a repeat_kv copy is kv head h // n_rep: every n_rep-th
            # head is the un-expanded K/V, concatenated once for the kernel
            full_k = torch.cat([t[:, ::n_rep] for t in cache_hidden[0]], dim=2)
            full_v = torch.cat([t[:, ::n_rep] for t in cache_hidden[1]], dim=2)
            attn_output = run_tree_sparse_kernel(query_states.contiguous(), full_k, full_v, None, block_m=block_m,
                                                 block_n=block_n, metadata=meta)
        else:  # the original cache_hidden attention (eagle_tree_sparse_bridge.py:384-409)
            k0, v0 = cache_hidden[0][0], cache_hidden[1][0]
            # transposed operand materialised: batched half-precision products with a
            # transposed right operand are avoided on this platform (same result)
            attn_weights = torch.matmul(query_states, k0.transpose(2, 3).contiguous()) / math.sqrt(self.head_dim)
            if attention_mask is not None:
                attn_weights = attn_weights + attention_mask
            l_total = len(cache_hidden[0])
            for i in range(1, l_total):
                ki = cache_hidden[0][i]
                wi = (query_states * ki).sum(-1) / math.sqrt(self.head_dim)
                attn_weights = torch.cat((attn_weights, wi[..., None]), dim=-1)
            attn_weights = torch.nn.functional.softmax(attn_weights, dim=-1, dtype=torch.float32).to(
                query_states.dtype)
            attn_output = torch.matmul(attn_weights[..., :q_len], v0.contiguous())
            for i in range(1, l_total):
                attn_output = attn_output + attn_weights[..., q_len + i - 1][..., None] * cache_hidden[1][i]
        attn_output = attn_output.transpose(1, 2).contiguous().reshape(bsz, q_len, self.head_dim * self.num_heads)
        return self.o_proj(attn_output)

    cls.forward = _forward


def inject_tree_sparse_bridge(llama_module, *, block_m: int = 64, block_n: int = 64):
    """Patch both attention classes (eagle_tree_sparse_bridge.py:418-421)."""
    patch_llama_flex_attention(llama_module, block_m=block_m, block_n=block_n)
    patch_llama_attention(llama_module, block_m=block_m, block_n=block_n)
