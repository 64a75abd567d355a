"""A minimal stand-in for the EAGLE llama module the bridge patches (the symbols
eagle_tree_sparse_bridge.py:166-421 uses).  The un-patched forwards implement the
reference's non-tree paths: LlamaFlexAttention through create_block_mask /
flex_attention (here: dense masked attention over the mask_mod), LlamaAttention's
cache_hidden branch through the manual softmax.  dense_flex_reference() gives the
ground truth for a verify call: the same projections, RoPE and cache update, then
softmax(QK^T/sqrt(D) + attention_mask) V.  Transposed operands of batched
products are made contiguous first (batched half-precision products with a
transposed right operand are avoided on this platform)."""

from __future__ import annotations

import math
import types

import torch
from torch import nn


class Config:
    rope_scaling = {"mrope_section": [16, 24, 24]}


class LlamaRotaryEmbedding(nn.Module):
    def __init__(self, dim, base=10000.0):
        super().__init__()
        self.dim = dim
        self.base = base

    def forward(self, x, seq_len):
        inv = 1.0 / (self.base ** (torch.arange(0, self.dim, 2, dtype=torch.float32, device=x.device) / self.dim))
        t = torch.arange(seq_len, dtype=torch.float32, device=x.device)
        freqs = torch.outer(t, inv)
        emb = torch.cat((freqs, freqs), dim=-1)
        return emb.cos().to(x.dtype), emb.sin().to(x.dtype)


class LlamaMutiRotaryEmbedding(LlamaRotaryEmbedding):
    pass


def rotate_half(x):
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def apply_rotary_pos_emb(q, k, cos, sin, position_ids):
    cos = cos[position_ids].unsqueeze(1)
    sin = sin[position_ids].unsqueeze(1)
    return q * cos + rotate_half(q) * sin, k * cos + rotate_half(k) * sin


def apply_multimodal_rotary_pos_emb(q, k, cos, sin, mrope_section):
    raise NotImplementedError("multimodal RoPE is not exercised by the mock")


def repeat_kv(x, n_rep):
    b, h, s, d = x.shape
    if n_rep == 1:
        return x
    return x[:, :, None].expand(b, h, n_rep, s, d).reshape(b, h * n_rep, s, d)


def generate_eagle3_mask(seq_lengths, Q_LEN, KV_LEN, lck):
    prefix = KV_LEN - Q_LEN

    def mask_mod(b, h, q_idx, kv_idx):  # causal behind the cached prefix
        return kv_idx <= q_idx + prefix

    return mask_mod


def create_block_mask(mask_mod, B, H, Q_LEN, KV_LEN, device):
    q = torch.arange(Q_LEN, device=device)[:, None]
    kv = torch.arange(KV_LEN, device=device)[None, :]
    return mask_mod(None, None, q, kv).expand(B, H, Q_LEN, KV_LEN)


def flex_attention(query, key, value, block_mask, enable_gqa=False):
    g = query.shape[1] // key.shape[1]
    k = key.repeat_interleave(g, dim=1).float()
    v = value.repeat_interleave(g, dim=1).float()
    s = query.float() @ k.transpose(-1, -2).contiguous() / math.sqrt(query.shape[-1])
    s = s.masked_fill(~block_mask, float("-inf"))
    return (torch.softmax(s, dim=-1) @ v).to(query.dtype)


compile_friendly_create_block_mask = create_block_mask
compile_friendly_flex_attention = flex_attention


class DynamicCache:
    def __init__(self, k=None, v=None):
        self.k, self.v = k, v

    def get_seq_length(self):
        return 0 if self.k is None else self.k.shape[2]

    def update(self, key_states, value_states, layer_idx=0, cache_kwargs=None):
        self.k = key_states if self.k is None else torch.cat([self.k, key_states], dim=2)
        self.v = value_states if self.v is None else torch.cat([self.v, value_states], dim=2)
        return self.k, self.v

    def clone(self):
        return DynamicCache(None if self.k is None else self.k.clone(), None if self.v is None else self.v.clone())


class _AttnBase(nn.Module):
    def __init__(self, hidden, num_heads, num_kv_heads, head_dim):
        super().__init__()
        self.config = Config()
        self.num_heads, self.num_key_value_heads, self.head_dim = num_heads, num_kv_heads, head_dim
        self.num_key_value_groups = num_heads // num_kv_heads
        self.q_proj = nn.Linear(hidden, num_heads * head_dim, bias=False)
        self.k_proj = nn.Linear(hidden, num_kv_heads * head_dim, bias=False)
        self.v_proj = nn.Linear(hidden, num_kv_heads * head_dim, bias=False)
        self.o_proj = nn.Linear(num_heads * head_dim, hidden, bias=False)
        self.rotary_emb = LlamaRotaryEmbedding(head_dim)

    def _qkv(self, hidden_states):
        b, q_len, _ = hidden_states.shape
        q = self.q_proj(hidden_states).view(b, q_len, self.num_heads, self.head_dim).transpose(1, 2)
        k = self.k_proj(hidden_states).view(b, q_len, self.num_key_value_heads, self.head_dim).transpose(1, 2)
        v = self.v_proj(hidden_states).view(b, q_len, self.num_key_value_heads, self.head_dim).transpose(1, 2)
        return q, k, v

    def _out(self, attn, b, q_len):
        return self.o_proj(attn.transpose(1, 2).contiguous().reshape(b, q_len, self.num_heads * self.head_dim))


class LlamaFlexAttention(_AttnBase):
    def forward(self, hidden_states, cache_hidden=None, attention_mask=None, position_ids=None,
                past_key_values=None, output_attentions=False, use_cache=False):
        b, q_len, _ = hidden_states.shape
        past = past_key_values.get_seq_length()
        q, k, v = self._qkv(hidden_states)
        lck = past // q_len
        cos, sin = self.rotary_emb(q, seq_len=q_len + lck)
        q, k = apply_rotary_pos_emb(q, k, cos, sin, position_ids + lck)
        kc, vc = past_key_values.update(k, v, layer_idx=0, cache_kwargs={})
        kv_len = kc.shape[-2]
        seq_lengths = attention_mask.sum(dim=-1) - lck
        bm = create_block_mask(generate_eagle3_mask(seq_lengths, q_len, kv_len, lck), b, 1, q_len, kv_len, q.device)
        return self._out(flex_attention(q, kc.contiguous(), vc.contiguous(), bm, enable_gqa=True), b, q_len)


class LlamaAttention(_AttnBase):
    def forward(self, hidden_states, cache_hidden=None, attention_mask=None, position_ids=None,
                past_key_values=None, output_attentions=False, use_cache=False):
        b, q_len, _ = hidden_states.shape
        q, k, v = self._qkv(hidden_states)
        if cache_hidden is None:  # plain attention with the additive mask
            cos, sin = self.rotary_emb(q, seq_len=q_len)
            q, k = apply_rotary_pos_emb(q, k, cos, sin, position_ids)
            k, v = repeat_kv(k, self.num_key_value_groups), repeat_kv(v, self.num_key_value_groups)
            w = q @ k.transpose(2, 3).contiguous() / math.sqrt(self.head_dim)
            if attention_mask is not None:
                w = w + attention_mask
            w = torch.softmax(w, dim=-1, dtype=torch.float32).to(q.dtype)
            return self._out(w @ v.contiguous(), b, q_len)
        lck = len(cache_hidden[0])
        cos, sin = self.rotary_emb(q, seq_len=q_len + lck)
        q, k = apply_rotary_pos_emb(q, k, cos, sin, position_ids + lck)
        k, v = repeat_kv(k, self.num_key_value_groups), repeat_kv(v, self.num_key_value_groups)
        cache_hidden[0] = cache_hidden[0] + [k]
        cache_hidden[1] = cache_hidden[1] + [v]
        k0, v0 = cache_hidden[0][0], cache_hidden[1][0]
        w = torch.matmul(q, k0.transpose(2, 3).contiguous()) / math.sqrt(self.head_dim)
        if attention_mask is not None:
            w = w + attention_mask
        n = len(cache_hidden[0])
        for i in range(1, n):
            w = torch.cat((w, ((q * cache_hidden[0][i]).sum(-1) / math.sqrt(self.head_dim))[..., None]), dim=-1)
        w = torch.softmax(w, dim=-1, dtype=torch.float32).to(q.dtype)
        out = torch.matmul(w[..., :q_len], v0.contiguous())
        for i in range(1, n):
            out = out + w[..., q_len + i - 1][..., None] * cache_hidden[1][i]
        return self._out(out, b, q_len)


def dense_flex_reference(module, hidden_states, attention_mask, position_ids, past_key_values):
    """Ground truth of a verify call of LlamaFlexAttention (fp32 attention)."""
    b, q_len, _ = hidden_states.shape
    past = past_key_values.get_seq_length()
    q, k, v = module._qkv(hidden_states)
    lck = past // q_len
    cos, sin = module.rotary_emb(q, seq_len=q_len + lck)
    q, k = apply_rotary_pos_emb(q, k, cos, sin, position_ids + lck)
    kc, vc = past_key_values.update(k, v)
    g = module.num_key_value_groups
    kf, vf = kc.repeat_interleave(g, dim=1).float(), vc.repeat_interleave(g, dim=1).float()
    s = q.float() @ kf.transpose(-1, -2).contiguous() / math.sqrt(module.head_dim) + attention_mask.float()
    attn = (torch.softmax(s, dim=-1) @ vf).to(q.dtype)
    return module._out(attn, b, q_len)


def make_module():
    """A fresh module object exposing the patched symbols (patching mutates classes)."""
    ns = {name: globals()[name] for name in (
        "LlamaMutiRotaryEmbedding", "apply_rotary_pos_emb", "apply_multimodal_rotary_pos_emb", "repeat_kv",
        "create_block_mask", "flex_attention", "compile_friendly_create_block_mask",
        "compile_friendly_flex_attention", "generate_eagle3_mask")}
    ns["LlamaFlexAttention"] = type("LlamaFlexAttention", (LlamaFlexAttention,), {})
    ns["LlamaAttention"] = type("LlamaAttention", (LlamaAttention,), {})
    return types.SimpleNamespace(**ns)


def additive_mask(tree_mask_bool, prefix_len, batch, dtype):
    """[B, 1, Q, P+Q] additive mask: 0 on the prefix and visible tree keys, -inf elsewhere."""
    q = tree_mask_bool.shape[0]
    vis = torch.ones(q, prefix_len + q, dtype=torch.bool)
    vis[:, prefix_len:] = tree_mask_bool
    m = torch.zeros(q, prefix_len + q, dtype=dtype).masked_fill(~vis, float("-inf"))
    return m[None, None].expand(batch, 1, q, prefix_len + q).contiguous()
