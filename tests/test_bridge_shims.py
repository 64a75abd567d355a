"""Model shims on the CPU: patching is idempotent, and every non-tree call
(q_len 1, no tree in the mask, no cache_hidden) goes through the reference's
fallback and equals the un-patched forward exactly."""

import numpy as np
import torch

import eagle_tree_sparse_bridge as bridge
from tests import llama_mock
from tsfa import trees


def _hidden(b, q, hidden=64, seed=0):
    return torch.randn(b, q, hidden, generator=torch.Generator().manual_seed(seed))


def test_inject_is_idempotent_and_keeps_the_original():
    mod = llama_mock.make_module()
    f0, a0 = mod.LlamaFlexAttention.forward, mod.LlamaAttention.forward
    bridge.inject_tree_sparse_bridge(mod, block_m=16, block_n=32)
    f1, a1 = mod.LlamaFlexAttention.forward, mod.LlamaAttention.forward
    bridge.inject_tree_sparse_bridge(mod, block_m=16, block_n=32)
    assert mod.LlamaFlexAttention.forward is f1 and mod.LlamaAttention.forward is a1
    assert mod.LlamaFlexAttention._orig_forward_tree_sparse_bridge is f0
    assert mod.LlamaAttention._orig_forward_tree_sparse_bridge is a0


def test_flex_single_token_decode_falls_back():
    torch.manual_seed(0)
    mod = llama_mock.make_module()
    m = mod.LlamaFlexAttention(64, 4, 2, 16)
    h = _hidden(1, 1)
    mask = torch.zeros(1, 1, 1, 9)
    pos = torch.zeros(1, 1, dtype=torch.long)
    prefix = llama_mock.DynamicCache(torch.randn(1, 2, 8, 16), torch.randn(1, 2, 8, 16))
    want = m(h, attention_mask=mask, position_ids=pos, past_key_values=prefix.clone())
    bridge.patch_llama_flex_attention(mod)
    got = m(h, attention_mask=mask, position_ids=pos, past_key_values=prefix.clone())
    assert torch.equal(got, want)


def test_flex_mask_without_tree_falls_back():
    torch.manual_seed(1)
    mod = llama_mock.make_module()
    m = mod.LlamaFlexAttention(64, 4, 2, 16)
    h = _hidden(1, 4)
    mask = torch.zeros(1, 1, 4, 10)[..., :9]  # smaller than KV: no tree can be extracted
    pos = torch.arange(4)[None]
    prefix = llama_mock.DynamicCache(torch.randn(1, 2, 6, 16), torch.randn(1, 2, 6, 16))
    want = m(h, attention_mask=mask, position_ids=pos, past_key_values=prefix.clone())
    bridge.patch_llama_flex_attention(mod)
    assert bridge.extract_tree_mask_from_attention_mask(mask, 4, 10) is None
    got = m(h, attention_mask=mask, position_ids=pos, past_key_values=prefix.clone())
    assert torch.equal(got, want)


def test_attention_without_cache_hidden_calls_the_original():
    torch.manual_seed(2)
    mod = llama_mock.make_module()
    m = mod.LlamaAttention(64, 4, 2, 16)
    h = _hidden(2, 5)
    pos = torch.arange(5)[None].expand(2, 5)
    mask = llama_mock.additive_mask(torch.from_numpy(trees.ancestor_mask(trees.kary_bfs_parents(5, 2))), 0, 2,
                                    torch.float32)
    want = m(h, attention_mask=mask, position_ids=pos)
    bridge.patch_llama_attention(mod)
    got = m(h, attention_mask=mask, position_ids=pos)
    assert torch.equal(got, want)


def test_attention_cache_hidden_without_tree_falls_back():
    torch.manual_seed(3)
    mod = llama_mock.make_module()
    m = mod.LlamaAttention(64, 4, 2, 16)
    h1, h2 = _hidden(1, 4, seed=1), _hidden(1, 4, seed=2)
    pos = torch.arange(4)[None]
    mask = llama_mock.additive_mask(torch.from_numpy(trees.ancestor_mask(trees.random_parents(
        4, np.random.default_rng(0)))), 0, 1, torch.float32)
    # step 2 of a TTT loop: the mask covers only the first chunk, so no tree is extracted
    ch_want, ch_got = [[], []], [[], []]
    m(h1, cache_hidden=ch_want, attention_mask=mask, position_ids=pos)
    want = m(h2, cache_hidden=ch_want, attention_mask=mask, position_ids=pos)
    bridge.patch_llama_attention(mod)
    m(h1, cache_hidden=ch_got, attention_mask=None, position_ids=pos)
    got = m(h2, cache_hidden=ch_got, attention_mask=mask, position_ids=pos)
    assert torch.equal(got, want)
    assert all(torch.equal(a, b) for a, b in zip(ch_got[0], ch_want[0]))  # the cache keeps repeat_kv copies
