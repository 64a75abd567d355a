"""Pins the fp32 attention oracle (oracle/attn_oracle.py).

Against an independent float64 per-row loop on tiny shapes, and against
special cases that reduce to textbook routines: an all-ones tree is plain
softmax attention over every key; a chain (tril) tree is causal attention
behind a visible prefix; prefix 0 with an identity tree returns V exactly;
prefix 0 with an empty tree row is NaN (0/0), as in the reference.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle.attn_oracle import brute_force_attention, dense_mask_attention
from tsfa import trees


def _inputs(b, hq, hkv, t, p, d, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, hq, t, d, generator=g)
    k = torch.randn(b, hkv, p + t, d, generator=g)
    v = torch.randn(b, hkv, p + t, d, generator=g)
    return q, k, v


@pytest.mark.parametrize("b,hq,hkv,t,p,d", [(1, 2, 1, 9, 5, 8), (2, 4, 2, 7, 0, 4), (1, 3, 3, 12, 3, 16)])
def test_matches_float64_brute_force(b, hq, hkv, t, p, d):
    q, k, v = _inputs(b, hq, hkv, t, p, d)
    rng = np.random.default_rng(1)
    masks = torch.from_numpy(np.stack([trees.ancestor_mask(trees.random_parents(t, rng)) for _ in range(b)]))
    out = dense_mask_attention(q, k, v, masks, p)
    ref = brute_force_attention(q, k, v, masks, p)
    np.testing.assert_allclose(out.numpy(), ref, atol=2e-6, rtol=1e-5)
    # shared [T, T] mask == the same mask repeated per sequence
    out_shared = dense_mask_attention(q, k, v, masks[0], p)
    out_rep = dense_mask_attention(q, k, v, masks[0].expand(b, t, t), p)
    torch.testing.assert_close(out_shared, out_rep)


def test_head_chunking_is_exact():
    q, k, v = _inputs(2, 8, 2, 10, 6, 8)
    m = torch.from_numpy(trees.ancestor_mask(trees.kary_bfs_parents(10, 3)))
    torch.testing.assert_close(dense_mask_attention(q, k, v, m, 6), dense_mask_attention(q, k, v, m, 6, head_chunk=3))


def test_all_ones_tree_is_plain_attention():
    q, k, v = _inputs(1, 4, 2, 6, 5, 8)
    out = dense_mask_attention(q, k, v, torch.ones(6, 6, dtype=torch.bool), 5)
    ke, ve = k.repeat_interleave(2, dim=1), v.repeat_interleave(2, dim=1)
    ref = F.scaled_dot_product_attention(q, ke, ve)
    torch.testing.assert_close(out, ref, atol=1e-5, rtol=1e-5)


def test_chain_tree_is_causal_behind_prefix():
    t, p = 8, 4
    q, k, v = _inputs(1, 2, 2, t, p, 8)
    chain = torch.from_numpy(trees.ancestor_mask(np.arange(-1, t - 1)))
    assert torch.equal(chain, torch.tril(torch.ones(t, t, dtype=torch.bool)))
    out = dense_mask_attention(q, k, v, chain, p)
    allowed = torch.ones(t, p + t, dtype=torch.bool)
    allowed[:, p:] = torch.tril(torch.ones(t, t, dtype=torch.bool))
    ref = F.scaled_dot_product_attention(q, k, v, attn_mask=allowed)
    torch.testing.assert_close(out, ref, atol=1e-5, rtol=1e-5)


def test_identity_tree_without_prefix_returns_v():
    q, k, v = _inputs(2, 4, 2, 5, 0, 8)
    out = dense_mask_attention(q, k, v, torch.eye(5, dtype=torch.bool), 0)
    torch.testing.assert_close(out, v.repeat_interleave(2, dim=1), atol=0, rtol=0)


def test_empty_row_without_prefix_is_nan():
    q, k, v = _inputs(1, 1, 1, 3, 0, 4)
    m = torch.eye(3, dtype=torch.bool)
    m[1, 1] = False
    out = dense_mask_attention(q, k, v, m, 0)
    assert torch.isnan(out[0, 0, 1]).all()
    assert not torch.isnan(out[0, 0, 0]).any() and not torch.isnan(out[0, 0, 2]).any()
    assert np.isnan(brute_force_attention(q, k, v, m, 0)[0, 0, 1]).all()


def test_gqa_mapping_is_h_div_group():
    # heads 0..3 share kv head 0, heads 4..7 kv head 1 (repeat_interleave, benchmark.py:17-18)
    q, k, v = _inputs(1, 8, 2, 4, 3, 8)
    m = torch.ones(4, 4, dtype=torch.bool)
    out = dense_mask_attention(q, k, v, m, 3)
    for h in range(8):
        ref = F.scaled_dot_product_attention(q[:, h:h + 1], k[:, h // 4:h // 4 + 1], v[:, h // 4:h // 4 + 1])
        torch.testing.assert_close(out[:, h:h + 1], ref, atol=1e-5, rtol=1e-5)


def test_scale_is_inverse_sqrt_head_dim():
    q, k, v = _inputs(1, 1, 1, 1, 1, 16)
    out = dense_mask_attention(q, k, v, torch.ones(1, 1, dtype=torch.bool), 1)
    s = (q[0, 0] @ k[0, 0].T) / math.sqrt(16)
    ref = torch.softmax(s, -1) @ v[0, 0]
    torch.testing.assert_close(out[0, 0], ref, atol=1e-6, rtol=1e-6)


@pytest.mark.parametrize("p_dtype", [torch.bfloat16, torch.float16])
def test_reference_p_rounding_matches_a_per_row_loop(p_dtype):
    # the reference's own numerics (p rounded to the input dtype before P.V,
    # the row sum from unrounded p; tree_sparse_flashattn.py:273-278): against
    # a float64 loop that gathers each row's visible keys and rounds each p
    # explicitly, and within 2^-(mantissa+1) * sum(p|v|) / l of the plain oracle
    b, hq, hkv, t, p, d = 2, 4, 2, 11, 6, 8
    q, k, v = _inputs(b, hq, hkv, t, p, d, seed=3)
    q = q * 3  # wide score spread: most p far from 1
    rng = np.random.default_rng(4)
    masks = torch.from_numpy(np.stack([trees.ancestor_mask(trees.random_parents(t, rng)) for _ in range(b)]))
    out = dense_mask_attention(q, k, v, masks, p, p_dtype=p_dtype)
    plain = dense_mask_attention(q, k, v, masks, p)
    np.testing.assert_allclose(dense_mask_attention(q, k, v, masks, p, p_dtype=torch.float32).numpy(),
                               plain.numpy(), atol=1e-6, rtol=1e-6)
    ref = np.empty(out.shape)
    bound = np.empty(out.shape)
    mant = 8 if p_dtype == torch.bfloat16 else 11
    for bi in range(b):
        for h in range(hq):
            kv = h // (hq // hkv)
            for r in range(t):
                keys = list(range(p)) + [p + j for j in range(t) if masks[bi, r, j]]
                s = np.array([float(q[bi, h, r].double() @ k[bi, kv, j].double()) for j in keys]) / math.sqrt(d)
                pe = np.exp(s - s.max())
                pr = torch.from_numpy(pe).float().to(p_dtype).double().numpy()
                vv = v[bi, kv, keys].double().numpy()
                ref[bi, h, r] = pr @ vv / pe.sum()
                bound[bi, h, r] = 2.0 ** -mant * (pe @ np.abs(vv)) / pe.sum()
    np.testing.assert_allclose(out.numpy(), ref, atol=2e-6, rtol=1e-5)
    assert np.all(np.abs(out.numpy() - plain.numpy()) <= bound + 2e-6)
    assert np.abs(out.numpy() - plain.numpy()).max() > 0  # the rounding is visible
