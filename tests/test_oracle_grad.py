"""Pins the gradient oracle (oracle/attn_grad_oracle.py).

The reference has no backward, so nothing can be restated from it: the
closed forms are checked against finite differences (gradcheck, float64),
against an independent autograd formulation, and against special cases the
mathematics fixes (a single visible key: dV = dO exactly and dQ = dK = 0; a
uniform row: the LSE is the log of the key count)."""

import math

import numpy as np
import pytest
import torch

from oracle.attn_grad_oracle import attention_grads, brute_force_grads
from oracle.attn_oracle import dense_mask_attention
from tsfa import trees


def _inputs(b, hq, hkv, t, p, d, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, hq, t, d, generator=g, dtype=torch.float64)
    k = torch.randn(b, hkv, p + t, d, generator=g, dtype=torch.float64)
    v = torch.randn(b, hkv, p + t, d, generator=g, dtype=torch.float64)
    do = torch.randn(b, hq, t, d, generator=g, dtype=torch.float64)
    return q, k, v, do


def _mask(t, seed):
    return torch.from_numpy(trees.ancestor_mask(trees.random_parents(t, np.random.default_rng(seed))))


def _dense64(q, k, v, mask, p, scale):
    """float64 differentiable dense+mask attention (the forward the oracle differentiates)."""
    b, hq, t, d = q.shape
    group = hq // k.shape[1]
    ke = k.repeat_interleave(group, dim=1)
    ve = v.repeat_interleave(group, dim=1)
    full = torch.zeros((t, k.shape[2]), dtype=torch.bool)
    full[:, :p] = True
    full[:, p:] = mask
    z = (q @ ke.transpose(-2, -1)) * scale
    z = z.masked_fill(~full, float("-inf"))
    return torch.softmax(z, dim=-1) @ ve


def test_brute_force_matches_finite_differences():
    q, k, v, do = _inputs(1, 2, 1, 5, 3, 4, seed=1)
    mask = _mask(5, 1)
    scale = 0.37
    f = lambda q_, k_, v_: (_dense64(q_, k_, v_, mask, 3, scale) * do).sum()
    assert torch.autograd.gradcheck(f, (q.clone().requires_grad_(), k.clone().requires_grad_(),
                                        v.clone().requires_grad_()))
    qq, kk, vv = (x.clone().requires_grad_() for x in (q, k, v))
    f(qq, kk, vv).backward()
    bq, bk, bv, _ = brute_force_grads(q, k, v, mask, 3, do, scale=scale)
    for got, ref in ((bq, qq.grad), (bk, kk.grad), (bv, vv.grad)):
        torch.testing.assert_close(got, ref, rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("b,hq,hkv,t,p,d", [(1, 2, 2, 6, 4, 8), (2, 4, 2, 7, 0, 4), (1, 6, 2, 5, 9, 8)])
def test_closed_forms_match_brute_force(b, hq, hkv, t, p, d):
    q, k, v, do = _inputs(b, hq, hkv, t, p, d, seed=t + p)
    mask = _mask(t, t) if b == 1 else torch.stack([_mask(t, s) for s in range(b)])
    dq, dk, dv, lse = attention_grads(q, k, v, mask, p, do)
    bq, bk, bv, blse = brute_force_grads(q, k, v, mask, p, do)
    for got, ref in ((dq, bq), (dk, bk), (dv, bv), (lse, blse)):
        torch.testing.assert_close(got.double(), ref, rtol=2e-5, atol=2e-5)


def test_forward_consistency():
    # O recomputed from the oracle's P reproduces the forward oracle
    q, k, v, do = _inputs(1, 4, 2, 9, 5, 8, seed=3)
    mask = _mask(9, 3)
    _, _, _, lse = attention_grads(q, k, v, mask, 5, do)
    o = dense_mask_attention(q, k, v, mask, 5)
    # lse against an explicit log-sum-exp of the visible scaled scores of row (0, 0, t)
    for t in range(9):
        keys = list(range(5)) + [5 + j for j in range(9) if mask[t, j]]
        z = (k[0, 0, keys] @ q[0, 0, t]) / math.sqrt(8)
        assert abs(float(torch.logsumexp(z, 0)) - float(lse[0, 0, t])) < 1e-5
    assert torch.isfinite(o).all()


def test_single_visible_key_special_case():
    # P = 0 prefix and an identity tree: each row sees only itself, P = 1, so
    # O = V, dV = dO (summed over the group), dQ = dK = 0 and lse = the score
    q, k, v, do = _inputs(1, 2, 1, 4, 0, 8, seed=5)
    mask = torch.eye(4, dtype=torch.bool)
    dq, dk, dv, lse = attention_grads(q, k, v, mask, 0, do)
    assert float(dq.abs().max()) == 0.0 and float(dk.abs().max()) < 1e-6
    torch.testing.assert_close(dv[0, 0].double(), (do[0, 0] + do[0, 1]), rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(lse[0, 0].double(), (q[0, 0] * k[0, 0]).sum(-1) / math.sqrt(8), rtol=1e-6, atol=1e-6)


def test_uniform_row_lse_is_log_count():
    # zero queries: every visible score is 0, so lse = log(#visible keys)
    q, k, v, do = _inputs(1, 1, 1, 6, 10, 4, seed=2)
    q.zero_()
    mask = _mask(6, 2)
    _, _, _, lse = attention_grads(q, k, v, mask, 10, do)
    counts = 10 + mask.sum(-1)
    torch.testing.assert_close(lse[0, 0].double(), torch.log(counts.double()), rtol=1e-6, atol=1e-6)


def test_empty_rows_contribute_nothing():
    q, k, v, do = _inputs(1, 2, 2, 4, 0, 4, seed=8)
    mask = torch.eye(4, dtype=torch.bool)
    mask[2, 2] = False  # row 2 sees no key
    dq, dk, dv, lse = attention_grads(q, k, v, mask, 0, do)
    assert torch.isneginf(lse[0, :, 2]).all()
    assert float(dq[0, :, 2].abs().max()) == 0.0
    assert float(dv[0, :, 2].abs().max()) == 0.0  # key 2 is seen by nobody
