"""Gradient oracle for tree-sparse attention (dQ, dK, dV and the row LSE).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

The reference has no backward (README.md:198 lists it as missing), so there
is no reference code to restate: the oracle is the textbook gradient of the
function the reference's forward computes (tree_sparse_flashattn.py:163-339,
restated densely at benchmark.py:8-35), with z = scale * q.k over the row's
visible keys (prefix [0, P) plus the tree keys of the row's mask row):

    P = softmax(z),  O = P V,  lse = logsumexp(z)
    dV = P^T dO,  dP = dO V^T,  dS = P * (dP - rowsum(dO * O))
    dQ = scale * dS K,  dK = scale * dS^T Q

summed over the G query heads that share a kv head.  ``attention_grads``
evaluates these closed forms in float32 on the CPU (chunked over heads);
``brute_force_grads`` is an independent float64 formulation for tiny shapes
(torch autograd through an explicit per-row gather).  Both are pinned by
finite differences (torch.autograd.gradcheck) in tests/test_oracle_grad.py.
Rows with no visible key (lse = -inf) contribute nothing to any gradient and
get dQ = 0.
"""

from __future__ import annotations

import math

import torch

from .attn_oracle import _full_mask


def attention_grads(q, k, v, tree_mask, prefix_len: int, dout, *, scale: float | None = None,
                    head_chunk: int | None = None):
    """(dq, dk, dv, lse) in float32 on the CPU for O = tree-sparse attention(q, k, v).

    q, dout [B, Hq, T, D]; k, v [B, Hkv, P+T, D]; tree_mask [T, T] or [B, T, T];
    lse [B, Hq, T] is the natural-log log-sum-exp of the scaled visible scores.
    """
    q, k, v, do = (x.detach().to("cpu", torch.float32) for x in (q, k, v, dout))
    bsz, n_heads, q_len, head_dim = q.shape
    _, n_kv_heads, kv_len, _ = k.shape
    group = n_heads // n_kv_heads
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)
    mask = _full_mask(tree_mask, bsz, q_len, kv_len, prefix_len)
    chunk = n_heads if head_chunk is None else max(1, int(head_chunk))
    dq = torch.zeros_like(q)
    dk = torch.zeros_like(k)
    dv = torch.zeros_like(v)
    lse = torch.empty((bsz, n_heads, q_len), dtype=torch.float32)
    for h0 in range(0, n_heads, chunk):
        h1 = min(n_heads, h0 + chunk)
        kv_idx = torch.arange(h0, h1) // group
        ke, ve = k[:, kv_idx], v[:, kv_idx]
        z = torch.matmul(q[:, h0:h1], ke.transpose(-2, -1).contiguous()) * scale
        z = z.masked_fill(~mask, float("-inf"))
        m = torch.logsumexp(z, dim=-1, keepdim=True)               # -inf for a row with no key
        empty = torch.isinf(m) & (m < 0)
        p = torch.where(empty, torch.zeros_like(z), torch.exp(z - m.masked_fill(empty, 0.0)))
        o = torch.matmul(p, ve)
        dop = do[:, h0:h1]
        dvec = (dop * o).sum(-1, keepdim=True)
        dp = torch.matmul(dop, ve.transpose(-2, -1).contiguous())
        ds = p * (dp - dvec)
        dq[:, h0:h1] = scale * torch.matmul(ds, ke)
        dk_e = scale * torch.matmul(ds.transpose(-2, -1).contiguous(), q[:, h0:h1])
        dv_e = torch.matmul(p.transpose(-2, -1).contiguous(), dop)
        dk.index_add_(1, kv_idx, dk_e)
        dv.index_add_(1, kv_idx, dv_e)
        lse[:, h0:h1] = m.squeeze(-1)
    return dq, dk, dv, lse


def brute_force_grads(q, k, v, tree_mask, prefix_len: int, dout, *, scale: float | None = None):
    """float64 (dq, dk, dv, lse) by autograd through a per-row gather of the visible keys.

    Tiny shapes only; rows with no visible key are skipped (they touch nothing)."""
    q = q.detach().to("cpu", torch.float64).requires_grad_(True)
    k = k.detach().to("cpu", torch.float64).requires_grad_(True)
    v = v.detach().to("cpu", torch.float64).requires_grad_(True)
    do = dout.detach().to("cpu", torch.float64)
    tm = tree_mask.detach().cpu().to(torch.bool)
    bsz, n_heads, q_len, head_dim = q.shape
    group = n_heads // k.shape[1]
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)
    lse = torch.full((bsz, n_heads, q_len), float("-inf"), dtype=torch.float64)
    total = torch.zeros((), dtype=torch.float64)
    for b in range(bsz):
        tmb = tm if tm.ndim == 2 else tm[b]
        for h in range(n_heads):
            kvh = h // group
            for t in range(q_len):
                keys = list(range(prefix_len)) + [prefix_len + j for j in range(q_len) if bool(tmb[t, j])]
                if not keys:
                    continue
                idx = torch.tensor(keys)
                z = scale * (k[b, kvh, idx] @ q[b, h, t])
                w = torch.softmax(z, dim=0)
                total = total + torch.dot(w @ v[b, kvh, idx], do[b, h, t])
                lse[b, h, t] = torch.logsumexp(z, dim=0).detach()
    total.backward()
    return q.grad, k.grad, v.grad, lse
