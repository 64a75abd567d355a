"""Folded tree units, and block kinds other than MIXED.

When a row chunk's prefix run also runs the chunk's tree units (the folded
plan: one slot, whose kernel writes O, or several slots with the tree in the
last), the chunk's block states, visible tree units and mask words are built
after the run inside the same launch.  These cases run such plans against the
fp32 dense+mask oracle (per-sequence trees in capacity layout, BN 16 to 128,
FULL and MIXED blocks, FULL only with an empty offset array, chunks of more
than 64 CSR entries, runs of one step, 128-token q-blocks) and through
the paged cache, bit-exact against the contiguous call.

Also here: a block kind other than MIXED (1) is FULL, as in the reference
(tree_sparse_flashattn.py:313-318: only blk_type == 1 reads the bitset), in
every kernel that reads the metadata.
"""

import dataclasses

import numpy as np
import pytest
import torch

import tree_sparse_flashattn as tsf
from oracle.attn_grad_oracle import attention_grads
from tsfa import _lib, configs, trees
from tests.gpu_util import assert_close_to_oracle, oracle_out, storage_roundings
from tests.test_gpu_bwd import _check

pytestmark = pytest.mark.gpu

BF, FP = torch.bfloat16, torch.float16


def _tree(kind, t, rng):
    if kind == "random":
        return trees.ancestor_mask(trees.random_parents(t, rng))
    if kind == "eagle":
        return trees.ancestor_mask(trees.eagle_parents(t, 5, 6, rng))
    if kind == "chain":  # FULL blocks below the diagonal, MIXED on it
        return np.tril(np.ones((t, t), dtype=bool))
    if kind == "ones":  # every block FULL: no MIXED block, no offsets
        return np.ones((t, t), dtype=bool)
    return trees.ancestor_mask(trees.kary_bfs_parents(t, 3))


def _qkv(b, hq, hkv, t, p, d, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, hq, t, d, generator=g).to(dtype)
    k = torch.randn(b, hkv, p + t, d, generator=g).to(dtype)
    v = torch.randn(b, hkv, p + t, d, generator=g).to(dtype)
    return q, k, v


def _fwd_nan_filled(qd, kd, vd, meta):
    # O and the workspace start as NaN, so a skipped or mis-mapped row shows
    out = torch.full_like(qd, float("nan"))
    ws = torch.full((max(tsf.fwd_workspace_bytes(qd, kd, meta), 1),), 0xFF, dtype=torch.uint8, device=qd.device)
    return tsf.tree_sparse_attention_fwd(qd, kd, vd, meta, out=out, workspace=ws)


# folded tree, two key streams, one prefix run per chunk (more units per run
# than any prefix here holds): one slot, the kernel that writes O
ONE_SLOT = {"TSFA_FOLD_TREE": "1", "TSFA_STREAMS": "2", "TSFA_PREFIX_UNITS_PER_SPLIT": "4096"}

CASES = [
    # b, hq, hkv, t, p, dtype, bm, bn, tree, per-sequence trees
    (3, 8, 2, 64, 2048, BF, 16, 64, "eagle", True),   # the 16-sequence decode layout, 3 sequences
    (1, 8, 2, 96, 1024, FP, 64, 32, "random", False),
    (2, 4, 4, 100, 512, BF, 16, 128, "chain", False),  # G = 1, FULL and MIXED blocks, partial last unit
    (1, 8, 2, 64, 1024, BF, 16, 64, "ones", False),    # FULL blocks only, empty offset array
    (1, 2, 2, 512, 1024, FP, 16, 32, "chain", False),  # the last chunks hold > 64 CSR entries
    (1, 2, 2, 256, 512, BF, 128, 64, "random", False),  # 128 tokens of one q-block per chunk
    (2, 8, 2, 40, 64, FP, 16, 32, "kary", False),      # two prefix units: one step per run
]


@pytest.mark.parametrize("case", CASES, ids=[f"t{i}" for i in range(len(CASES))])
def test_folded_one_slot_plans(case, monkeypatch):
    b, hq, hkv, t, p, dtype, bm, bn, kind, per_seq = case
    # one run per chunk over the whole prefix: the one-slot plan
    for key, val in ONE_SLOT.items():
        monkeypatch.setenv(key, val)
    plan = _lib.fwd_plan(b, hq, hkv, t, p + t, p, 128)
    # the folded one-slot plan with rings that meet every step (4 stages of 2 streams)
    assert plan["fold_tree"] == 1 and plan["slots"] == 1 and plan["ring_stages"] == 4, plan
    print(f"[folded] case {case} plan {plan}", flush=True)
    rng = np.random.default_rng(t + p + bm)
    if per_seq:
        mask = torch.from_numpy(np.stack([_tree(kind, t, rng) for _ in range(b)]))
        meta = tsf.prepare_tree_sparse_metadata_batched(mask.cuda(), p, bm, bn)
    else:
        mask = torch.from_numpy(_tree(kind, t, rng))
        meta = tsf.prepare_tree_sparse_metadata(mask.cuda(), p, bm, bn)
    q, k, v = _qkv(b, hq, hkv, t, p, 128, dtype, seed=t + p)
    out = _fwd_nan_filled(q.cuda(), k.cuda(), v.cuda(), meta)
    torch.cuda.synchronize()
    assert_close_to_oracle(out, oracle_out(q, k, v, mask, p), dtype,
                           half_ulps=storage_roundings(q, k, p) if p < 256 else 0)


def test_folded_one_slot_paged(monkeypatch):
    # the paged kernel takes the same folded path (its tree units through the
    # page table); paged and contiguous agree bit for bit
    for key, val in ONE_SLOT.items():
        monkeypatch.setenv(key, val)
    b, hq, hkv, t, p, dtype, bm, bn = 3, 8, 2, 64, 2048, BF, 16, 64
    rng = np.random.default_rng(11)
    mask = torch.from_numpy(np.stack([_tree("eagle", t, rng) for _ in range(b)]))
    meta = tsf.prepare_tree_sparse_metadata_batched(mask.cuda(), p, bm, bn)
    q, k, v = _qkv(b, hq, hkv, t, p, 128, dtype, seed=5)
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    cache, indptr, indices = configs.make_paged_kv(kd, vd, 16, layout="NHD", seed=3, spare_pages=3)
    out_c = tsf.tree_sparse_attention_fwd(qd, kd, vd, meta)
    out_p = tsf.tree_sparse_attention_fwd_paged(qd, cache, indices, meta, kv_len=p + t, kv_indptr=indptr)
    torch.cuda.synchronize()
    assert torch.equal(out_p, out_c)
    assert_close_to_oracle(out_p, oracle_out(q, k, v, mask, p), dtype)


def test_folded_multi_slot_plans(monkeypatch):
    # folded plans of several slots: the tree units in the last run, partials
    # merged by the combine
    for key, val in {"TSFA_FOLD_TREE": "1", "TSFA_STREAMS": "2", "TSFA_PREFIX_UNITS_PER_SPLIT": "16"}.items():
        monkeypatch.setenv(key, val)
    b, hq, hkv, t, p, dtype, bm, bn = 2, 8, 2, 64, 1024, BF, 16, 64
    plan = _lib.fwd_plan(b, hq, hkv, t, p + t, p, 128)
    assert plan["fold_tree"] == 1 and plan["slots"] > 1, plan
    rng = np.random.default_rng(17)
    mask = torch.from_numpy(_tree("eagle", t, rng))
    meta = tsf.prepare_tree_sparse_metadata(mask.cuda(), p, bm, bn)
    q, k, v = _qkv(b, hq, hkv, t, p, 128, dtype, seed=17)
    out = _fwd_nan_filled(q.cuda(), k.cuda(), v.cuda(), meta)
    torch.cuda.synchronize()
    assert_close_to_oracle(out, oracle_out(q, k, v, mask, p), dtype)


def _with_kind_two(mask, meta, t, bm, bn, n_change, seed):
    """Metadata with n_change MIXED entries marked 2 (FULL for the reference)
    and the dense mask those blocks then stand for (clipped to the tree)."""
    bt = meta.blk_type.cpu().numpy().copy()
    rp = meta.row_ptr.cpu().numpy()
    ci = meta.col_idx.cpu().numpy()
    mixed = np.flatnonzero(bt == 1)
    assert mixed.size >= n_change
    pick = np.random.default_rng(seed).choice(mixed, n_change, replace=False)
    dense = mask.clone()
    for e in pick:
        bt[e] = 2
        qb = int(np.searchsorted(rp, e, side="right") - 1)
        tb = int(ci[e])
        dense[qb * bm:min(qb * bm + bm, t), tb * bn:min(tb * bn + bn, t)] = True
    changed = dataclasses.replace(meta, blk_type=torch.from_numpy(bt).to(meta.blk_type.device))
    as_full = bt.copy()
    as_full[pick] = 0
    full = dataclasses.replace(meta, blk_type=torch.from_numpy(as_full).to(meta.blk_type.device))
    return changed, full, dense


# the folded one-slot plan (BN 32), separate tree items,
# the generic kernel (head_dim 256) and the 64-wide kernel
@pytest.mark.parametrize("d,p,bn,fold", [(128, 2048, 32, "1"), (128, 300, 16, "0"), (256, 300, 16, None),
                                         (64, 100, 16, None)])
def test_block_kind_other_than_mixed_is_full(d, p, bn, fold, monkeypatch):
    if fold is not None:
        monkeypatch.setenv("TSFA_FOLD_TREE", fold)
    if fold == "1":
        monkeypatch.setenv("TSFA_PREFIX_UNITS_PER_SPLIT", ONE_SLOT["TSFA_PREFIX_UNITS_PER_SPLIT"])
    b, hq, hkv, t, bm, dtype = 1, 8, 2, 64, 16, BF
    rng = np.random.default_rng(d + p)
    mask = torch.from_numpy(_tree("random", t, rng))
    meta = tsf.prepare_tree_sparse_metadata(mask.cuda(), p, bm, bn)
    changed, full, dense = _with_kind_two(mask, meta, t, bm, bn, 3, seed=d)
    print(f"[kind] d={d} p={p} fold={fold}", flush=True)
    q, k, v = _qkv(b, hq, hkv, t, p, d, dtype, seed=p)
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    out2 = _fwd_nan_filled(qd, kd, vd, changed)
    out0 = _fwd_nan_filled(qd, kd, vd, full)
    torch.cuda.synchronize()
    assert torch.equal(out2, out0)
    assert_close_to_oracle(out2, oracle_out(q, k, v, dense, p), dtype,
                           half_ulps=storage_roundings(q, k, p) if p < 256 else 0)


def test_block_kind_other_than_mixed_is_full_backward():
    # against the gradient oracle with those blocks fully visible (dQ sums
    # its split tiles with atomics, so two runs need not agree bit for bit)
    b, hq, hkv, t, p, bm, bn, d, dtype = 1, 8, 2, 64, 200, 16, 16, 128, BF
    rng = np.random.default_rng(21)
    mask = torch.from_numpy(_tree("random", t, rng))
    meta = tsf.prepare_tree_sparse_metadata(mask.cuda(), p, bm, bn)
    changed, _, dense = _with_kind_two(mask, meta, t, bm, bn, 3, seed=4)
    q, k, v = _qkv(b, hq, hkv, t, p, d, dtype, seed=9)
    do = torch.randn(q.shape, generator=torch.Generator().manual_seed(2)).to(dtype)
    qd, kd, vd, dod = q.cuda(), k.cuda(), v.cuda(), do.cuda()
    o, lse = tsf.tree_sparse_attention_fwd(qd, kd, vd, changed, return_lse=True)
    dq, dk, dv = tsf.tree_sparse_attention_bwd(qd, kd, vd, o, lse, dod, changed)
    torch.cuda.synchronize()
    rq, rk, rv, _ = attention_grads(q, k, v, dense, p, do, head_chunk=8)
    for name, got, ref in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        _check(name, got, ref, dtype)
