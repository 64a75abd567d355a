"""Paged K/V forward on the GPU: tree_sparse_attention_fwd_paged vs the
contiguous forward and the fp32 oracle.

The paged kernel moves the same key rows into the same LDS slots as the
contiguous one (only the addresses differ), so its O must equal the
contiguous forward's bit for bit; the contiguous forward is held to the fp32
oracle in test_gpu_fwd.py, and the cases here check the paged output against
the oracle as well.  Pages are scattered over the pool in seeded random
order with unreferenced spare pages, and the prefix lengths include ones that
make 4- and 8-row loads straddle page boundaries.
"""

import numpy as np
import pytest
import torch

import tree_sparse_flashattn as tsf
from tsfa import configs, trees
from tests.gpu_util import assert_close_to_oracle, oracle_out, storage_roundings

pytestmark = pytest.mark.gpu

BF, FP = torch.bfloat16, torch.float16

CASES = [
    # b, hq, hkv, t, p, d, dtype, bm, bn, tree, page_size, layout, table
    (1, 4, 4, 128, 32, 64, BF, 64, 64, "random", 16, "NHD", "csr"),
    (1, 8, 2, 37, 100, 128, BF, 16, 16, "random", 16, "NHD", "csr"),    # P % 4 = 0 but P % 16 != 0
    (1, 8, 2, 37, 101, 128, FP, 16, 16, "random", 16, "HND", "csr"),    # P % 4 = 1: loads straddle pages
    (2, 8, 1, 50, 0, 128, FP, 16, 32, "eagle", 32, "HND", "dense"),     # no prefix, G = 8
    (1, 2, 2, 300, 7, 128, FP, 128, 64, "random", 64, "NHD", "dense"),  # several row chunks, P = 7
    (3, 6, 2, 20, 130, 64, BF, 16, 16, "depth", 16, "HND", "csr"),      # D = 64 (8-row loads), P % 8 = 2
    (2, 4, 2, 33, 61, 64, FP, 16, 16, "kary", 32, "NHD", "dense"),      # D = 64, P % 8 = 5
    (1, 16, 1, 200, 1000, 128, FP, 64, 32, "random", 256, "NHD", "csr"),
    (1, 32, 8, 64, 1, 128, BF, 16, 64, "eagle", 128, "NHD", "csr"),     # prefix of one key
    (2, 8, 2, 96, 2048, 128, BF, 64, 64, "random", 16, "NHD", "csr"),   # long prefix, P % 32 = 0
]


def _tree(kind, t, rng):
    if kind == "random":
        return trees.ancestor_mask(trees.random_parents(t, rng))
    if kind == "eagle":
        return trees.ancestor_mask(trees.eagle_parents(t, 5, 6, rng))
    if kind == "kary":
        return trees.ancestor_mask(trees.kary_bfs_parents(t, 3))
    return trees.ancestor_mask(trees.depth_limited_parents(t, 4, rng))


def _qkv(b, hq, hkv, t, p, d, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, hq, t, d, generator=g).to(dtype)
    k = torch.randn(b, hkv, p + t, d, generator=g).to(dtype)
    v = torch.randn(b, hkv, p + t, d, generator=g).to(dtype)
    return q, k, v


def _paged_vs_contiguous(q, k, v, meta, page_size, layout, dense, seed):
    dev = torch.device("cuda", 0)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    cache, indptr, indices = configs.make_paged_kv(kd, vd, page_size, layout=layout, seed=seed, spare_pages=3,
                                                   dense_table=dense)
    # both outputs (and the contiguous call's workspace) start as NaN, so a
    # work item that is skipped or mis-mapped cannot pass on a stale value
    ws = torch.full((max(tsf.fwd_workspace_bytes(qd, kd, meta), 1),), 0xFF, dtype=torch.uint8, device=dev)
    out_c = tsf.tree_sparse_attention_fwd(qd, kd, vd, meta, out=torch.full_like(qd, float("nan")), workspace=ws)
    out_p = tsf.tree_sparse_attention_fwd_paged(qd, cache, indices, meta, kv_len=k.shape[2], kv_indptr=indptr,
                                                kv_layout=layout, out=torch.full_like(qd, float("nan")))
    torch.cuda.synchronize()
    assert torch.equal(torch.isnan(out_p), torch.isnan(out_c))
    assert torch.equal(out_p.nan_to_num(0.0), out_c.nan_to_num(0.0)), \
        f"paged != contiguous: max diff {float((out_p.float() - out_c.float()).nan_to_num(0).abs().max()):.3e}"
    return out_p


@pytest.mark.parametrize("case", CASES, ids=[f"p{i}" for i in range(len(CASES))])
def test_paged_cases(case):
    b, hq, hkv, t, p, d, dtype, bm, bn, kind, ps, layout, table = case
    print(f"[paged] case {case}", flush=True)
    rng = np.random.default_rng(t * 31 + p)
    mask = torch.from_numpy(_tree(kind, t, rng))
    q, k, v = _qkv(b, hq, hkv, t, p, d, dtype, seed=t + p)
    meta = tsf.prepare_tree_sparse_metadata(mask.cuda(), p, bm, bn)
    out = _paged_vs_contiguous(q, k, v, meta, ps, layout, table == "dense", seed=t)
    assert_close_to_oracle(out, oracle_out(q, k, v, mask, p), dtype,
                           half_ulps=storage_roundings(q, k, p) if p < 256 else 0)


@pytest.mark.parametrize("case", [CASES[i] for i in (2, 4, 5, 9)], ids=["p2", "p4", "p5", "p9"])
def test_paged_one_stream_kernel(case, monkeypatch):
    monkeypatch.setenv("TSFA_STREAMS", "1")
    test_paged_cases(case)


@pytest.mark.parametrize("case", [CASES[i] for i in (0, 2, 4, 5, 7)], ids=["p0", "p2", "p4", "p5", "p7"])
def test_paged_64bit_offsets(case, monkeypatch):
    # caches below 4 GB take the 32-bit-offset kernel by default; this runs
    # the 64-bit one on the same cases
    monkeypatch.setenv("TSFA_PAGED32", "0")
    test_paged_cases(case)


# Runs of at least 32 units (one key stream, or two with a cache below
# 4 GB or writing O) take the instance that reads each run's page ids into
# an LDS table with Q and refills from it (head_dim 128); runs of 64 units
# (two runs and the combine) and of 128 with the tree folded in (one slot:
# the kernel writes O), pages of 16 (two per unit) and 64 keys, both cache
# layouts, CSR and dense page lists, 32- and 64-bit page offsets (the latter
# with partials: the general refill path).
@pytest.mark.parametrize("streams,ups,page_size,layout,dense,paged32", [
    ("1", 64, 16, "NHD", False, "1"), ("1", 128, 64, "HND", True, "1"), ("1", 128, 16, "HND", False, "1"),
    ("2", 64, 16, "NHD", False, "1"), ("2", 128, 32, "HND", True, "1"),
    ("2", 128, 16, "NHD", False, "0"), ("2", 64, 16, "NHD", False, "0")])
def test_paged_page_table_runs(streams, ups, page_size, layout, dense, paged32, monkeypatch):
    env = {"TSFA_STREAMS": streams, "TSFA_PREFIX_UNITS_PER_SPLIT": str(ups), "TSFA_PAGED32": paged32}
    if ups == 128:
        env["TSFA_FOLD_TREE"] = "1"
    for key, val in env.items():
        monkeypatch.setenv(key, val)
    b, hq, hkv, t, p, d, dtype = 2, 8, 2, 64, 4096, 128, BF
    print(f"[paged] page table streams {streams} ups {ups} page_size {page_size} {layout} dense {dense} "
          f"paged32 {paged32}", flush=True)
    rng = np.random.default_rng(ups + page_size)
    mask = torch.from_numpy(_tree("random", t, rng))
    q, k, v = _qkv(b, hq, hkv, t, p, d, dtype, seed=ups)
    meta = tsf.prepare_tree_sparse_metadata(mask.cuda(), p, 64, 64)
    out = _paged_vs_contiguous(q, k, v, meta, page_size, layout, dense, seed=page_size)
    assert_close_to_oracle(out, oracle_out(q, k, v, mask, p), dtype)



# A prefix with a partial last unit takes the unchecked steps on the paged
# kernels too (the page-id table where it applies): two streams over 32- and
# 64-bit offsets, with partials and one-slot (the kernel that writes O), and
# one stream; each bit-exact against the contiguous call and within the bar
# of the oracle.
@pytest.mark.parametrize("streams,ups,paged32,p", [
    ("2", 24, "1", 2047), ("2", 128, "0", 2017), ("2", 24, "0", 2047), ("1", 24, "0", 2017)])
def test_paged_partial_last_unit(streams, ups, paged32, p, monkeypatch):
    env = {"TSFA_STREAMS": streams, "TSFA_PREFIX_UNITS_PER_SPLIT": str(ups), "TSFA_PAGED32": paged32}
    if ups == 128:
        env["TSFA_FOLD_TREE"] = "1"
    for key, val in env.items():
        monkeypatch.setenv(key, val)
    b, hq, hkv, t, d, dtype = 2, 8, 2, 64, 128, BF
    print(f"[paged] partial last unit streams {streams} ups {ups} paged32 {paged32} p {p}", flush=True)
    rng = np.random.default_rng(p + ups)
    mask = torch.from_numpy(_tree("random", t, rng))
    q, k, v = _qkv(b, hq, hkv, t, p, d, dtype, seed=p)
    meta = tsf.prepare_tree_sparse_metadata(mask.cuda(), p, 64, 64)
    out = _paged_vs_contiguous(q, k, v, meta, 16, "NHD", False, seed=p)
    assert_close_to_oracle(out, oracle_out(q, k, v, mask, p), dtype)

@pytest.mark.parametrize("page_size", [16, 64])
def test_paged_workload_llama3_8b(page_size):
    w = configs.WORKLOADS["llama3-8b-eagle64-p4096"]
    print(f"[paged] {w.name} page_size {page_size}", flush=True)
    q, k, v = configs.make_qkv(w)
    mask = configs.make_tree_mask(w)
    meta = tsf.prepare_tree_sparse_metadata(mask.cuda(), w.prefix_len, w.block_m, w.block_n)
    out = _paged_vs_contiguous(q, k, v, meta, page_size, "NHD", False, seed=page_size)
    assert_close_to_oracle(out, oracle_out(q, k, v, mask, w.prefix_len), w.dtype)


def test_paged_per_sequence_trees():
    w = configs.WORKLOADS["batched-decode-b16-p2048"]
    print(f"[paged] {w.name}", flush=True)
    q, k, v = configs.make_qkv(w)
    mask = configs.make_tree_mask(w)
    meta = tsf.prepare_tree_sparse_metadata_batched(mask.cuda(), w.prefix_len, w.block_m, w.block_n)
    out = _paged_vs_contiguous(q, k, v, meta, 16, "HND", False, seed=3)
    # every row sees the prefix: the heads the oracle skips must be written too
    assert not torch.isnan(out).any()
    heads = (0, 7, 21, 31)
    ref = oracle_out(q, k, v, mask, w.prefix_len, heads=heads)
    assert_close_to_oracle(out, ref, w.dtype, heads=heads)


def test_paged_out_of_range_page_ids_are_clamped():
    # ids below 0 or past the pool read page 0 / the last page (never outside
    # the cache): O equals the forward over the host-clamped table
    b, hq, hkv, t, p, d = 2, 8, 2, 24, 90, 128
    rng = np.random.default_rng(9)
    mask = torch.from_numpy(_tree("random", t, rng))
    q, k, v = (x.cuda() for x in _qkv(b, hq, hkv, t, p, d, BF, seed=9))
    meta = tsf.prepare_tree_sparse_metadata(mask.cuda(), p, 16, 16)
    cache, indptr, indices = configs.make_paged_kv(k, v, 16, seed=4, spare_pages=2)
    n_pages = cache.shape[0]
    bad = indices.clone()
    bad[1], bad[4], bad[-1] = -5, n_pages + 100, 2 ** 31 - 1
    out_bad = tsf.tree_sparse_attention_fwd_paged(q, cache, bad, meta, kv_len=p + t, kv_indptr=indptr)
    out_ref = tsf.tree_sparse_attention_fwd_paged(q, cache, bad.clamp(0, n_pages - 1), meta, kv_len=p + t,
                                                  kv_indptr=indptr)
    torch.cuda.synchronize()
    assert torch.equal(out_bad.nan_to_num(0.0), out_ref.nan_to_num(0.0))


def test_paged_graph_capture_replays():
    w = configs.WORKLOADS["llama3-8b-eagle64-p4096"]
    q, k, v = (x.cuda() for x in configs.make_qkv(w))
    mask = configs.make_tree_mask(w).cuda()
    meta = tsf.prepare_tree_sparse_metadata(mask, w.prefix_len, w.block_m, w.block_n)
    cache, indptr, indices = configs.make_paged_kv(k, v, 16, seed=1)
    kv_len = k.shape[2]
    eager = tsf.tree_sparse_attention_fwd_paged(q, cache, indices, meta, kv_len=kv_len, kv_indptr=indptr)
    out = torch.empty_like(q)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):  # warm the allocator and the LDS attribute outside capture
        tsf.tree_sparse_attention_fwd_paged(q, cache, indices, meta, kv_len=kv_len, kv_indptr=indptr, out=out)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        tsf.tree_sparse_attention_fwd_paged(q, cache, indices, meta, kv_len=kv_len, kv_indptr=indptr, out=out)
    for i in range(3):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"


def test_paged_lse_matches_contiguous():
    b, hq, hkv, t, p, d = 2, 8, 2, 30, 77, 128
    mask = torch.from_numpy(_tree("random", t, np.random.default_rng(12)))
    q, k, v = (x.cuda() for x in _qkv(b, hq, hkv, t, p, d, BF, seed=12))
    meta = tsf.prepare_tree_sparse_metadata(mask.cuda(), p, 16, 16)
    cache, indptr, indices = configs.make_paged_kv(k, v, 32, seed=2)
    o_c, lse_c = tsf.tree_sparse_attention_fwd(q, k, v, meta, return_lse=True)
    o_p, lse_p = tsf.tree_sparse_attention_fwd_paged(q, cache, indices, meta, kv_len=p + t, kv_indptr=indptr,
                                                     return_lse=True)
    torch.cuda.synchronize()
    assert torch.equal(o_c, o_p) and torch.equal(lse_c, lse_p)
