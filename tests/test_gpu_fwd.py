"""HIP tree-sparse forward vs the fp32 dense+mask oracle.

Bar (written per dtype in tests/gpu_util.py): max_abs_err <= 8e-3 (bf16),
<= 2e-3 (fp16) against the oracle computed in fp32 from the same inputs; NaN
exactly where the oracle is NaN (rows with no visible key).
"""

import math

import numpy as np
import pytest
import torch

from tsfa import configs, trees
from tests.gpu_util import MANT, TOL, assert_close_to_oracle, oracle_out, storage_roundings

pytestmark = pytest.mark.gpu

import eagle_tree_sparse_bridge as bridge  # noqa: E402
import tree_sparse_flashattn as tsf  # noqa: E402


def _qkv(b, hq, hkv, t, p, d, dtype, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, hq, t, d, generator=g).to(dtype)
    k = torch.randn(b, hkv, p + t, d, generator=g).to(dtype)
    v = torch.randn(b, hkv, p + t, d, generator=g).to(dtype)
    return q, k, v


def _run(q, k, v, mask, bm, bn):
    return bridge.run_tree_sparse_kernel(q.cuda(), k.cuda(), v.cuda(), mask.cuda(), block_m=bm, block_n=bn)


def _run_nan_filled(q, k, v, mask, prefix_len, bm, bn):
    # O and the split-KV workspace start as NaN (every byte 0xFF), so a work
    # item that is mis-mapped or skipped leaves NaN in O instead of a stale
    # but correct value from an earlier call
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    build = tsf.prepare_tree_sparse_metadata_batched if mask.dim() == 3 else tsf.prepare_tree_sparse_metadata
    meta = build(mask.cuda(), prefix_len, bm, bn)
    out = torch.full_like(qd, float("nan"))
    ws = torch.full((max(tsf.fwd_workspace_bytes(qd, kd, meta), 1),), 0xFF, dtype=torch.uint8, device=qd.device)
    return tsf.tree_sparse_attention_fwd(qd, kd, vd, meta, out=out, workspace=ws)


@pytest.mark.parametrize("name", ["llama3-8b-eagle64-p4096", "batched-decode-b16-p2048"])
def test_workload_full(name):
    w = configs.WORKLOADS[name]
    print(f"[fwd] {name}", flush=True)
    q, k, v = configs.make_qkv(w)
    mask = configs.make_tree_mask(w)
    out = _run_nan_filled(q, k, v, mask, w.prefix_len, w.block_m, w.block_n)
    torch.cuda.synchronize()
    err = assert_close_to_oracle(out, oracle_out(q, k, v, mask, w.prefix_len), w.dtype)
    print(f"[fwd] {name} max_abs_err {err:.3e}", flush=True)


def _heads_per_kv(w, shift=0):
    # one query head of every kv head: query head g*kvh + (kvh + shift) % g
    g = w.q_heads // w.kv_heads
    return tuple(g * h + (h + shift) % g for h in range(w.kv_heads))


@pytest.mark.parametrize("name", ["wide-tree-1024-p16384", "llama3-70b-b4-p32768"])
def test_workload_heads_of_every_kv_head(name):
    # one query head of each kv head, every sequence, against the oracle; the
    # rest of O must be finite (NaN-filled O and workspace beforehand)
    w = configs.WORKLOADS[name]
    heads = _heads_per_kv(w)
    print(f"[fwd] {name} heads {heads}", flush=True)
    q, k, v = configs.make_qkv(w)
    mask = configs.make_tree_mask(w)
    out = _run_nan_filled(q, k, v, mask, w.prefix_len, w.block_m, w.block_n)
    torch.cuda.synchronize()
    assert not torch.isnan(out).any()
    err = assert_close_to_oracle(out, oracle_out(q, k, v, mask, w.prefix_len, heads=heads), w.dtype, heads=heads)
    print(f"[fwd] {name} max_abs_err {err:.3e} (bar {TOL[w.dtype]:.0e})", flush=True)


@pytest.mark.parametrize("block_m,block_n", [(64, 32), (64, 128), (16, 64)])
def test_workload_70b_block_sweep(block_m, block_n):
    # the 70B-layout workload swept over BLOCK_N in {32, 64, 128} and BLOCK_M
    # in {16, 64}; (64, 64) runs above
    w = configs.WORKLOADS["llama3-70b-b4-p32768"]
    heads = _heads_per_kv(w, shift=3)
    print(f"[fwd] {w.name} BLOCK_M {block_m} BLOCK_N {block_n} heads {heads}", flush=True)
    q, k, v = configs.make_qkv(w)
    mask = configs.make_tree_mask(w)
    out = _run_nan_filled(q, k, v, mask, w.prefix_len, block_m, block_n)
    torch.cuda.synchronize()
    assert not torch.isnan(out).any()
    err = assert_close_to_oracle(out, oracle_out(q, k, v, mask, w.prefix_len, heads=heads), w.dtype, heads=heads)
    print(f"[fwd] {w.name} BLOCK_M {block_m} BLOCK_N {block_n} max_abs_err {err:.3e}", flush=True)


CASES = [
    # b, hq, hkv, t, p, d, dtype, bm, bn, tree
    (1, 4, 4, 128, 32, 64, torch.bfloat16, 64, 64, "random"),     # the CPU-runnable shape, on MFMA
    (1, 4, 4, 128, 32, 64, torch.float16, 64, 64, "random"),
    (1, 8, 2, 37, 100, 128, torch.bfloat16, 16, 16, "random"),    # T % BM != 0, P % 64 != 0
    (2, 8, 1, 50, 0, 128, torch.float16, 16, 32, "eagle"),        # no prefix, G = 8
    (1, 4, 2, 64, 64, 64, torch.bfloat16, 32, 128, "kary"),       # BN > tile
    (1, 2, 2, 300, 7, 128, torch.float16, 128, 64, "random"),     # several row chunks
    (3, 6, 2, 20, 130, 64, torch.bfloat16, 16, 16, "depth"),      # G = 3
    (1, 16, 1, 200, 1000, 128, torch.float16, 64, 32, "random"),  # G = 16, tpc = 16
    (1, 32, 8, 64, 1, 128, torch.bfloat16, 16, 64, "eagle"),      # prefix of one key
]


def _tree(kind, t, rng):
    if kind == "random":
        return trees.ancestor_mask(trees.random_parents(t, rng))
    if kind == "eagle":
        return trees.ancestor_mask(trees.eagle_parents(t, 5, 6, rng))
    if kind == "kary":
        return trees.ancestor_mask(trees.kary_bfs_parents(t, 3))
    return trees.ancestor_mask(trees.depth_limited_parents(t, 4, rng))


@pytest.mark.parametrize("case", CASES, ids=[f"c{i}" for i in range(len(CASES))])
def test_cases(case):
    b, hq, hkv, t, p, d, dtype, bm, bn, kind = case
    print(f"[fwd] case {case}", flush=True)
    rng = np.random.default_rng(t * 31 + p)
    mask = torch.from_numpy(_tree(kind, t, rng))
    q, k, v = _qkv(b, hq, hkv, t, p, d, dtype, seed=t + p)
    out = _run(q, k, v, mask, bm, bn)
    torch.cuda.synchronize()
    # short prefixes leave rows with few keys and |O| ~ 1-4: one storage rounding beyond the bar
    assert_close_to_oracle(out, oracle_out(q, k, v, mask, p), dtype,
                           half_ulps=storage_roundings(q, k, p) if p < 256 else 0)


# The planner's other kernels and load flavours, forced through its
# environment switches: the 8-wave kernel with one key stream or two (the
# planner picks two below 1024 rows per (batch, kv head)), the K/V loads with
# and without the non-temporal hint (chosen by the row-chunk count), the
# three dispatch orders of the work items, and the tree units run by their own
# workgroup or by the last prefix run of each chunk.
KERNELS = {"one-stream": {"TSFA_STREAMS": "1"}, "two-streams": {"TSFA_STREAMS": "2"},
           "kv-nt": {"TSFA_KV_NT": "1"}, "kv-temporal": {"TSFA_KV_NT": "0"},
           "items-natural": {"TSFA_ITEM_ORDER": "0"}, "items-tree-first": {"TSFA_ITEM_ORDER": "2"},
           "tree-folded": {"TSFA_FOLD_TREE": "1"}, "tree-separate": {"TSFA_FOLD_TREE": "0"},
           "one-stream-tree-folded": {"TSFA_STREAMS": "1", "TSFA_FOLD_TREE": "1"}}


@pytest.mark.parametrize("kernel", sorted(KERNELS))
@pytest.mark.parametrize("case", [CASES[i] for i in (0, 2, 3, 5, 7, 8)], ids=[f"c{i}" for i in (0, 2, 3, 5, 7, 8)])
def test_cases_other_kernels(case, kernel, monkeypatch):
    for key, val in KERNELS[kernel].items():
        monkeypatch.setenv(key, val)
    b, hq, hkv, t, p, d, dtype, bm, bn, kind = case
    print(f"[fwd] {kernel} case {case}", flush=True)
    rng = np.random.default_rng(t * 31 + p)
    mask = torch.from_numpy(_tree(kind, t, rng))
    q, k, v = _qkv(b, hq, hkv, t, p, d, dtype, seed=t + p)
    out = _run(q, k, v, mask, bm, bn)
    torch.cuda.synchronize()
    assert_close_to_oracle(out, oracle_out(q, k, v, mask, p), dtype,
                           half_ulps=storage_roundings(q, k, p) if p < 256 else 0)


def _assert_same_steps(fast, checked, d):
    # The unchecked and checked steps run the same arithmetic in the same
    # order, but as separately compiled loops: at head_dim 64 with two key
    # streams one fp32 multiply-add can be contracted in one loop and not in
    # the other, moving an element of O by one storage step (seen: one
    # element of 196608, 0.02710 against 0.02722, each path deterministic).
    # Head_dim 128 is bit-exact.
    assert torch.equal(torch.isnan(fast), torch.isnan(checked))
    if d == 128:
        assert torch.equal(fast, checked)
        return
    a, b = fast.float().nan_to_num(0.0), checked.float().nan_to_num(0.0)
    step = torch.finfo(fast.dtype).eps * torch.maximum(a.abs(), b.abs())
    assert bool(((a - b).abs() <= step).all()), f"max diff {float((a - b).abs().max()):.3e}"


# A prefix whose length is a multiple of 32 takes the kernel with unchecked
# prefix ring steps (one key stream or two; with two, its non-temporal
# flavour too).  The runs here are 24, 24 and 16 units (a shorter last run),
# so the steady ring steps and the checked tail both run; the result must
# equal the checked kernel's (_assert_same_steps) and match the oracle.
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("streams,nt", [("1", "0"), ("2", "0"), ("2", "1")])
def test_fast_ring_matches_checked_steps(d, streams, nt, monkeypatch):
    b, hq, hkv, t, p, dtype = 2, 8, 2, 96, 2048, torch.bfloat16
    for key, val in {"TSFA_STREAMS": streams, "TSFA_KV_NT": nt, "TSFA_PREFIX_UNITS_PER_SPLIT": "24"}.items():
        monkeypatch.setenv(key, val)
    print(f"[fwd] fast ring d={d} streams={streams} nt={nt}", flush=True)
    rng = np.random.default_rng(d)
    mask = torch.from_numpy(_tree("random", t, rng))
    q, k, v = _qkv(b, hq, hkv, t, p, d, dtype, seed=d)
    outs = {}
    for fast in ("1", "0"):
        monkeypatch.setenv("TSFA_FAST_RING", fast)
        outs[fast] = _run_nan_filled(q, k, v, mask, p, 64, 64)
        torch.cuda.synchronize()
    _assert_same_steps(outs["1"], outs["0"], d)
    assert_close_to_oracle(outs["1"], oracle_out(q, k, v, mask, p), dtype)


# A prefix whose length is not a multiple of 32 takes the unchecked steps too
# when its last, partial unit lies within kv_len: that unit is the last of
# its run, and its keys past the prefix are masked after the loop.  Runs of
# 24 units (the partial one in the last run), one-slot plans (the kernel that
# writes O), and a tree too short to fill the last unit (the checked steps,
# by the host's test); every result equals the checked kernel's
# (_assert_same_steps) and matches the oracle.
@pytest.mark.parametrize("d,streams,nt,p,t,one_slot", [
    (128, "2", "1", 2047, 96, False), (128, "2", "0", 2017, 96, False), (128, "1", "0", 2047, 96, False),
    (64, "2", "0", 2033, 96, False), (64, "1", "0", 2017, 96, False),
    (128, "2", "1", 2017, 64, True), (128, "1", "0", 1025, 64, True),
    (128, "2", "1", 2017, 16, False)])  # 2017 + 16 < 2048: the checked steps
def test_fast_ring_partial_last_unit(d, streams, nt, p, t, one_slot, monkeypatch):
    b, hq, hkv, dtype = 2, 8, 2, torch.bfloat16
    env = {"TSFA_STREAMS": streams, "TSFA_KV_NT": nt}
    if one_slot:
        env.update({"TSFA_FOLD_TREE": "1", "TSFA_PREFIX_UNITS_PER_SPLIT": "4096"})
    else:
        env["TSFA_PREFIX_UNITS_PER_SPLIT"] = "24"
    for key, val in env.items():
        monkeypatch.setenv(key, val)
    print(f"[fwd] fast ring, partial last unit d={d} streams={streams} nt={nt} p={p} t={t} one_slot={one_slot}",
          flush=True)
    rng = np.random.default_rng(p + d)
    mask = torch.from_numpy(_tree("random", t, rng))
    q, k, v = _qkv(b, hq, hkv, t, p, d, dtype, seed=p)
    outs = {}
    for fast in ("1", "0"):
        monkeypatch.setenv("TSFA_FAST_RING", fast)
        outs[fast] = _run_nan_filled(q, k, v, mask, p, 64, 64)
        torch.cuda.synchronize()
    _assert_same_steps(outs["1"], outs["0"], d)
    assert_close_to_oracle(outs["1"], oracle_out(q, k, v, mask, p), dtype)


# A plan of one slot (one prefix run per chunk with the tree folded in, or
# the tree alone) writes O from the split kernel and skips the combine; the
# result must equal the combine's bit for bit (a one-slot merge returns the
# partial) and match the oracle.  Two streams with non-temporal loads and one
# stream with plain ones.
@pytest.mark.parametrize("streams,nt,p", [("2", "1", 512), ("1", "0", 512), ("2", "1", 0), ("1", "0", 1024)])
def test_one_slot_direct_output_matches_combine(streams, nt, p, monkeypatch):
    b, hq, hkv, t, dtype = 3, 8, 2, 40, torch.float16
    env = {"TSFA_STREAMS": streams, "TSFA_KV_NT": nt, "TSFA_FOLD_TREE": "1"}
    if p:
        env["TSFA_PREFIX_UNITS_PER_SPLIT"] = str(p // 32)
    for key, val in env.items():
        monkeypatch.setenv(key, val)
    print(f"[fwd] one-slot direct output streams={streams} nt={nt} p={p}", flush=True)
    rng = np.random.default_rng(p + int(streams))
    mask = torch.from_numpy(_tree("kary", t, rng))
    q, k, v = _qkv(b, hq, hkv, t, p, 64 if streams == "1" else 128, dtype, seed=p + 7)
    outs = {}
    for direct in ("1", "0"):
        monkeypatch.setenv("TSFA_DIRECT_OUT", direct)
        outs[direct] = _run_nan_filled(q, k, v, mask, p, 16, 32)
        torch.cuda.synchronize()
    assert torch.equal(outs["1"], outs["0"])
    assert_close_to_oracle(outs["1"], oracle_out(q, k, v, mask, p), dtype,
                           half_ulps=storage_roundings(q, k, p) if p < 256 else 0)


@pytest.mark.parametrize("kernel", sorted(KERNELS))
def test_workload_other_kernels(kernel, monkeypatch):
    for key, val in KERNELS[kernel].items():
        monkeypatch.setenv(key, val)
    w = configs.WORKLOADS["llama3-8b-eagle64-p4096"]
    print(f"[fwd] {kernel} {w.name}", flush=True)
    q, k, v = configs.make_qkv(w)
    mask = configs.make_tree_mask(w)
    out = _run_nan_filled(q, k, v, mask, w.prefix_len, w.block_m, w.block_n)
    torch.cuda.synchronize()
    assert_close_to_oracle(out, oracle_out(q, k, v, mask, w.prefix_len), w.dtype)


@pytest.mark.parametrize("fold", [None, "1"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_per_sequence_trees(dtype, fold, monkeypatch):
    if fold is not None:  # the tree units run by the last prefix run of each chunk
        monkeypatch.setenv("TSFA_FOLD_TREE", fold)
    b, hq, hkv, t, p, d = 3, 8, 2, 45, 70, 128
    rng = np.random.default_rng(3)
    masks = torch.from_numpy(np.stack([_tree("random", t, rng) for _ in range(b)]))
    q, k, v = _qkv(b, hq, hkv, t, p, d, dtype)
    out = _run(q, k, v, masks, 16, 32)
    torch.cuda.synchronize()
    assert_close_to_oracle(out, oracle_out(q, k, v, masks, p), dtype, half_ulps=storage_roundings(q, k, p))


def test_all_full_blocks_no_offsets():
    # all-ones tree: every block FULL, empty mixed_mask_offset
    q, k, v = _qkv(1, 4, 2, 64, 96, 128, torch.bfloat16)
    mask = torch.ones(64, 64, dtype=torch.bool)
    meta = tsf.prepare_tree_sparse_metadata(mask.cuda(), 96, 16, 16)
    assert meta.mixed_mask_offset.numel() == 0
    out = _run(q, k, v, mask, 16, 16)
    torch.cuda.synchronize()
    assert_close_to_oracle(out, oracle_out(q, k, v, mask, 96), torch.bfloat16)


def test_identity_without_prefix_returns_v():
    q, k, v = _qkv(1, 4, 2, 40, 0, 64, torch.float16)
    out = _run(q, k, v, torch.eye(40, dtype=torch.bool), 16, 16)
    torch.cuda.synchronize()
    # single visible key: O = V exactly (p = 1, l = 1)
    torch.testing.assert_close(out.cpu(), v.repeat_interleave(2, dim=1), atol=0, rtol=0)


def test_empty_row_without_prefix_is_nan():
    q, k, v = _qkv(1, 2, 1, 20, 0, 64, torch.bfloat16)
    mask = torch.eye(20, dtype=torch.bool)
    mask[5, 5] = False
    out = _run(q, k, v, mask, 16, 16)
    torch.cuda.synchronize()
    assert torch.isnan(out[0, :, 5].float()).all()
    assert not torch.isnan(out[0, :, :5].float()).any() and not torch.isnan(out[0, :, 6:].float()).any()


def test_reference_grid_launch_and_strided_inputs():
    # The raw launch of benchmark.py:182-194 (B=2, 32/8 heads, D=128, P=1024,
    # T=64, BM=BN=16, fp16, tril with random branch dropout and the diagonal
    # set), with q/k/v/o given as [B, N, H, D] storage viewed as [B, H, N, D].
    B, H, HKV, D, P, Q = 2, 32, 8, 128, 1024, 64
    g = torch.Generator().manual_seed(42)
    qs = torch.randn(B, Q, H, D, generator=g).half().cuda()
    ks = torch.randn(B, P + Q, HKV, D, generator=g).half().cuda()
    vs = torch.randn(B, P + Q, HKV, D, generator=g).half().cuda()
    q, k, v = qs.transpose(1, 2), ks.transpose(1, 2), vs.transpose(1, 2)
    mask = torch.tril(torch.ones(Q, Q, dtype=torch.bool)) & ~(torch.rand(Q, Q, generator=g) > 0.6)
    mask.fill_diagonal_(True)
    meta = tsf.prepare_tree_sparse_metadata(mask.cpu(), P, 16, 16)
    meta.row_ptr, meta.col_idx, meta.blk_type = meta.row_ptr.cuda(), meta.col_idx.cuda(), meta.blk_type.cuda()
    meta.mixed_mask_payload, meta.mixed_mask_offset = meta.mixed_mask_payload.cuda(), meta.mixed_mask_offset.cuda()
    o = torch.empty(B, Q, H, D, dtype=torch.float16, device="cuda").transpose(1, 2)
    grid = (meta.n_q_blocks, B * H)
    tsf.block_sparse_tree_fwd_kernel[grid](
        q, k, v, o, meta.row_ptr, meta.col_idx, meta.blk_type, meta.mixed_mask_payload, meta.mixed_mask_offset,
        q.stride(0), q.stride(1), q.stride(2), q.stride(3), k.stride(0), k.stride(1), k.stride(2), k.stride(3),
        v.stride(0), v.stride(1), v.stride(2), v.stride(3), o.stride(0), o.stride(1), o.stride(2), o.stride(3),
        1.0 / math.sqrt(D), B, H, HKV, Q, P + Q, P, meta.n_q_blocks, meta.n_tree_blocks, H // HKV,
        BLOCK_M=16, BLOCK_N=16, BLOCK_D=D, num_warps=4, num_stages=2)
    torch.cuda.synchronize()
    assert_close_to_oracle(o, oracle_out(q.cpu(), k.cpu(), v.cpu(), mask, P), torch.float16)


def _grid_launch(q, k, v, o, meta, P, D, bm, bn):
    B, H, Q = q.shape[0], q.shape[1], q.shape[2]
    HKV = k.shape[1]
    tsf.block_sparse_tree_fwd_kernel[(meta.n_q_blocks, B * H)](
        q, k, v, o, meta.row_ptr, meta.col_idx, meta.blk_type, meta.mixed_mask_payload, meta.mixed_mask_offset,
        q.stride(0), q.stride(1), q.stride(2), q.stride(3), k.stride(0), k.stride(1), k.stride(2), k.stride(3),
        v.stride(0), v.stride(1), v.stride(2), v.stride(3), o.stride(0), o.stride(1), o.stride(2), o.stride(3),
        1.0 / math.sqrt(D), B, H, HKV, Q, k.shape[2], P, meta.n_q_blocks, meta.n_tree_blocks, H // HKV,
        BLOCK_M=bm, BLOCK_N=bn, BLOCK_D=D)


@pytest.mark.parametrize("layout", ["d-stride-2", "unaligned-rows", "o-d-stride-2"])
def test_reference_grid_launch_layouts_the_kernel_does_not_address(layout):
    # every d stride and row alignment the reference takes
    # (tree_sparse_flashattn.py:174-189): copied to dense operands, O
    # written back through a temporary
    B, H, HKV, D, P, Q = 1, 8, 2, 64, 96, 40
    g = torch.Generator().manual_seed(3)
    rng = np.random.default_rng(3)
    mask = torch.from_numpy(_tree("random", Q, rng))
    if layout == "d-stride-2":
        q = torch.randn(B, H, Q, 2 * D, generator=g).bfloat16().cuda()[..., ::2]
        k = torch.randn(B, HKV, P + Q, 2 * D, generator=g).bfloat16().cuda()[..., ::2]
        v = torch.randn(B, HKV, P + Q, 2 * D, generator=g).bfloat16().cuda()[..., ::2]
    else:
        q, k, v = (x.cuda() for x in _qkv(B, H, HKV, Q, P, D, torch.bfloat16, seed=3))
    if layout == "unaligned-rows":
        # rows of 65 elements, a base one element past an allocation's start
        def shift(t):
            buf = torch.zeros(t.numel() // D * 65 + 1, dtype=t.dtype, device=t.device)
            view = buf[1:].as_strided(t.shape, (t.shape[1] * t.shape[2] * 65, t.shape[2] * 65, 65, 1))
            view.copy_(t)
            return view
        q, k, v = shift(q), shift(k), shift(v)
    if layout == "o-d-stride-2":
        o = torch.full((B, H, Q, 2 * D), float("nan"), dtype=torch.bfloat16, device="cuda")[..., ::2]
    else:
        o = torch.full((B, H, Q, D), float("nan"), dtype=torch.bfloat16, device="cuda")
    meta = tsf.prepare_tree_sparse_metadata(mask.cuda(), P, 16, 16)
    _grid_launch(q, k, v, o, meta, P, D, 16, 16)
    torch.cuda.synchronize()
    err = assert_close_to_oracle(o, oracle_out(q.cpu(), k.cpu(), v.cpu(), mask, P), torch.bfloat16,
                                 half_ulps=storage_roundings(q, k, P))
    print(f"[fwd] grid launch {layout} max_abs_err {err:.3e}", flush=True)


@pytest.mark.parametrize("d", [16, 32, 96])
def test_head_dims_below_a_kernel_width(d):
    # the reference takes any power-of-two BLOCK_D (README.md:190): head dims
    # below 64 / 128 run zero-padded (zeros add nothing to q.k; O sliced)
    B, H, HKV, P, Q = 2, 4, 2, 70, 33
    rng = np.random.default_rng(d)
    mask = torch.from_numpy(_tree("eagle", Q, rng))
    q, k, v = (x.cuda() for x in _qkv(B, H, HKV, Q, P, d, torch.float16, seed=d))
    meta = tsf.prepare_tree_sparse_metadata(mask.cuda(), P, 16, 16)
    o = torch.full_like(q, float("nan"))
    _grid_launch(q, k, v, o, meta, P, d, 16, 16)
    out = tsf.tree_sparse_attention_fwd(q, k, v, meta)
    torch.cuda.synchronize()
    ref = oracle_out(q.cpu(), k.cpu(), v.cpu(), mask, P)
    assert_close_to_oracle(o, ref, torch.float16, half_ulps=storage_roundings(q, k, P))
    assert_close_to_oracle(out, ref, torch.float16, half_ulps=storage_roundings(q, k, P))
    assert out.shape == q.shape


def test_head_dim_above_the_widest_kernel_raises():
    q, k, v = (x.cuda() for x in _qkv(1, 2, 2, 8, 8, 512, torch.bfloat16))
    with pytest.raises(NotImplementedError):
        _run(q, k, v, torch.eye(8, dtype=torch.bool), 16, 16)


def test_repeat_calls_are_deterministic():
    w = configs.WORKLOADS["llama3-8b-eagle64-p4096"]
    q, k, v = (x.cuda() for x in configs.make_qkv(w))
    mask = configs.make_tree_mask(w).cuda()
    a = bridge.run_tree_sparse_kernel(q, k, v, mask, block_m=w.block_m, block_n=w.block_n)
    b = bridge.run_tree_sparse_kernel(q, k, v, mask, block_m=w.block_m, block_n=w.block_n)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", [torch.float64])
def test_unsupported_dtype_raises(dtype):
    q, k, v = _qkv(1, 2, 2, 8, 8, 64, dtype)
    with pytest.raises(NotImplementedError):
        _run(q, k, v, torch.eye(8, dtype=torch.bool), 16, 16)


def test_tolerances_declared():
    assert TOL[torch.bfloat16] == 8e-3 and TOL[torch.float16] == 2e-3
    assert MANT[torch.bfloat16] == 8 and MANT[torch.float16] == 11
