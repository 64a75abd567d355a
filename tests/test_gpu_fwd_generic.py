"""head_dim 256 (bf16 / fp16) and fp32 inputs: the generic kernel against the
fp32 dense+mask oracle.

The reference takes any power-of-two BLOCK_D (tree_sparse_flashattn.py:
200-202, README.md:190) and any dtype tl.dot takes (fp32 included,
tree_sparse_flashattn.py:269, :278).  Bars: 8e-3 (bf16) / 2e-3 (fp16) as
the forward's parity bar states them, 1e-4 for fp32 (tests/gpu_util.py); O and the
workspace start NaN-filled so an unwritten row fails.
"""

import math

import numpy as np
import pytest
import torch

from tsfa import configs, trees
from tests.gpu_util import TOL, assert_close_to_oracle, oracle_out, storage_roundings

pytestmark = pytest.mark.gpu

import eagle_tree_sparse_bridge as bridge  # noqa: E402
import tree_sparse_flashattn as tsf  # noqa: E402


def _qkv(b, hq, hkv, t, p, d, dtype, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, hq, t, d, generator=g).to(dtype)
    k = torch.randn(b, hkv, p + t, d, generator=g).to(dtype)
    v = torch.randn(b, hkv, p + t, d, generator=g).to(dtype)
    return q, k, v


def _run_nan_filled(q, k, v, mask, prefix_len, bm, bn, return_lse=False):
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    build = tsf.prepare_tree_sparse_metadata_batched if mask.dim() == 3 else tsf.prepare_tree_sparse_metadata
    meta = build(mask.cuda(), prefix_len, bm, bn)
    out = torch.full_like(qd, float("nan"))
    ws = torch.full((max(tsf.fwd_workspace_bytes(qd, kd, meta), 1),), 0xFF, dtype=torch.uint8, device=qd.device)
    return tsf.tree_sparse_attention_fwd(qd, kd, vd, meta, out=out, workspace=ws, return_lse=return_lse)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_head_dim_256_at_the_llama3_8b_decode_shape(dtype):
    # the Llama-3-8B verification shape (32 / 8 heads, 4096-token prefix,
    # 64-node EAGLE tree, BLOCK_M 16, BLOCK_N 64) with head_dim 256
    w = configs.WORKLOADS["llama3-8b-eagle64-p4096"]
    print(f"[gen] head_dim 256 {dtype}", flush=True)
    q, k, v = _qkv(1, 32, 8, 64, 4096, 256, dtype, seed=42)
    mask = configs.make_tree_mask(w)
    out = _run_nan_filled(q, k, v, mask, 4096, 16, 64)
    torch.cuda.synchronize()
    assert not torch.isnan(out).any()
    err = assert_close_to_oracle(out, oracle_out(q, k, v, mask, 4096), dtype)
    print(f"[gen] head_dim 256 {dtype} max_abs_err {err:.3e}", flush=True)


def test_fp32_cpu_runnable_workload_on_the_gpu():
    # the CPU-runnable configuration (B=1, 4 / 4 heads, head_dim 64, prefix 32,
    # 128 random-parent tree tokens, fp32, BLOCK 64 x 64) on the device
    w = configs.WORKLOADS["tiny-random-tree-fp32"]
    print(f"[gen] {w.name}", flush=True)
    q, k, v = configs.make_qkv(w)
    mask = configs.make_tree_mask(w)
    out = _run_nan_filled(q, k, v, mask, w.prefix_len, w.block_m, w.block_n)
    torch.cuda.synchronize()
    assert out.dtype == torch.float32
    err = assert_close_to_oracle(out, oracle_out(q, k, v, mask, w.prefix_len), torch.float32)
    print(f"[gen] {w.name} max_abs_err {err:.3e}", flush=True)


CASES = [
    # b, hq, hkv, t, p, d, dtype, bm, bn, tree
    (1, 8, 2, 37, 100, 256, torch.bfloat16, 16, 16, "random"),   # T % BM != 0, P % 32 != 0
    (2, 6, 2, 50, 0, 256, torch.float16, 16, 32, "eagle"),       # no prefix, G = 3
    (1, 16, 1, 70, 1000, 256, torch.bfloat16, 64, 64, "random"),  # G = 16, several chunks
    (1, 4, 4, 128, 32, 64, torch.float32, 64, 64, "random"),
    (2, 8, 2, 45, 300, 128, torch.float32, 16, 32, "eagle"),
    (1, 6, 3, 33, 77, 256, torch.float32, 16, 16, "depth"),
    (1, 32, 8, 64, 1, 128, torch.float32, 16, 64, "eagle"),      # prefix of one key
]


def _tree(kind, t, rng):
    if kind == "random":
        return trees.ancestor_mask(trees.random_parents(t, rng))
    if kind == "eagle":
        return trees.ancestor_mask(trees.eagle_parents(t, 5, 6, rng))
    return trees.ancestor_mask(trees.depth_limited_parents(t, 4, rng))


@pytest.mark.parametrize("case", CASES, ids=[f"g{i}" for i in range(len(CASES))])
def test_generic_cases(case):
    b, hq, hkv, t, p, d, dtype, bm, bn, kind = case
    print(f"[gen] case {case}", flush=True)
    rng = np.random.default_rng(t * 31 + p + d)
    mask = torch.from_numpy(_tree(kind, t, rng))
    q, k, v = _qkv(b, hq, hkv, t, p, d, dtype, seed=t + p)
    out = _run_nan_filled(q, k, v, mask, p, bm, bn)
    torch.cuda.synchronize()
    assert_close_to_oracle(out, oracle_out(q, k, v, mask, p), dtype,
                           half_ulps=storage_roundings(q, k, p) if p < 256 and dtype != torch.float32 else 0)


@pytest.mark.parametrize("dtype,d", [(torch.bfloat16, 256), (torch.float32, 256)])
def test_long_tree_builds_its_words_in_the_loop(dtype, d):
    # 1100 tree tokens and no prefix: one split of 35 units, all with tree
    # columns, more than the prologue's LDS word table holds (32 units), so
    # the kernel instance that builds each unit's words in the loop runs
    t = 1100
    print(f"[gen] long tree {dtype} head_dim {d}", flush=True)
    rng = np.random.default_rng(d)
    mask = torch.from_numpy(_tree("depth", t, rng))
    q, k, v = _qkv(1, 4, 2, t, 0, d, dtype, seed=d + 1)
    out = _run_nan_filled(q, k, v, mask, 0, 64, 64)
    torch.cuda.synchronize()
    assert_close_to_oracle(out, oracle_out(q, k, v, mask, 0), dtype,
                           half_ulps=storage_roundings(q, k, 0) if dtype != torch.float32 else 0)


@pytest.mark.parametrize("dtype,d", [(torch.bfloat16, 256), (torch.float32, 64)])
def test_one_split_plans_write_o_directly(dtype, d, monkeypatch):
    # 16 sequences x 8 kv heads x 2 row chunks = 256 groups: one split, so
    # the kernel writes O itself; TSFA_DIRECT_OUT=0 keeps the partial (in
    # the input dtype; fp32 for fp32) and the combine, whose one-slot merge
    # (l * x) / l may move x by an fp32 ulp: the two agree within one ulp of
    # the output dtype
    b, hq, hkv, t, p = 16, 32, 8, 64, 200
    print(f"[gen] one split {dtype} head_dim {d}", flush=True)
    rng = np.random.default_rng(d + 3)
    masks = torch.from_numpy(np.stack([_tree("eagle", t, rng) for _ in range(b)]))
    masks[3, 5, :] = False  # a row with no visible tree key (the prefix still shows)
    q, k, v = _qkv(b, hq, hkv, t, p, d, dtype, seed=d + 5)
    outs = {}
    for direct in ("1", "0"):
        monkeypatch.setenv("TSFA_DIRECT_OUT", direct)
        outs[direct] = _run_nan_filled(q, k, v, masks, p, 16, 32)
        torch.cuda.synchronize()
    ref = oracle_out(q, k, v, masks, p)
    for direct, out in outs.items():
        assert_close_to_oracle(out, ref, dtype)
    a, c = outs["1"].float().cpu(), outs["0"].float().cpu()
    assert torch.equal(a.isnan(), c.isnan())
    from tests.gpu_util import half_ulp
    assert ((a - c).abs().nan_to_num(0) <= 2 * half_ulp(c, dtype) + 1e-30).all()


@pytest.mark.parametrize("dtype,d", [(torch.bfloat16, 256), (torch.float32, 128)])
def test_per_sequence_trees_and_lse(dtype, d):
    b, hq, hkv, t, p = 3, 8, 2, 40, 150
    rng = np.random.default_rng(d)
    masks = torch.from_numpy(np.stack([_tree("random", t, rng) for _ in range(b)]))
    q, k, v = _qkv(b, hq, hkv, t, p, d, dtype, seed=d)
    out, lse = _run_nan_filled(q, k, v, masks, p, 16, 32, return_lse=True)
    torch.cuda.synchronize()
    assert_close_to_oracle(out, oracle_out(q, k, v, masks, p), dtype,
                           half_ulps=storage_roundings(q, k, p) if dtype != torch.float32 else 0)
    # lse = log sum_j exp(s_j) over the row's visible keys, fp32
    kf, qf = k.float().repeat_interleave(hq // hkv, dim=1), q.float()
    s = torch.matmul(qf, kf.transpose(-2, -1)) / math.sqrt(d)
    vis = torch.ones(b, 1, t, p + t, dtype=torch.bool)
    vis[:, 0, :, p:] = masks
    ref_lse = torch.logsumexp(s.masked_fill(~vis, float("-inf")), dim=-1)
    assert (lse.cpu() - ref_lse).abs().max() < 1e-3


def test_identity_without_prefix_returns_v_in_fp32_and_head_dim_256():
    for dtype, d in ((torch.float32, 64), (torch.bfloat16, 256)):
        q, k, v = _qkv(1, 4, 2, 40, 0, d, dtype)
        out = bridge.run_tree_sparse_kernel(q.cuda(), k.cuda(), v.cuda(), torch.eye(40, dtype=torch.bool).cuda(),
                                            block_m=16, block_n=16)
        torch.cuda.synchronize()
        # a single visible key: p = 1, l = 1, O = V exactly
        torch.testing.assert_close(out.cpu(), v.repeat_interleave(2, dim=1), atol=0, rtol=0)


def test_empty_row_without_prefix_is_nan_in_fp32():
    q, k, v = _qkv(1, 2, 1, 20, 0, 128, torch.float32)
    mask = torch.eye(20, dtype=torch.bool)
    mask[5, 5] = False
    out = bridge.run_tree_sparse_kernel(q.cuda(), k.cuda(), v.cuda(), mask.cuda(), block_m=16, block_n=16)
    torch.cuda.synchronize()
    assert torch.isnan(out[0, :, 5]).all()
    assert not torch.isnan(out[0, :, :5]).any() and not torch.isnan(out[0, :, 6:]).any()


def test_reference_grid_launch_in_fp32_with_strided_views():
    # the raw launch of benchmark.py:182-194 with fp32 operands given as
    # [B, N, H, D] storage viewed as [B, H, N, D]
    B, H, HKV, D, P, Q = 2, 8, 2, 64, 200, 40
    g = torch.Generator().manual_seed(5)
    qs = torch.randn(B, Q, H, D, generator=g).cuda()
    ks = torch.randn(B, P + Q, HKV, D, generator=g).cuda()
    vs = torch.randn(B, P + Q, HKV, D, generator=g).cuda()
    q, k, v = qs.transpose(1, 2), ks.transpose(1, 2), vs.transpose(1, 2)
    mask = torch.tril(torch.ones(Q, Q, dtype=torch.bool)) & ~(torch.rand(Q, Q, generator=g) > 0.6)
    mask.fill_diagonal_(True)
    meta = tsf.prepare_tree_sparse_metadata(mask.cuda(), P, 16, 16)
    o = torch.full((B, Q, H, D), float("nan"), device="cuda").transpose(1, 2)
    tsf.block_sparse_tree_fwd_kernel[(meta.n_q_blocks, B * H)](
        q, k, v, o, meta.row_ptr, meta.col_idx, meta.blk_type, meta.mixed_mask_payload, meta.mixed_mask_offset,
        q.stride(0), q.stride(1), q.stride(2), q.stride(3), k.stride(0), k.stride(1), k.stride(2), k.stride(3),
        v.stride(0), v.stride(1), v.stride(2), v.stride(3), o.stride(0), o.stride(1), o.stride(2), o.stride(3),
        1.0 / math.sqrt(D), B, H, HKV, Q, P + Q, P, meta.n_q_blocks, meta.n_tree_blocks, H // HKV,
        BLOCK_M=16, BLOCK_N=16, BLOCK_D=D)
    torch.cuda.synchronize()
    assert_close_to_oracle(o, oracle_out(q.cpu(), k.cpu(), v.cpu(), mask, P), torch.float32)


@pytest.mark.parametrize("dtype,d", [(torch.bfloat16, 160), (torch.float16, 200), (torch.float32, 96)])
def test_head_dims_between_kernel_widths_run_zero_padded(dtype, d):
    # 160 / 200 run the head_dim 256 kernel, fp32 96 the fp32 128 one, on
    # zero-padded copies (zeros add nothing to q.k and give zero columns of O)
    print(f"[gen] padded {dtype} head_dim {d}", flush=True)
    rng = np.random.default_rng(d)
    mask = torch.from_numpy(_tree("eagle", 40, rng))
    q, k, v = _qkv(2, 8, 4, 40, 150, d, dtype, seed=d)
    out = tsf.tree_sparse_attention_fwd(q.cuda(), k.cuda(), v.cuda(),
                                        tsf.prepare_tree_sparse_metadata(mask.cuda(), 150, 16, 32))
    torch.cuda.synchronize()
    assert out.shape == q.shape
    assert_close_to_oracle(out, oracle_out(q, k, v, mask, 150), dtype,
                           half_ulps=storage_roundings(q, k, 150) if dtype != torch.float32 else 0)


def test_paged_and_backward_refuse_the_generic_shapes():
    q, k, v = (x.cuda() for x in _qkv(1, 4, 2, 16, 32, 256, torch.bfloat16))
    meta = tsf.prepare_tree_sparse_metadata(torch.eye(16, dtype=torch.bool).cuda(), 32, 16, 16)
    cache, indptr, indices = configs.make_paged_kv(k, v, 16)
    with pytest.raises(NotImplementedError):
        tsf.tree_sparse_attention_fwd_paged(q, cache, indices, meta, kv_len=k.shape[2], kv_indptr=indptr)
    o, lse = tsf.tree_sparse_attention_fwd(q, k, v, meta, return_lse=True)
    with pytest.raises(NotImplementedError):
        tsf.tree_sparse_attention_bwd(q, k, v, o, lse, torch.ones_like(o), meta)


def test_tolerances_declared():
    assert TOL[torch.float32] == 1e-4
