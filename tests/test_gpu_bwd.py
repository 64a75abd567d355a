"""HIP backward (tree_sparse_attention_bwd) and the forward's row LSE vs the
fp32 gradient oracle (oracle/attn_grad_oracle.py).

Bar: for each of dQ, dK, dV, max |got - ref| <= GRAD_REL[dtype] * max |ref|
+ GRAD_ABS[dtype], with ref computed in fp32 from the same (bf16 / fp16)
inputs.  The kernel rounds P and dS to the input dtype before their MFMAs
(2^-9 relative for bf16, 2^-12 for fp16) and, like any FlashAttention
backward, takes rowsum(dO * O) from the forward's O rounded to the input
dtype; those roundings, summed over up to a few thousand keys / rows, bound
the error.  LSE: |got - ref| <= 1e-3 (scores are exact fp32 products of the
rounded inputs).
"""

import math

import numpy as np
import pytest
import torch

import tree_sparse_flashattn as tsf
from oracle.attn_grad_oracle import attention_grads
from tsfa import configs, trees

pytestmark = pytest.mark.gpu

# Measured worst cases over the cases below: 5.5e-3 (bf16) and 6.4e-4 (fp16)
# of max |ref|, i.e. ~3 roundings of the input dtype; the bar is about twice
# that.
GRAD_REL = {torch.bfloat16: 1.2e-2, torch.float16: 1.5e-3}
GRAD_ABS = {torch.bfloat16: 1e-4, torch.float16: 2e-5}
BF, FP = torch.bfloat16, torch.float16


def _tree(kind, t, rng):
    if kind == "random":
        return trees.ancestor_mask(trees.random_parents(t, rng))
    if kind == "eagle":
        return trees.ancestor_mask(trees.eagle_parents(t, 5, 6, rng))
    if kind == "kary":
        return trees.ancestor_mask(trees.kary_bfs_parents(t, 3))
    return trees.ancestor_mask(trees.depth_limited_parents(t, 4, rng))


def _inputs(b, hq, hkv, t, p, d, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, hq, t, d, generator=g).to(dtype)
    k = torch.randn(b, hkv, p + t, d, generator=g).to(dtype)
    v = torch.randn(b, hkv, p + t, d, generator=g).to(dtype)
    do = torch.randn(b, hq, t, d, generator=g).to(dtype)
    return q, k, v, do


def _check(name, got, ref, dtype):
    got = got.float().cpu()
    assert torch.isfinite(got).all(), f"{name}: non-finite values"
    scale = float(ref.abs().max())
    err = float((got - ref).abs().max())
    bound = GRAD_REL[dtype] * scale + GRAD_ABS[dtype]
    print(f"[bwd] {name}: max_abs_err {err:.3e} (max|ref| {scale:.3e}, rel {err / max(scale, 1e-30):.2e})",
          flush=True)
    assert err <= bound, f"{name}: max_abs_err {err:.3e} > {bound:.3e}"


def _run_and_check(q, k, v, do, mask, p, bm, bn, dtype, sm_scale=None, batched=False):
    dev = torch.device("cuda", 0)
    qd, kd, vd, dod = (x.to(dev) for x in (q, k, v, do))
    if batched:
        meta = tsf.prepare_tree_sparse_metadata_batched(mask.to(dev), p, bm, bn)
    else:
        meta = tsf.prepare_tree_sparse_metadata(mask.to(dev), p, bm, bn)
    o, lse = tsf.tree_sparse_attention_fwd(qd, kd, vd, meta, sm_scale=sm_scale, return_lse=True)
    # the gradients start as NaN, so a work item that is skipped or mapped to
    # the wrong rows / keys (keys no row sees included: their dK, dV are 0)
    # leaves NaN for _check to find instead of a stale correct value
    dq, dk, dv = (torch.full_like(x, float("nan")) for x in (qd, kd, vd))
    got = tsf.tree_sparse_attention_bwd(qd, kd, vd, o, lse, dod, meta, sm_scale=sm_scale, dq=dq, dk=dk, dv=dv)
    assert all(g is x for g, x in zip(got, (dq, dk, dv)))
    torch.cuda.synchronize()
    rq, rk, rv, rlse = attention_grads(q, k, v, mask, p, do, scale=sm_scale, head_chunk=8)
    fin = torch.isfinite(rlse)
    lse_c = lse.cpu()
    assert torch.equal(torch.isfinite(lse_c), fin)
    assert float((lse_c[fin] - rlse[fin]).abs().max()) <= 1e-3
    _check("dq", dq, rq, dtype)
    _check("dk", dk, rk, dtype)
    _check("dv", dv, rv, dtype)
    return dq, dk, dv


CASES = [
    # b, hq, hkv, t, p, d, dtype, bm, bn, tree
    (1, 4, 4, 128, 32, 64, BF, 64, 64, "random"),
    (1, 4, 4, 128, 32, 64, FP, 64, 64, "random"),
    (1, 8, 2, 37, 100, 128, BF, 16, 16, "random"),    # T % BM != 0, P % 128 != 0
    (2, 8, 1, 50, 0, 128, FP, 16, 32, "eagle"),       # no prefix, G = 8
    (1, 4, 2, 64, 64, 64, BF, 32, 128, "kary"),
    (1, 2, 2, 300, 7, 128, FP, 128, 64, "random"),    # several tree key blocks, 10 row tiles
    (3, 6, 2, 20, 130, 64, BF, 16, 16, "depth"),      # G = 3
    (1, 16, 1, 200, 1000, 128, FP, 64, 32, "random"),  # G = 16: 100 row tiles
    (1, 32, 8, 64, 1, 128, BF, 16, 64, "eagle"),
]


@pytest.mark.parametrize("case", CASES, ids=[f"c{i}" for i in range(len(CASES))])
def test_bwd_cases(case):
    b, hq, hkv, t, p, d, dtype, bm, bn, kind = case
    print(f"[bwd] case {case}", flush=True)
    rng = np.random.default_rng(t * 31 + p)
    mask = torch.from_numpy(_tree(kind, t, rng))
    q, k, v, do = _inputs(b, hq, hkv, t, p, d, dtype, seed=t + p)
    _run_and_check(q, k, v, do, mask, p, bm, bn, dtype)


def test_bwd_workload_llama3_8b():
    w = configs.WORKLOADS["llama3-8b-eagle64-p4096"]
    print(f"[bwd] {w.name}", flush=True)
    q, k, v = configs.make_qkv(w)
    do = torch.randn(q.shape, generator=torch.Generator().manual_seed(7)).to(w.dtype)
    mask = configs.make_tree_mask(w)
    _run_and_check(q, k, v, do, mask, w.prefix_len, w.block_m, w.block_n, w.dtype)


@pytest.mark.parametrize("dtype", [BF, FP])
def test_bwd_per_sequence_trees(dtype):
    b, hq, hkv, t, p, d = 3, 8, 2, 45, 70, 128
    rng = np.random.default_rng(3)
    mask = torch.from_numpy(np.stack([_tree("random", t, rng) for _ in range(b)]))
    q, k, v, do = _inputs(b, hq, hkv, t, p, d, dtype, seed=11)
    _run_and_check(q, k, v, do, mask, p, 16, 16, dtype, batched=True)


def test_bwd_negative_scale():
    b, hq, hkv, t, p, d = 1, 4, 2, 40, 50, 128
    mask = torch.from_numpy(_tree("eagle", t, np.random.default_rng(2)))
    q, k, v, do = _inputs(b, hq, hkv, t, p, d, BF, seed=5)
    _run_and_check(q, k, v, do, mask, p, 16, 16, BF, sm_scale=-0.05)


def test_bwd_empty_rows_contribute_nothing():
    # no prefix and an identity tree with one hole: row 5 sees no key
    b, hq, hkv, t, d = 1, 4, 2, 24, 64
    mask = torch.eye(t, dtype=torch.bool)
    mask[5, 5] = False
    q, k, v, do = _inputs(b, hq, hkv, t, 0, d, BF, seed=9)
    dq, dk, dv = _run_and_check(q, k, v, do, mask, 0, 16, 16, BF)
    assert float(dq[:, :, 5].abs().max()) == 0.0
    assert float(dk[:, :, 5].abs().max()) == 0.0 and float(dv[:, :, 5].abs().max()) == 0.0


def test_autograd_function_matches_direct_call():
    b, hq, hkv, t, p, d = 1, 8, 2, 32, 64, 128
    mask = torch.from_numpy(_tree("random", t, np.random.default_rng(4)))
    q, k, v, do = (x.cuda() for x in _inputs(b, hq, hkv, t, p, d, BF, seed=4))
    meta = tsf.prepare_tree_sparse_metadata(mask.cuda(), p, 16, 16)
    qg, kg, vg = (x.clone().requires_grad_(True) for x in (q, k, v))
    out = tsf.tree_sparse_attention(qg, kg, vg, meta)
    out.backward(do)
    o, lse = tsf.tree_sparse_attention_fwd(q, k, v, meta, return_lse=True)
    dq, dk, dv = tsf.tree_sparse_attention_bwd(q, k, v, o, lse, do, meta)
    torch.cuda.synchronize()
    assert torch.equal(out.detach(), o)
    # dQ sums fp32 atomics in a run-dependent order: equal within rounding
    torch.testing.assert_close(qg.grad, dq, rtol=1e-2, atol=1e-3)
    assert torch.equal(kg.grad, dk) and torch.equal(vg.grad, dv)


def test_lse_matches_plain_forward_output():
    # return_lse does not change O
    b, hq, hkv, t, p, d = 2, 8, 2, 30, 90, 128
    mask = torch.from_numpy(_tree("random", t, np.random.default_rng(6)))
    q, k, v, _ = (x.cuda() for x in _inputs(b, hq, hkv, t, p, d, BF, seed=6))
    meta = tsf.prepare_tree_sparse_metadata(mask.cuda(), p, 16, 16)
    o1 = tsf.tree_sparse_attention_fwd(q, k, v, meta)
    o2, _ = tsf.tree_sparse_attention_fwd(q, k, v, meta, return_lse=True)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)


def test_bwd_sync_free_batched_metadata():
    # the bridge's capacity-layout record (no host sync), one tree per sequence
    import eagle_tree_sparse_bridge as bridge
    b, hq, hkv, t, p, d = 2, 8, 2, 40, 96, 128
    rng = np.random.default_rng(21)
    mask = torch.from_numpy(np.stack([_tree("eagle", t, rng) for _ in range(b)]))
    q, k, v, do = _inputs(b, hq, hkv, t, p, d, BF, seed=21)
    meta = bridge.build_tree_metadata(mask.cuda(), p, 16, 64)
    qd, kd, vd, dod = (x.cuda() for x in (q, k, v, do))
    o, lse = tsf.tree_sparse_attention_fwd(qd, kd, vd, meta, return_lse=True)
    dq, dk, dv = tsf.tree_sparse_attention_bwd(qd, kd, vd, o, lse, dod, meta)
    torch.cuda.synchronize()
    rq, rk, rv, _ = attention_grads(q, k, v, mask, p, do)
    _check("dq", dq, rq, BF)
    _check("dk", dk, rk, BF)
    _check("dv", dv, rv, BF)


def test_bwd_graph_capture_replays():
    b, hq, hkv, t, p, d = 1, 8, 2, 48, 200, 128
    mask = torch.from_numpy(_tree("random", t, np.random.default_rng(22)))
    q, k, v, do = (x.cuda() for x in _inputs(b, hq, hkv, t, p, d, BF, seed=22))
    meta = tsf.prepare_tree_sparse_metadata(mask.cuda(), p, 16, 16)
    o, lse = tsf.tree_sparse_attention_fwd(q, k, v, meta, return_lse=True)
    eager = tsf.tree_sparse_attention_bwd(q, k, v, o, lse, do, meta)
    dq, dk, dv = (torch.empty_like(x) for x in (q, k, v))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):  # warm the allocator and the LDS attributes outside capture
        tsf.tree_sparse_attention_bwd(q, k, v, o, lse, do, meta, dq=dq, dk=dk, dv=dv)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        tsf.tree_sparse_attention_bwd(q, k, v, o, lse, do, meta, dq=dq, dk=dk, dv=dv)
    for i in range(3):
        for x in (dq, dk, dv):
            x.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        # dK / dV have a fixed summation order; dQ sums fp32 atomics of the key splits
        assert torch.equal(dk, eager[1]) and torch.equal(dv, eager[2]), f"replay {i}"
        torch.testing.assert_close(dq, eager[0], rtol=1e-2, atol=1e-3)


def test_bwd_two_streams_at_once(monkeypatch):
    # each caller stream gets its own side stream for the dQ kernel: two
    # backward calls in flight on two streams give the single-stream results
    b, hq, hkv, t, p, d = 1, 32, 8, 64, 1024, 128
    mask = torch.from_numpy(_tree("eagle", t, np.random.default_rng(5)))
    meta = tsf.prepare_tree_sparse_metadata(mask.cuda(), p, 16, 64)
    ins = []
    for seed in (31, 32):
        q, k, v, do = (x.cuda() for x in _inputs(b, hq, hkv, t, p, d, BF, seed=seed))
        o, lse = tsf.tree_sparse_attention_fwd(q, k, v, meta, return_lse=True)
        ins.append((q, k, v, o, lse, do))
    with monkeypatch.context() as m:
        m.setenv("TSFA_BWD_CONCURRENT", "0")
        refs = [tsf.tree_sparse_attention_bwd(*x, meta) for x in ins]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    outs = [[], []]
    for _ in range(8):
        for j in (0, 1):
            with torch.cuda.stream(streams[j]):
                outs[j].append(tsf.tree_sparse_attention_bwd(*ins[j], meta))
    torch.cuda.synchronize()
    for j in (0, 1):
        for dq, dk, dv in outs[j]:
            assert torch.equal(dk, refs[j][1]) and torch.equal(dv, refs[j][2])
            torch.testing.assert_close(dq, refs[j][0], rtol=1e-2, atol=1e-3)
