"""Bridge path on the GPU: sync-free metadata (a whole call captured in a HIP
graph and replayed), metadata reuse across calls, one tree broadcast over the
batch, lazily read counts.  Outputs are compared bit-for-bit with the eager
path and with the fp32 oracle at the dtype's bar."""

import numpy as np
import pytest
import torch

from oracle import meta_oracle
from tsfa import trees
from tests.gpu_util import assert_close_to_oracle, oracle_out

pytestmark = pytest.mark.gpu

import eagle_tree_sparse_bridge as bridge  # noqa: E402
import tree_sparse_flashattn as tsf  # noqa: E402


def _inputs(b=2, hq=8, hkv=2, t=64, p=300, d=128, dtype=torch.bfloat16, seed=0):
    rng = np.random.default_rng(seed)
    mask = torch.from_numpy(trees.ancestor_mask(trees.eagle_parents(t, 5, 6, rng)))
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, hq, t, d, generator=g).to(dtype)
    k = torch.randn(b, hkv, p + t, d, generator=g).to(dtype)
    v = torch.randn(b, hkv, p + t, d, generator=g).to(dtype)
    return q, k, v, mask


def test_whole_call_captures_in_a_graph_and_replays():
    print("[bridge] graph capture", flush=True)
    q, k, v, mask = _inputs()
    qd, kd, vd, md = q.cuda(), k.cuda(), v.cuda(), mask.cuda()
    bm, bn = 16, 64
    eager = bridge.run_tree_sparse_kernel(qd, kd, vd, md, block_m=bm, block_n=bn)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        bridge.run_tree_sparse_kernel(qd, kd, vd, md, block_m=bm, block_n=bn)  # warm-up on the side stream
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            out = bridge.run_tree_sparse_kernel(qd, kd, vd, md, block_m=bm, block_n=bn)
    torch.cuda.synchronize()
    for rep in range(3):
        qd.copy_(torch.roll(q, shifts=rep, dims=2).cuda())  # new inputs between replays
        ref = bridge.run_tree_sparse_kernel(qd, kd, vd, md, block_m=bm, block_n=bn)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {rep} differs from the eager call"
    assert torch.equal(eager, bridge.run_tree_sparse_kernel(q.cuda(), kd, vd, md, block_m=bm, block_n=bn))


def test_metadata_reused_across_calls_matches_per_call_builds():
    print("[bridge] metadata reuse", flush=True)
    q, k, v, mask = _inputs(seed=3)
    md = mask.cuda()
    meta = bridge.build_tree_metadata(md, k.shape[2] - q.shape[2], 16, 64)
    for layer in range(3):  # "layers": new q/k/v, one metadata
        ql, kl, vl = (x.cuda() * (1.0 + 0.25 * layer) for x in (q, k, v))
        a = bridge.run_tree_sparse_kernel(ql, kl, vl, md, block_m=16, block_n=64)
        b = bridge.run_tree_sparse_kernel(ql, kl, vl, None, block_m=16, block_n=64, metadata=meta)
        torch.cuda.synchronize()
        assert torch.equal(a, b)
    with pytest.raises(ValueError):
        bridge.run_tree_sparse_kernel(q.cuda(), k.cuda(), v.cuda(), None, block_m=16, block_n=32, metadata=meta)
    with pytest.raises(ValueError):
        bridge.run_tree_sparse_kernel(q.cuda(), k[:, :, 1:].cuda(), v[:, :, 1:].cuda(), None, block_m=16,
                                      block_n=64, metadata=meta)


def test_cache_builds_once_per_mask_and_geometry():
    print("[bridge] cache", flush=True)
    q, k, v, mask = _inputs(seed=5)
    qd, kd, vd, md = q.cuda(), k.cuda(), v.cuda(), mask.cuda()
    p = k.shape[2] - q.shape[2]
    cache = bridge.TreeSparseMetadataCache()
    outs = []
    for _ in range(4):
        meta = cache.get(md, (p, 16, 64), lambda: bridge.build_tree_metadata(md, p, 16, 64))
        outs.append(bridge.run_tree_sparse_kernel(qd, kd, vd, None, block_m=16, block_n=64, metadata=meta))
    torch.cuda.synchronize()
    assert cache.builds == 1 and cache.hits == 3
    assert all(torch.equal(outs[0], o) for o in outs[1:])
    err = assert_close_to_oracle(outs[0], oracle_out(q, k, v, mask, p), torch.bfloat16)
    print(f"[bridge] cache max_abs_err {err:.3e}", flush=True)


def test_one_tree_broadcast_equals_reference_record():
    print("[bridge] broadcast", flush=True)
    q, k, v, mask = _inputs(b=3, seed=7, dtype=torch.float16)
    qd, kd, vd, md = q.cuda(), k.cuda(), v.cuda(), mask.cuda()
    p = k.shape[2] - q.shape[2]
    one = tsf.prepare_tree_sparse_metadata_batched(md, p, 16, 32)
    assert one.n_trees == 1
    ref_meta = tsf.prepare_tree_sparse_metadata(md, p, 16, 32)
    a = tsf.tree_sparse_attention_fwd(qd, kd, vd, one)
    b = tsf.tree_sparse_attention_fwd(qd, kd, vd, ref_meta)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    # lazily read counts agree with the reference-shaped record and the oracle
    om = meta_oracle.build_metadata(mask.numpy(), p, 16, 32)
    assert one.nnz == [ref_meta.col_idx.numel()] == [om.col_idx.size]
    assert one.n_mixed == [int((om.blk_type == 1).sum())]
    seq = one.sequence(0)
    for f in ("row_ptr", "col_idx", "blk_type", "mixed_mask_payload", "mixed_mask_offset"):
        assert np.array_equal(getattr(seq, f).cpu().numpy(), getattr(om, f)), f


# ------------------------------------------------------------ model shims
from tests import llama_mock  # noqa: E402
from tests.gpu_util import TOL  # noqa: E402


def _module(cls, heads=8, kv_heads=2, head_dim=64, seed=0):
    torch.manual_seed(seed)
    m = cls(heads * head_dim, heads, kv_heads, head_dim)
    with torch.no_grad():
        m.o_proj.weight.copy_(torch.eye(heads * head_dim))  # the attention output itself
    return m.to(device="cuda", dtype=torch.bfloat16)


def test_flex_verify_uses_the_tree_kernel_and_one_build_serves_every_layer():
    print("[bridge] flex shim", flush=True)
    mod = llama_mock.make_module()
    bridge.patch_llama_flex_attention(mod, block_m=16, block_n=64)
    b, q_len, p, heads, kvh, d = 2, 64, 200, 8, 2, 64
    rng = np.random.default_rng(11)
    tree = torch.from_numpy(trees.ancestor_mask(trees.eagle_parents(q_len, 5, 6, rng)))
    mask = llama_mock.additive_mask(tree, p, b, torch.bfloat16).cuda()
    g = torch.Generator().manual_seed(4)
    h = torch.randn(b, q_len, heads * d, generator=g).to(torch.bfloat16).cuda()
    pos = torch.arange(q_len)[None].expand(b, q_len).cuda()
    layers = [_module(mod.LlamaFlexAttention, heads, kvh, d, seed=s) for s in range(3)]
    cache = mod.LlamaFlexAttention._tree_sparse_metadata_cache
    cache.clear()
    b0, h0 = cache.builds, cache.hits
    for layer in layers:
        pk = torch.randn(b, kvh, p, d, generator=g).to(torch.bfloat16).cuda()
        pv = torch.randn(b, kvh, p, d, generator=g).to(torch.bfloat16).cuda()
        got = layer(h, attention_mask=mask, position_ids=pos, past_key_values=llama_mock.DynamicCache(pk, pv))
        want = llama_mock.dense_flex_reference(layer, h, mask, pos, llama_mock.DynamicCache(pk, pv))
        torch.cuda.synchronize()
        err = float((got.float() - want.float()).abs().max())
        print(f"[bridge] flex shim max_abs_err {err:.3e}", flush=True)
        assert err <= TOL[torch.bfloat16], err
    assert cache.builds - b0 == 1 and cache.hits - h0 == 2


def test_cache_hidden_verify_uses_the_tree_kernel_with_gqa_heads():
    print("[bridge] cache_hidden shim", flush=True)
    mod = llama_mock.make_module()
    bridge.patch_llama_attention(mod, block_m=16, block_n=32)
    b, q_len, heads, kvh, d = 2, 48, 8, 2, 64
    rng = np.random.default_rng(12)
    tree = torch.from_numpy(trees.ancestor_mask(trees.random_parents(q_len, rng)))
    mask = llama_mock.additive_mask(tree, 0, b, torch.bfloat16).cuda()
    m = _module(mod.LlamaAttention, heads, kvh, d, seed=7)
    g = torch.Generator().manual_seed(5)
    h = torch.randn(b, q_len, heads * d, generator=g).to(torch.bfloat16).cuda()
    pos = torch.arange(q_len)[None].expand(b, q_len).cuda()
    ch_got, ch_want = [[], []], [[], []]
    got = m(h, cache_hidden=ch_got, attention_mask=mask, position_ids=pos)
    want = mod.LlamaAttention._orig_forward_tree_sparse_bridge(m, h, cache_hidden=ch_want, attention_mask=mask,
                                                               position_ids=pos)
    torch.cuda.synchronize()
    err = float((got.float() - want.float()).abs().max())
    print(f"[bridge] cache_hidden shim max_abs_err {err:.3e}", flush=True)
    # the original path rounds its softmax to bf16 before the product; bar = kernel bar + that rounding
    assert err <= TOL[torch.bfloat16] + 1e-2, err
    assert all(torch.equal(a, c) for a, c in zip(ch_got[0], ch_want[0]))
    assert ch_got[0][0].shape[1] == heads  # the cache still holds the repeat_kv copies


@pytest.mark.parametrize("case", ["shared", "per-sequence", "strided", "fp16-d64", "float-mask"])
def test_one_call_path_matches_the_metadata_path(case):
    # run_tree_sparse_kernel(q, k, v, tree_mask) on a device bool mask runs
    # tsfa_tree_attention (metadata build + forward in one C call); its O must
    # equal the general path (device metadata record, then tsfa_fwd) bit for
    # bit, and a float mask (nonzero = visible) takes the general path
    print(f"[bridge] one-call path {case}", flush=True)
    dtype, d = (torch.float16, 64) if case == "fp16-d64" else (torch.bfloat16, 128)
    q, k, v, mask = _inputs(b=3, hq=8, hkv=2, t=40, p=200, d=d, dtype=dtype, seed=11)
    if case == "per-sequence":
        rng = np.random.default_rng(12)
        mask = torch.from_numpy(np.stack([trees.ancestor_mask(trees.random_parents(40, rng)) for _ in range(3)]))
    qd, kd, vd, md = q.cuda(), k.cuda(), v.cuda(), mask.cuda()
    if case == "strided":
        # [B, N, H, D] storage viewed as [B, H, N, D], as benchmark.py:182-194 passes it
        qd = qd.transpose(1, 2).contiguous().transpose(1, 2)
        kd = kd.transpose(1, 2).contiguous().transpose(1, 2)
        vd = vd.transpose(1, 2).contiguous().transpose(1, 2)
    if case == "float-mask":
        md = md.float()
    bridge._TREE_CALLS.clear()
    out = bridge.run_tree_sparse_kernel(qd, kd, vd, md, block_m=16, block_n=32)
    took_one_call = any(e is not False for e in bridge._TREE_CALLS.values())
    assert took_one_call == (case != "float-mask")
    meta = bridge.build_tree_metadata(md.bool() if case == "float-mask" else md, k.shape[2] - q.shape[2], 16, 32)
    ref = tsf.tree_sparse_attention_fwd(qd, kd, vd, meta)
    torch.cuda.synchronize()
    assert torch.equal(out.isnan(), ref.isnan())
    assert torch.equal(out.nan_to_num(0.0), ref.nan_to_num(0.0))
    assert_close_to_oracle(out, oracle_out(q, k, v, mask, k.shape[2] - q.shape[2]), dtype)


def test_one_call_path_refuses_kv_shorter_than_q():
    q, k, v, mask = _inputs(b=1, t=40, p=0)
    with pytest.raises(ValueError):
        bridge.run_tree_sparse_kernel(q.cuda(), k[:, :, :30].cuda(), v[:, :, :30].cuda(), mask.cuda(),
                                      block_m=16, block_n=32)
