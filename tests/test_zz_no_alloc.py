"""tsfa_fwd_noalloc -- the forward without a workspace argument, its split-KV
partials in the library's per-GPU device array -- against tsfa_fwd with a
caller workspace, called through the C-ABI: identical O on two calls in a
row, the second on a smaller input; the same under HIP graph capture on a
non-default stream (the use the entry point is for); and the size refusal."""

import pytest
import torch

import tree_sparse_flashattn as tsf
from tsfa import _lib, configs

pytestmark = pytest.mark.gpu

NOALLOC_MAX_BYTES = 64 << 20  # TSFA_FWD_NOALLOC_MAX_BYTES (include/tsfa.h)


def _noalloc(q, k, v, meta, out):
    lib = _lib.load()
    bsz, n_heads, q_len, head_dim = q.shape
    tensors, meta_strides = tsf._meta_arrays(meta, bsz)
    strides = (*q.stride(), *k.stride(), *v.stride(), *out.stride())
    args = (bsz, n_heads, k.shape[1], q_len, k.shape[2], meta.prefix_len, meta.n_q_blocks, meta.n_tree_blocks,
            n_heads // k.shape[1], meta.block_m, meta.block_n, head_dim, _lib.dtype_code(q.dtype))
    with torch.cuda.device(q.device):
        return lib.tsfa_fwd_noalloc(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(out),
                                    *(_lib.ptr(t) for t in tensors), _lib.i64_array(meta_strides),
                                    _lib.i64_array(strides), float(head_dim ** -0.5), *args,
                                    _lib.stream_handle(q.device))


def _inputs(name=None, small=False):
    if small:
        g = torch.Generator().manual_seed(5)
        q = torch.randn(1, 8, 37, 128, generator=g).to(torch.bfloat16)
        k = torch.randn(1, 2, 137, 128, generator=g).to(torch.bfloat16)
        v = torch.randn(1, 2, 137, 128, generator=g).to(torch.bfloat16)
        mask = torch.tril(torch.ones(37, 37, dtype=torch.bool))
        prefix, bm, bn = 100, 16, 16
    else:
        w = configs.WORKLOADS[name]
        q, k, v = configs.make_qkv(w)
        mask = configs.make_tree_mask(w)
        prefix, bm, bn = w.prefix_len, w.block_m, w.block_n
    q, k, v = q.cuda(), k.cuda(), v.cuda()
    meta = tsf.prepare_tree_sparse_metadata(mask.cuda(), prefix, bm, bn)
    return q, k, v, meta


def test_noalloc_matches_tsfa_fwd_on_two_calls():
    for label, inputs in (("llama3-8b-eagle64-p4096", _inputs("llama3-8b-eagle64-p4096")),
                          ("small", _inputs(small=True))):
        q, k, v, meta = inputs
        print(f"[noalloc] {label} q {tuple(q.shape)} k {tuple(k.shape)}", flush=True)
        assert tsf.fwd_workspace_bytes(q, k, meta) <= NOALLOC_MAX_BYTES
        ref = tsf.tree_sparse_attention_fwd(q, k, v, meta)  # tsfa_fwd, torch-allocated workspace
        out = torch.full_like(q, float("nan"))
        _lib.check("tsfa_fwd_noalloc", _noalloc(q, k, v, meta, out))
        torch.cuda.synchronize()
        assert torch.equal(out.isnan(), ref.isnan())
        assert torch.equal(out.nan_to_num(0.0), ref.nan_to_num(0.0)), \
            f"{label}: max diff {float((out.float() - ref.float()).nan_to_num(0).abs().max()):.3e}"


def test_noalloc_matches_tsfa_fwd_on_the_generic_kernel():
    # head_dim 256 and fp32 run the generic kernel, whose partials (in the
    # input dtype, fp32 for fp32 inputs) the entry point sizes against its
    # array by dtype
    g = torch.Generator().manual_seed(11)
    for dtype, head_dim in ((torch.float32, 128), (torch.bfloat16, 256), (torch.float32, 64)):
        q = torch.randn(2, 8, 29, head_dim, generator=g).to(dtype).cuda()
        k = torch.randn(2, 4, 29 + 300, head_dim, generator=g).to(dtype).cuda()
        v = torch.randn(2, 4, 29 + 300, head_dim, generator=g).to(dtype).cuda()
        mask = torch.tril(torch.ones(29, 29, dtype=torch.bool))
        mask[7, :7] = False
        meta = tsf.prepare_tree_sparse_metadata(mask.cuda(), 300, 16, 16)
        print(f"[noalloc] generic {dtype} head_dim {head_dim}", flush=True)
        assert tsf.fwd_workspace_bytes(q, k, meta) <= NOALLOC_MAX_BYTES
        ref = tsf.tree_sparse_attention_fwd(q, k, v, meta)
        out = torch.full_like(q, float("nan"))
        _lib.check("tsfa_fwd_noalloc", _noalloc(q, k, v, meta, out))
        torch.cuda.synchronize()
        assert torch.equal(out.isnan(), ref.isnan())
        assert torch.equal(out.nan_to_num(0.0), ref.nan_to_num(0.0)), f"{dtype} {head_dim}"


def test_noalloc_refuses_calls_past_its_array():
    # the 70B layout at 32 sequences: its partials (at least one slot of
    # 32*64*256 rows) exceed the array, so the call is refused on the host
    # before any launch (the data pointers are never read, so none are passed)
    w = configs.WORKLOADS["llama3-70b-b4-p32768"]
    batch = 32
    lib = _lib.load()
    need = lib.tsfa_fwd_workspace_bytes(batch, w.q_heads, w.kv_heads, w.tree_len, w.kv_len, w.prefix_len,
                                        w.head_dim)
    print(f"[noalloc] {w.name} at {batch} sequences needs {need} bytes", flush=True)
    assert need > NOALLOC_MAX_BYTES
    nqb = -(-w.tree_len // w.block_m)
    ntb = -(-w.tree_len // w.block_n)
    strides = (0,) * 16
    st = lib.tsfa_fwd_noalloc(None, None, None, None, None, None, None, None, None, _lib.i64_array((0,) * 5),
                              _lib.i64_array(strides), 0.088, batch, w.q_heads, w.kv_heads, w.tree_len, w.kv_len,
                              w.prefix_len, nqb, ntb, w.q_heads // w.kv_heads, w.block_m, w.block_n, w.head_dim,
                              _lib.dtype_code(w.dtype), None)
    assert st == _lib.TSFA_ERR_WORKSPACE


def test_noalloc_captured_in_a_graph_on_a_side_stream():
    # tsfa_fwd_noalloc captured into a HIP graph on a non-default stream and
    # replayed three times, with eager work between the replays (the array
    # keeps the last call's contents): every replay equals tsfa_fwd's O
    q, k, v, meta = _inputs("llama3-8b-eagle64-p4096")
    ref = tsf.tree_sparse_attention_fwd(q, k, v, meta)
    out = torch.full_like(q, float("nan"))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        _lib.check("tsfa_fwd_noalloc", _noalloc(q, k, v, meta, out))  # takes the array's address
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            _lib.check("tsfa_fwd_noalloc", _noalloc(q, k, v, meta, out))
    torch.cuda.synchronize()
    small = _inputs(small=True)
    for rep in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        print(f"[noalloc] graph replay {rep}", flush=True)
        assert torch.equal(out.isnan(), ref.isnan())
        assert torch.equal(out.nan_to_num(0.0), ref.nan_to_num(0.0)), f"replay {rep} differs from tsfa_fwd"
        # an eager call on another shape between replays overwrites the array
        tmp = torch.empty_like(small[0])
        _lib.check("tsfa_fwd_noalloc", _noalloc(*small, tmp))
        torch.cuda.synchronize()
