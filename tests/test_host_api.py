"""Host-side behaviour of the drop-in modules that needs no GPU: the
reference's errors and the attention-mask extraction contract."""

import pytest
import torch

import eagle_tree_sparse_bridge as bridge
import tree_sparse_flashattn as tsf


def test_public_names():
    assert tsf.FULL_BLOCK == 0 and tsf.MIXED_BLOCK == 1
    fields = [f for f in tsf.TreeSparseMetadata.__dataclass_fields__]
    assert fields == ["row_ptr", "col_idx", "blk_type", "mixed_mask_payload", "mixed_mask_offset",
                      "n_q_blocks", "n_tree_blocks", "block_m", "block_n", "prefix_len"]
    assert callable(tsf.block_sparse_tree_fwd_kernel[(4, 32)])
    with pytest.raises(TypeError):
        tsf.block_sparse_tree_fwd_kernel()


@pytest.mark.parametrize("mask", [torch.ones(3, 4), torch.ones(2, 2, 2), torch.ones(5)])
def test_prepare_rejects_shapes(mask):
    with pytest.raises(ValueError):
        tsf.prepare_tree_sparse_metadata(mask, 0, 16, 16)


def test_prepare_rejects_blocks():
    with pytest.raises(ValueError):
        tsf.prepare_tree_sparse_metadata(torch.ones(4, 4), 0, 0, 16)
    with pytest.raises(ValueError):
        tsf.prepare_tree_sparse_metadata(torch.ones(4, 4), 0, 16, -1)


def test_forward_has_no_cpu_fallback():
    # the metadata protocol runs on the host for a CPU mask; the forward
    # itself refuses host tensors instead of computing on the CPU
    q = torch.zeros(1, 2, 4, 64, dtype=torch.bfloat16)
    k = torch.zeros(1, 2, 8, 64, dtype=torch.bfloat16)
    meta = tsf.prepare_tree_sparse_metadata(torch.ones(4, 4, dtype=torch.bool), 4, 16, 16)
    assert meta.row_ptr.device.type == "cpu"
    with pytest.raises(ValueError):
        tsf.tree_sparse_attention_fwd(q, k, k, meta)


def _hf_mask(q, kv, tree):
    m = torch.zeros(2, 1, q, kv)
    m[:, :, :, kv - q:] = torch.where(tree, 0.0, float("-inf"))
    return m


def test_extract_float_mask():
    tree = torch.tril(torch.ones(4, 4, dtype=torch.bool))
    tree[3, 1] = False
    got = bridge.extract_tree_mask_from_attention_mask(_hf_mask(4, 10, tree), 4, 10)
    assert got.dtype == torch.bool and torch.equal(got, tree)


def test_extract_bool_and_int_masks():
    tree = torch.eye(3, dtype=torch.bool)
    m = torch.zeros(1, 1, 3, 5, dtype=torch.bool)
    m[0, 0, :, 2:] = tree
    assert torch.equal(bridge.extract_tree_mask_from_attention_mask(m, 3, 5), tree)
    assert torch.equal(bridge.extract_tree_mask_from_attention_mask(m.to(torch.int64) * 3, 3, 5), tree)


def test_extract_positive_and_nonfinite_values():
    m = torch.tensor([[[[5.0, 1.0, float("nan"), -1e-9, float("inf"), 0.0]]]]).expand(1, 1, 2, 6).clone()
    got = bridge.extract_tree_mask_from_attention_mask(m, 2, 6)   # tree columns 4..5
    assert got.tolist() == [[False, True], [False, True]]


@pytest.mark.parametrize("args", [
    (None, 4, 10), (torch.zeros(1, 1, 4, 10), 1, 10), (torch.zeros(4, 10), 4, 10),
    (torch.zeros(1, 1, 3, 10), 4, 10), (torch.zeros(1, 1, 4, 8), 4, 10), (torch.zeros(1, 1, 4, 10), 4, 3),
])
def test_extract_fallback_none(args):
    assert bridge.extract_tree_mask_from_attention_mask(*args) is None


def test_extract_batch_idx():
    m = torch.zeros(2, 1, 2, 4)
    m[1, 0, 0, 3] = float("-inf")
    assert bridge.extract_tree_mask_from_attention_mask(m, 2, 4).all()
    assert bridge.extract_tree_mask_from_attention_mask(m, 2, 4, batch_idx=1).tolist() == [[True, False],
                                                                                           [True, True]]


def test_run_requires_device_tensors():
    q = torch.zeros(1, 2, 4, 64)
    k = torch.zeros(1, 2, 8, 64)
    with pytest.raises(AssertionError):
        bridge.run_tree_sparse_kernel(q, k, k, torch.eye(4, dtype=torch.bool), block_m=16, block_n=16)


def _cpu_meta(t=4, p=4):
    z = torch.zeros(1, dtype=torch.int32)
    return tsf.TreeSparseMetadata(z, z, z.to(torch.int8), z, z, 1, 1, 16, 16, p)


@pytest.mark.parametrize("bad", ["k_batch", "k_dim", "v_shape", "out_shape", "gqa"])
def test_fwd_rejects_mismatched_shapes(bad):
    # raised on the host before any launch (CPU tensors: nothing reaches a device)
    q, k, v, out = torch.zeros(2, 4, 4, 64), torch.zeros(2, 2, 8, 64), torch.zeros(2, 2, 8, 64), None
    if bad == "k_batch":
        k = v = torch.zeros(1, 2, 8, 64)
    elif bad == "k_dim":
        k = v = torch.zeros(2, 2, 8, 128)
    elif bad == "v_shape":
        v = torch.zeros(2, 2, 9, 64)
    elif bad == "out_shape":
        out = torch.zeros(2, 4, 5, 64)
    else:
        k = v = torch.zeros(2, 3, 8, 64)
    with pytest.raises(ValueError):
        tsf.tree_sparse_attention_fwd(q, k, v, _cpu_meta(), out=out)


@pytest.mark.parametrize("bad", ["dq", "dk", "dv", "o", "dout", "k_batch"])
def test_bwd_rejects_mismatched_shapes(bad):
    q, k = torch.zeros(2, 4, 4, 64), torch.zeros(2, 2, 8, 64)
    v, o, dout, lse = k.clone(), q.clone(), q.clone(), torch.zeros(2, 4, 4)
    kw = {}
    if bad in ("dq", "o", "dout"):
        wrong = torch.zeros(2, 4, 3, 64)
        if bad == "dq":
            kw["dq"] = wrong
        elif bad == "o":
            o = wrong
        else:
            dout = wrong
    elif bad in ("dk", "dv"):
        kw[bad] = torch.zeros(2, 2, 7, 64)
    else:
        k = v = torch.zeros(3, 2, 8, 64)
    with pytest.raises(ValueError):
        tsf.tree_sparse_attention_bwd(q, k, v, o, lse, dout, _cpu_meta(), **kw)


def test_paged_rejects_out_shape():
    q = torch.zeros(1, 4, 4, 64)
    cache = torch.zeros(2, 2, 16, 2, 64)
    with pytest.raises(ValueError):
        tsf.tree_sparse_attention_fwd_paged(q, cache, torch.zeros(1, 1, dtype=torch.int32), _cpu_meta(), kv_len=8,
                                            out=torch.zeros(1, 4, 4, 32))
