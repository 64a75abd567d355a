"""The metadata protocol on a CPU mask -- prepare_tree_sparse_metadata and
_pack_block_mask_to_int32 run on the host by libtsfa's C++ builder (no
device), as the reference runs them -- bit-exact with the oracle."""

import numpy as np
import pytest
import torch

from oracle import meta_oracle as mo
from tsfa import configs, trees
from tests.gpu_util import assert_meta_equal

import tree_sparse_flashattn as tsf  # noqa: E402


def test_readme_quick_start_on_cpu():
    # README.md:141-162 (the CPU-runnable configuration): tril(128x128),
    # prefix 32, 64x64 blocks, CPU tensors in and out
    mask = torch.tril(torch.ones((128, 128), dtype=torch.bool))
    meta = tsf.prepare_tree_sparse_metadata(mask, 32, 64, 64)
    for t in (meta.row_ptr, meta.col_idx, meta.blk_type, meta.mixed_mask_payload, meta.mixed_mask_offset):
        assert t.device.type == "cpu"
    assert meta.row_ptr.tolist() == [0, 1, 3]
    assert meta.col_idx.tolist() == [0, 0, 1]
    assert meta.blk_type.tolist() == [1, 0, 1]
    assert meta.mixed_mask_offset.tolist() == [0, 0, 128]
    assert meta.mixed_mask_payload[0] == 1 and meta.mixed_mask_payload[62] == -1
    assert_meta_equal(meta, mo.build_metadata(mask.numpy(), 32, 64, 64))


def _mask(kind, q_len, rng):
    if kind == "random":
        return rng.random((q_len, q_len)) < rng.random()
    if kind == "tree":
        return trees.ancestor_mask(trees.random_parents(q_len, rng))
    if kind == "ones":
        return np.ones((q_len, q_len), dtype=bool)
    if kind == "zeros":
        return np.zeros((q_len, q_len), dtype=bool)
    return np.eye(q_len, dtype=bool)


SHAPES = [(0, 16, 16), (1, 16, 16), (64, 16, 64), (100, 32, 48), (37, 16, 16), (130, 64, 64), (129, 1, 1),
          (70, 3, 5), (256, 128, 128), (33, 7, 32), (200, 64, 16), (64, 256, 8), (64, 4, 16), (96, 8, 8)]


@pytest.mark.parametrize("kind", ["random", "tree", "ones", "zeros", "eye"])
@pytest.mark.parametrize("q_len,bm,bn", SHAPES)
def test_host_builder_matches_oracle(q_len, bm, bn, kind):
    rng = np.random.default_rng(q_len * 7 + bm * 3 + bn)
    m = _mask(kind, q_len, rng)
    meta = tsf.prepare_tree_sparse_metadata(torch.from_numpy(m), 11, bm, bn)
    assert_meta_equal(meta, mo.build_metadata(m, 11, bm, bn))


@pytest.mark.parametrize("name", list(configs.WORKLOADS))
def test_workload_trees_on_host(name):
    w = configs.WORKLOADS[name]
    masks = configs.make_tree_mask(w)
    masks = masks.unsqueeze(0) if masks.ndim == 2 else masks
    for b in range(masks.shape[0]):
        meta = tsf.prepare_tree_sparse_metadata(masks[b], w.prefix_len, w.block_m, w.block_n)
        assert_meta_equal(meta, mo.build_metadata(masks[b].numpy(), w.prefix_len, w.block_m, w.block_n))


def test_batched_host_record_matches_each_sequence():
    rng = np.random.default_rng(4)
    masks = np.stack([trees.ancestor_mask(trees.random_parents(45, rng)) for _ in range(3)])
    rec = tsf.prepare_tree_sparse_metadata_batched(torch.from_numpy(masks), 70, 16, 32)
    assert rec.row_ptr.device.type == "cpu" and rec.n_trees == 3
    for b in range(3):
        assert_meta_equal(rec.sequence(b), mo.build_metadata(masks[b], 70, 16, 32))


def test_nonbool_cpu_masks():
    vals = torch.tensor([[0.0, float("nan"), -1.5], [2.0, 0.0, 0.0], [0.0, 0.0, 1e-30]])
    for m in (vals, vals.to(torch.float16), (vals != 0).to(torch.int32) * 7, vals.t()):
        meta = tsf.prepare_tree_sparse_metadata(m, 0, 2, 2)
        assert_meta_equal(meta, mo.build_metadata(m.float().numpy(), 0, 2, 2))


@pytest.mark.parametrize("shape", [(1, 1), (3, 5), (16, 16), (7, 33), (64, 64), (0, 4)])
def test_pack_block_on_host(shape):
    rng = np.random.default_rng(sum(shape))
    block = rng.random(shape) < 0.5
    got = tsf._pack_block_mask_to_int32(torch.from_numpy(block))
    assert got.device.type == "cpu" and got.dtype == torch.int32
    np.testing.assert_array_equal(got.numpy(), mo.pack_block_bits(block))


def test_host_builder_rejects_like_the_reference():
    with pytest.raises(ValueError):
        tsf.prepare_tree_sparse_metadata(torch.ones(4, 4), 0, 0, 16)
    with pytest.raises(ValueError):
        tsf.prepare_tree_sparse_metadata(torch.ones(4, 5), 0, 16, 16)


@pytest.mark.parametrize("view", ["row_stride_0", "transposed", "batched_expand"])
def test_host_builder_takes_overlapping_and_strided_masks(view):
    # views whose rows overlap or are not contiguous: the reference makes
    # them dense (.contiguous()); the host builder sees the dense copy
    rng = np.random.default_rng(5)
    if view == "row_stride_0":
        row = torch.from_numpy(rng.random(24) < 0.5)
        m = row.unsqueeze(0).expand(24, 24)
        assert m.stride(-2) == 0
    elif view == "transposed":
        m = torch.from_numpy(trees.ancestor_mask(trees.random_parents(40, rng))).t()
    else:
        one = torch.from_numpy(trees.ancestor_mask(trees.random_parents(32, rng)))
        m = one.unsqueeze(0).expand(3, 32, 32)
    dense = m.contiguous().numpy()
    if m.ndim == 2:
        meta = tsf.prepare_tree_sparse_metadata(m, 7, 16, 16)
        assert_meta_equal(meta, mo.build_metadata(dense, 7, 16, 16))
    else:
        bm = tsf.prepare_tree_sparse_metadata_batched(m, 7, 16, 16)
        for b in range(m.shape[0]):
            assert_meta_equal(bm.sequence(b), mo.build_metadata(dense[b], 7, 16, 16))
