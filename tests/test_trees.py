"""Seeded tree generators and the workload definitions (CPU)."""

import numpy as np
import pytest

from oracle import meta_oracle as mo
from tsfa import configs, trees


def _check_tree(parents, n):
    assert parents.shape == (n,) and parents[0] == -1
    assert np.all(parents[1:] >= 0) and np.all(parents[1:] < np.arange(1, n))


def test_ancestor_mask_closed_form():
    parents = np.array([-1, 0, 0, 1, 1, 2])
    m = trees.ancestor_mask(parents)
    expected = np.array([[1, 0, 0, 0, 0, 0], [1, 1, 0, 0, 0, 0], [1, 0, 1, 0, 0, 0],
                         [1, 1, 0, 1, 0, 0], [1, 1, 0, 0, 1, 0], [1, 0, 1, 0, 0, 1]], dtype=bool)
    np.testing.assert_array_equal(m, expected)
    with pytest.raises(ValueError):
        trees.ancestor_mask(np.array([-1, 2, 0]))


@pytest.mark.parametrize("name", list(configs.WORKLOADS))
def test_workload_trees_are_trees(name):
    w = configs.WORKLOADS[name]
    masks = configs.make_tree_mask(w).numpy()
    masks = masks[None] if masks.ndim == 2 else masks
    assert masks.shape[1:] == (w.tree_len, w.tree_len)
    for b in range(masks.shape[0]):
        m = masks[b]
        assert np.all(np.diag(m)) and not np.triu(m, 1).any()   # topological, self-visible
        assert np.all(m[:, 0])                                     # root is everyone's ancestor
        # ancestor closure: row i = row parent(i) + i
        parent = [int(np.nonzero(m[i, :i])[0].max()) if i else -1 for i in range(w.tree_len)]
        for i in range(1, w.tree_len):
            np.testing.assert_array_equal(m[i, :i], m[parent[i], :i])


def test_eagle_tree_shape_and_determinism():
    rng = np.random.default_rng(0)
    p = trees.eagle_parents(64, 6, 8, rng)
    _check_tree(p, 64)
    d = trees.depths(p)
    assert d.max() <= 6 and np.all(np.diff(d) >= 0)
    assert (d == 1).sum() <= 8
    np.testing.assert_array_equal(p, trees.eagle_parents(64, 6, 8, np.random.default_rng(0)))


def test_depth_limited_and_kary():
    p = trees.depth_limited_parents(256, 10, np.random.default_rng(1))
    _check_tree(p, 256)
    assert trees.depths(p).max() <= 10
    k = trees.kary_bfs_parents(1024, 4)
    _check_tree(k, 1024)
    assert trees.depths(k).max() == 5  # 1+4+16+64+256 = 341 < 1024 <= 1365


def test_wide_tree_metadata_counts():
    # 4-ary BFS tree of 1024 nodes, 64x64 blocks: deterministic structure
    w = configs.WORKLOADS["wide-tree-1024-p16384"]
    meta = mo.build_metadata(configs.make_tree_mask(w).numpy(), w.prefix_len, 64, 64)
    assert meta.n_q_blocks == meta.n_tree_blocks == 16
    assert meta.col_idx.size == 45
    assert (meta.blk_type == mo.FULL_BLOCK).sum() == 0   # ancestor masks give no FULL block


def test_headline_workload_geometry():
    w = configs.WORKLOADS[configs.HEADLINE]
    assert (w.batch, w.q_heads, w.kv_heads, w.head_dim, w.prefix_len, w.tree_len) == (1, 32, 8, 128, 4096, 64)
    assert w.kv_bytes() == 17_039_360
    meta = mo.build_metadata(configs.make_tree_mask(w).numpy(), w.prefix_len, w.block_m, w.block_n)
    assert meta.n_q_blocks == 4 and meta.n_tree_blocks == 1
    assert meta.col_idx.size == 4 and np.all(meta.blk_type == mo.MIXED_BLOCK)
