"""HIP metadata builder vs the oracle: bit-exact on every field."""

import numpy as np
import pytest
import torch

from oracle import meta_oracle as mo
from tsfa import configs
from tests.gpu_util import assert_meta_equal

pytestmark = pytest.mark.gpu

import tree_sparse_flashattn as tsf  # noqa: E402


@pytest.mark.parametrize("name", list(configs.WORKLOADS))
def test_workload_trees(name):
    w = configs.WORKLOADS[name]
    masks = configs.make_tree_mask(w)
    masks = masks.unsqueeze(0) if masks.ndim == 2 else masks
    for b in range(masks.shape[0]):
        print(f"[meta] {name} seq {b}", flush=True)
        meta = tsf.prepare_tree_sparse_metadata(masks[b].cuda(), w.prefix_len, w.block_m, w.block_n)
        assert_meta_equal(meta, mo.build_metadata(masks[b].numpy(), w.prefix_len, w.block_m, w.block_n))


def test_readme_known_answer_on_gpu():
    mask = torch.tril(torch.ones((128, 128), dtype=torch.bool))
    meta = tsf.prepare_tree_sparse_metadata(mask, 32, 64, 64)  # CPU in -> CPU out
    assert meta.row_ptr.device.type == "cpu"
    assert meta.row_ptr.tolist() == [0, 1, 3]
    assert meta.col_idx.tolist() == [0, 0, 1]
    assert meta.blk_type.tolist() == [1, 0, 1]
    assert meta.mixed_mask_offset.tolist() == [0, 0, 128]
    assert meta.mixed_mask_payload[0] == 1 and meta.mixed_mask_payload[62] == -1
    assert_meta_equal(meta, mo.build_metadata(mask.numpy(), 32, 64, 64))


def _sweep_cases():
    rng = np.random.default_rng(7)
    cases = []
    for q_len, bm, bn in [(1, 16, 16), (64, 16, 64), (100, 32, 48), (37, 16, 16), (130, 64, 64), (129, 1, 1),
                          (70, 3, 5), (256, 128, 128), (33, 7, 32), (200, 64, 16), (64, 256, 8),
                          (64, 4, 16), (96, 8, 8)]:  # 64 blocks (one wave ranks them), 144 (block-wide scan)
        for kind in ("random", "tree", "ones", "zeros", "eye"):
            cases.append((q_len, bm, bn, kind, int(rng.integers(1 << 30))))
    return cases


# "auto": trees whose packed words fit in LDS take the one-launch builder;
# "two-launch" forces classify + compact for every shape
@pytest.mark.parametrize("path", ["auto", "two-launch"])
@pytest.mark.parametrize("q_len,bm,bn,kind,seed", _sweep_cases())
def test_sweep(q_len, bm, bn, kind, seed, path, monkeypatch):
    if path == "two-launch":
        monkeypatch.setenv("TSFA_META_SMALL", "0")
    rng = np.random.default_rng(seed)
    if kind == "random":
        m = rng.random((q_len, q_len)) < rng.random()
    elif kind == "tree":
        from tsfa import trees
        m = trees.ancestor_mask(trees.random_parents(q_len, rng))
    elif kind == "ones":
        m = np.ones((q_len, q_len), dtype=bool)
    elif kind == "zeros":
        m = np.zeros((q_len, q_len), dtype=bool)
    else:
        m = np.eye(q_len, dtype=bool)
    meta = tsf.prepare_tree_sparse_metadata(torch.from_numpy(m).cuda(), 11, bm, bn)
    assert_meta_equal(meta, mo.build_metadata(m, 11, bm, bn))


def test_nonbool_masks():
    vals = torch.tensor([[0.0, float("nan"), -1.5], [2.0, 0.0, 0.0], [0.0, 0.0, 1e-30]])
    for m in (vals, vals.to(torch.float16), (vals != 0).to(torch.int32) * 7):
        meta = tsf.prepare_tree_sparse_metadata(m.cuda(), 0, 2, 2)
        assert_meta_equal(meta, mo.build_metadata(m.float().numpy(), 0, 2, 2))


def test_validation_errors():
    with pytest.raises(ValueError):
        tsf.prepare_tree_sparse_metadata(torch.ones(3, 4, device="cuda"), 0, 16, 16)
    with pytest.raises(ValueError):
        tsf.prepare_tree_sparse_metadata(torch.ones(4, 4, device="cuda"), 0, 0, 16)


@pytest.mark.parametrize("path", ["auto", "two-launch"])
def test_batched_matches_per_sequence(path, monkeypatch):
    if path == "two-launch":
        monkeypatch.setenv("TSFA_META_SMALL", "0")
    w = configs.WORKLOADS["batched-decode-b16-p2048"]
    masks = configs.make_tree_mask(w).cuda()
    bm = tsf.prepare_tree_sparse_metadata_batched(masks, w.prefix_len, w.block_m, w.block_n)
    for b in range(w.batch):
        assert_meta_equal(bm.sequence(b), mo.build_metadata(masks[b].cpu().numpy(), w.prefix_len, w.block_m,
                                                             w.block_n))


@pytest.mark.parametrize("shape", [(16, 64), (64, 64), (5, 7), (1, 32), (64, 128)])
def test_pack_block(shape):
    rng = np.random.default_rng(shape[0] * 1000 + shape[1])
    m = rng.random(shape) < 0.5
    m[-1, -1] = True
    got = tsf._pack_block_mask_to_int32(torch.from_numpy(m).cuda())
    np.testing.assert_array_equal(got.cpu().numpy(), mo.pack_block_bits(m))
