"""Pins the metadata oracle (oracle/meta_oracle.py) independently of its own code.

Checks: the README quick-start known answer derived by hand, closed forms
(all-ones / all-zeros / identity / clipped-edge FULL), bit-position brute
force including bit 31, and the decode invariant on random masks.
"""

import numpy as np
import pytest
from hypothesis import given, settings, strategies as st

from oracle import meta_oracle as mo


def _i32(u):
    return np.uint32(u & 0xFFFFFFFF).view(np.int32)


def test_readme_known_answer():
    # README.md:141-162: tril(128x128), prefix 32, 64x64 blocks.
    mask = np.tril(np.ones((128, 128), dtype=bool))
    meta = mo.build_metadata(mask, 32, 64, 64)
    assert meta.n_q_blocks == 2 and meta.n_tree_blocks == 2
    assert meta.row_ptr.tolist() == [0, 1, 3]
    assert meta.col_idx.tolist() == [0, 0, 1]
    assert meta.blk_type.tolist() == [1, 0, 1]
    assert meta.mixed_mask_offset.tolist() == [0, 0, 128]
    assert meta.mixed_mask_payload.shape == (256,)
    # Row r of a tril 64x64 block: word 2r holds columns 0..min(r,31),
    # word 2r+1 holds columns 32..r (r >= 32).
    expected = []
    for r in range(64):
        expected.append(_i32((1 << (min(r, 31) + 1)) - 1))
        expected.append(_i32((1 << (r - 31)) - 1) if r >= 32 else 0)
    expected = np.array(expected * 2, dtype=np.int32)
    np.testing.assert_array_equal(meta.mixed_mask_payload, expected)
    # spot values written out literally
    p = meta.mixed_mask_payload
    assert p[0] == 1 and p[62] == -1 and p[63] == 0 and p[126] == -1 and p[127] == -1
    assert p[128] == 1 and p[254] == -1 and p[255] == -1
    assert meta.row_ptr.dtype == np.int32 and meta.col_idx.dtype == np.int32
    assert meta.blk_type.dtype == np.int8 and meta.mixed_mask_payload.dtype == np.int32


def test_all_ones_every_block_full_and_offset_empty():
    # Edge blocks are clipped (100 = 3*32+4, 100 = 2*48+4) yet FULL.
    meta = mo.build_metadata(np.ones((100, 100)), 0, 32, 48)
    assert meta.n_q_blocks == 4 and meta.n_tree_blocks == 3
    assert meta.row_ptr.tolist() == [0, 3, 6, 9, 12]
    assert meta.col_idx.tolist() == [0, 1, 2] * 4
    assert meta.blk_type.tolist() == [0] * 12
    assert meta.mixed_mask_payload.size == 0
    assert meta.mixed_mask_offset.size == 0  # tree_sparse_flashattn.py:145-147


def test_all_zeros():
    meta = mo.build_metadata(np.zeros((40, 40), dtype=np.int32), 5, 16, 16)
    assert meta.row_ptr.tolist() == [0, 0, 0, 0]
    assert meta.col_idx.size == meta.blk_type.size == 0
    assert meta.mixed_mask_payload.size == meta.mixed_mask_offset.size == 0


def test_identity_unit_blocks_are_full():
    meta = mo.build_metadata(np.eye(7, dtype=bool), 0, 1, 1)
    assert meta.row_ptr.tolist() == list(range(8))
    assert meta.col_idx.tolist() == list(range(7))
    assert meta.blk_type.tolist() == [0] * 7
    assert meta.mixed_mask_offset.size == 0


def test_identity_16_blocks_mixed():
    meta = mo.build_metadata(np.eye(64, dtype=bool), 0, 16, 16)
    assert meta.row_ptr.tolist() == [0, 1, 2, 3, 4]
    assert meta.col_idx.tolist() == [0, 1, 2, 3]
    assert meta.blk_type.tolist() == [1, 1, 1, 1]
    assert meta.mixed_mask_offset.tolist() == [0, 8, 16, 24]
    # diagonal element r sits at flat 17r -> word 17r//32, bit 17r%32
    blk = np.zeros(8, dtype=np.int64)
    for r in range(16):
        blk[(17 * r) // 32] += 1 << ((17 * r) % 32)
    np.testing.assert_array_equal(meta.mixed_mask_payload[:8], np.array([_i32(int(x)) for x in blk]))


def test_full_is_decided_on_the_clipped_block():
    # q_len 10, 8x8 blocks: block (1,1) covers rows/cols 8..9 only.
    m = np.zeros((10, 10), dtype=bool)
    m[8:, 8:] = True
    m[0, 0] = True
    meta = mo.build_metadata(m, 0, 8, 8)
    assert meta.row_ptr.tolist() == [0, 1, 2]
    assert meta.col_idx.tolist() == [0, 1]
    assert meta.blk_type.tolist() == [1, 0]
    assert meta.mixed_mask_offset.tolist() == [0, 0]


@pytest.mark.parametrize("bit", range(32))
def test_single_bit_positions(bit):
    row = np.zeros((1, 32), dtype=bool)
    row[0, bit] = True
    words = mo.pack_block_bits(row)
    assert words.shape == (1,)
    assert int(words[0]) == int(_i32(1 << bit))
    if bit == 31:
        assert int(words[0]) == -(2 ** 31)


def test_pack_ragged_tail_word():
    # 5x7 = 35 bits -> 2 words; bits 32..34 land in word 1 bits 0..2
    m = np.zeros((5, 7), dtype=bool)
    m[4, 4:7] = True  # flat 32, 33, 34
    assert mo.pack_block_bits(m).tolist() == [0, 7]


def test_nan_counts_as_visible():
    m = np.array([[np.nan, 0.0], [0.0, 2.5]])
    meta = mo.build_metadata(m, 0, 2, 2)
    dense = mo.metadata_to_dense(meta, 2)
    assert dense.tolist() == [[True, False], [False, True]]


@pytest.mark.parametrize("bad", [np.zeros((3, 4)), np.zeros((2, 2, 2)), np.zeros(5)])
def test_shape_validation(bad):
    with pytest.raises(ValueError):
        mo.build_metadata(bad, 0, 16, 16)


@pytest.mark.parametrize("bm,bn", [(0, 16), (16, 0), (-1, 4)])
def test_block_validation(bm, bn):
    with pytest.raises(ValueError):
        mo.build_metadata(np.ones((4, 4)), 0, bm, bn)


@settings(max_examples=60, deadline=None)
@given(q_len=st.integers(1, 70), bm=st.integers(1, 40), bn=st.integers(1, 40),
       density=st.floats(0.0, 1.0), seed=st.integers(0, 2 ** 31))
def test_decode_invariant_random(q_len, bm, bn, density, seed):
    rng = np.random.default_rng(seed)
    mask = rng.random((q_len, q_len)) < density
    meta = mo.build_metadata(mask, 3, bm, bn)
    # the metadata encodes exactly the mask
    np.testing.assert_array_equal(mo.metadata_to_dense(meta, q_len), mask)
    nnz = meta.col_idx.size
    assert meta.row_ptr[0] == 0 and meta.row_ptr[-1] == nnz
    assert np.all(np.diff(meta.row_ptr) >= 0)
    w = mo.words_per_block(bm, bn)
    n_mixed = int((meta.blk_type == 1).sum())
    assert meta.mixed_mask_payload.size == n_mixed * w
    assert meta.mixed_mask_offset.size == (nnz if n_mixed else 0)
    cursor = 0
    for qb in range(meta.n_q_blocks):
        row = meta.col_idx[meta.row_ptr[qb]:meta.row_ptr[qb + 1]]
        assert np.all(np.diff(row) > 0)
        q0, q1 = qb * bm, min(qb * bm + bm, q_len)
        present = set(row.tolist())
        for tb in range(meta.n_tree_blocks):
            k0, k1 = tb * bn, min(tb * bn + bn, q_len)
            assert (tb in present) == bool(mask[q0:q1, k0:k1].any())  # ZERO <=> absent
        for ridx in range(meta.row_ptr[qb], meta.row_ptr[qb + 1]):
            if meta.blk_type[ridx] == 1:
                assert meta.mixed_mask_offset[ridx] == cursor
                cursor += w
            elif n_mixed:
                assert meta.mixed_mask_offset[ridx] == 0
    # padding bits of MIXED blocks are zero
    for ridx in np.nonzero(meta.blk_type == 1)[0]:
        qb = int(np.searchsorted(meta.row_ptr, ridx, side="right") - 1)
        tb = int(meta.col_idx[ridx])
        blk = mo.decode_block(meta.mixed_mask_payload, int(meta.mixed_mask_offset[ridx]), bm, bn)
        h, wd = min(bm, q_len - qb * bm), min(bn, q_len - tb * bn)
        assert not blk[h:, :].any() and not blk[:, wd:].any()
