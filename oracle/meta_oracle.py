"""numpy restatement of the tree-sparse metadata protocol.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Follows ``tree_sparse_flashattn.py`` of the reference:
  * block codes                 tree_sparse_flashattn.py:11-12
  * bitset packer               tree_sparse_flashattn.py:44-64
  * metadata builder            tree_sparse_flashattn.py:67-160

Pinning (what checks this restatement independently of its own formula):
  * the README quick-start known answer (tril 128x128, prefix 32, 64x64
    blocks; README.md:141-162), hand-derived word by word in
    tests/test_oracle_meta.py;
  * closed forms for all-ones masks (every block FULL, empty payload and
    empty offset tensor, tree_sparse_flashattn.py:142-147), identity masks and
    all-zero masks;
  * the decode invariant: unpacking every MIXED payload with the kernel's
    rule ``(word >> (flat % 32)) & 1`` (tree_sparse_flashattn.py:241-245,
    :313-318) reproduces the zero-padded block, FULL blocks are all-ones on
    their clipped extent and ZERO blocks are exactly the absent ones;
  * brute force over every bit position 0..31 of a word, including bit 31
    (negative int32 words).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

FULL_BLOCK = 0   # tree_sparse_flashattn.py:11
MIXED_BLOCK = 1  # tree_sparse_flashattn.py:12


@dataclass
class OracleMetadata:
    """Field-for-field mirror of ``TreeSparseMetadata`` (tree_sparse_flashattn.py:15-41)."""

    row_ptr: np.ndarray             # int32 [n_q_blocks + 1]
    col_idx: np.ndarray             # int32 [nnz]
    blk_type: np.ndarray            # int8  [nnz]
    mixed_mask_payload: np.ndarray  # int32 [n_mixed * words_per_block]
    mixed_mask_offset: np.ndarray   # int32 [nnz], or [0] when n_mixed == 0
    n_q_blocks: int
    n_tree_blocks: int
    block_m: int
    block_n: int
    prefix_len: int


def words_per_block(block_m: int, block_n: int) -> int:
    """int32 words per packed MIXED block: ceil(BM*BN/32) (tree_sparse_flashattn.py:53)."""
    return (block_m * block_n + 31) // 32


def pack_block_bits(block: np.ndarray) -> np.ndarray:
    """Pack a bool block row-major into int32 words; bit i of word w = flat[32w+i].

    Restates ``_pack_block_mask_to_int32`` (tree_sparse_flashattn.py:44-64):
    the reference scatter-adds ``1 << bit`` into int32 words, which for
    distinct bits equals the bitwise OR, read back as two's complement.
    """
    flat = np.asarray(block).reshape(-1).astype(bool)
    n_words = (flat.size + 31) // 32
    bits = np.zeros(n_words * 32, dtype=bool)
    bits[: flat.size] = flat
    packed = np.packbits(bits, bitorder="little")  # byte b bit i = bits[8b+i]
    return packed.view("<u4").view("<i4").astype(np.int32)


def _as_bool_mask(tree_mask) -> np.ndarray:
    """Nonzero -> True, NaN included (tree_sparse_flashattn.py:90)."""
    if hasattr(tree_mask, "detach"):  # torch tensor
        t = tree_mask.detach().cpu()
        if t.dtype.is_floating_point or t.dtype.is_complex:
            t = t.float()
        tree_mask = t.numpy()
    arr = np.asarray(tree_mask)
    return arr != 0


def build_metadata(tree_mask, prefix_len: int, block_m: int, block_n: int) -> OracleMetadata:
    """Restatement of ``prepare_tree_sparse_metadata`` (tree_sparse_flashattn.py:67-160)."""
    mask = _as_bool_mask(tree_mask)
    if mask.ndim != 2 or mask.shape[0] != mask.shape[1]:            # :85-86
        raise ValueError("tree_mask must be shape [q_len, q_len].")
    if block_m <= 0 or block_n <= 0:                                 # :87-88
        raise ValueError("BLOCK_M and BLOCK_N must be positive.")

    q_len = mask.shape[0]
    n_q_blocks = (q_len + block_m - 1) // block_m                    # :92
    n_tree_blocks = (q_len + block_n - 1) // block_n                 # :93

    row_ptr = [0]
    col_idx: list[int] = []
    blk_type: list[int] = []
    offsets: list[int] = []
    chunks: list[np.ndarray] = []
    cursor = 0
    for qb in range(n_q_blocks):                                     # :103
        q0, q1 = qb * block_m, min(qb * block_m + block_m, q_len)
        row_nnz = 0
        for tb in range(n_tree_blocks):                              # :108
            k0, k1 = tb * block_n, min(tb * block_n + block_n, q_len)
            local = mask[q0:q1, k0:k1]
            if not local.any():                                      # :113-114 ZERO
                continue
            col_idx.append(tb)
            row_nnz += 1
            if int(local.sum()) == local.size:                       # :122 FULL on the clipped block
                blk_type.append(FULL_BLOCK)
                offsets.append(0)
            else:                                                    # :125-134 MIXED
                blk_type.append(MIXED_BLOCK)
                padded = np.zeros((block_m, block_n), dtype=bool)
                padded[: q1 - q0, : k1 - k0] = local
                words = pack_block_bits(padded)
                chunks.append(words)
                offsets.append(cursor)
                cursor += words.size
        row_ptr.append(row_ptr[-1] + row_nnz)                        # :136

    if chunks:                                                       # :142-147
        payload = np.concatenate(chunks).astype(np.int32)
        offset = np.asarray(offsets, dtype=np.int32)
    else:
        payload = np.zeros((0,), dtype=np.int32)
        offset = np.zeros((0,), dtype=np.int32)

    return OracleMetadata(
        row_ptr=np.asarray(row_ptr, dtype=np.int32),
        col_idx=np.asarray(col_idx, dtype=np.int32),
        blk_type=np.asarray(blk_type, dtype=np.int8),
        mixed_mask_payload=payload,
        mixed_mask_offset=offset,
        n_q_blocks=n_q_blocks,
        n_tree_blocks=n_tree_blocks,
        block_m=block_m,
        block_n=block_n,
        prefix_len=prefix_len,
    )


def decode_block(payload: np.ndarray, offset: int, block_m: int, block_n: int) -> np.ndarray:
    """Unpack one MIXED block with the kernel's rule (tree_sparse_flashattn.py:241-245, :313-318)."""
    flat = np.arange(block_m * block_n)
    words = payload[offset + flat // 32].astype(np.int64)
    return (((words >> (flat % 32)) & 1) == 1).reshape(block_m, block_n)


def metadata_to_dense(meta: OracleMetadata, q_len: int) -> np.ndarray:
    """Rebuild the [q_len, q_len] visibility mask that the metadata encodes."""
    out = np.zeros((q_len, q_len), dtype=bool)
    bm, bn = meta.block_m, meta.block_n
    for qb in range(meta.n_q_blocks):
        q0, q1 = qb * bm, min(qb * bm + bm, q_len)
        for ridx in range(int(meta.row_ptr[qb]), int(meta.row_ptr[qb + 1])):
            tb = int(meta.col_idx[ridx])
            k0, k1 = tb * bn, min(tb * bn + bn, q_len)
            if int(meta.blk_type[ridx]) == FULL_BLOCK:
                out[q0:q1, k0:k1] = True
            else:
                blk = decode_block(meta.mixed_mask_payload, int(meta.mixed_mask_offset[ridx]), bm, bn)
                out[q0:q1, k0:k1] = blk[: q1 - q0, : k1 - k0]
    return out
