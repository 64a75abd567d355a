"""Paged K/V cache: the layout helper and the host-side argument checks of
tree_sparse_attention_fwd_paged (no device work; CPU tensors)."""

import pytest
import torch

import tree_sparse_flashattn as tsf
from tsfa import configs


def _reference_layout(k, v, page_size):
    """The cache benchmark.py:67-91 builds: request b owns pages b*n .. b*n+n-1,
    page p of it holds keys [p*page_size, min((p+1)*page_size, L)) as
    [rows, Hkv, D], K in slot 0 and V in slot 1, the rest zero."""
    bsz, hkv, kv_len, d = k.shape
    n = (kv_len + page_size - 1) // page_size
    cache = torch.zeros((bsz * n, 2, page_size, hkv, d), dtype=k.dtype)
    for b in range(bsz):
        for p in range(n):
            start, end = p * page_size, min((p + 1) * page_size, kv_len)
            cache[b * n + p, 0, :end - start] = k[b, :, start:end, :].transpose(0, 1)
            cache[b * n + p, 1, :end - start] = v[b, :, start:end, :].transpose(0, 1)
    return cache, n


@pytest.mark.parametrize("kv_len,page_size", [(50, 16), (64, 16), (33, 32), (300, 256)])
def test_make_paged_kv_matches_reference_layout(kv_len, page_size):
    g = torch.Generator().manual_seed(kv_len)
    k = torch.randn(3, 2, kv_len, 8, generator=g).to(torch.bfloat16)
    v = torch.randn(3, 2, kv_len, 8, generator=g).to(torch.bfloat16)
    cache, indptr, indices = configs.make_paged_kv(k, v, page_size)
    ref, n = _reference_layout(k, v, page_size)
    assert torch.equal(cache, ref)
    assert indptr.tolist() == [b * n for b in range(4)]
    assert indices.tolist() == list(range(3 * n))


@pytest.mark.parametrize("layout", ["NHD", "HND"])
@pytest.mark.parametrize("dense", [False, True])
def test_make_paged_kv_scattered_pages_hold_every_key(layout, dense):
    g = torch.Generator().manual_seed(1)
    k, v = torch.randn(2, 3, 70, 16, generator=g), torch.randn(2, 3, 70, 16, generator=g)
    cache, indptr, indices = configs.make_paged_kv(k, v, 16, layout=layout, seed=5, spare_pages=4,
                                                   dense_table=dense)
    assert cache.shape[0] == 2 * 5 + 4
    for b in range(2):
        pages = indices[b] if dense else indices[indptr[b]:indptr[b + 1]]
        assert len(pages) == 5
        for j in range(70):
            p, r = int(pages[j // 16]), j % 16
            kk = cache[p, 0, r] if layout == "NHD" else cache[p, 0, :, r]
            vv = cache[p, 1, r] if layout == "NHD" else cache[p, 1, :, r]
            assert torch.equal(kk, k[b, :, j]) and torch.equal(vv, v[b, :, j])
    used = indices.reshape(-1).tolist()
    assert len(set(used)) == len(used)  # no page shared by two sequences


def _meta(t=16, p=32, bm=16, bn=16):
    mask = torch.tril(torch.ones(t, t, dtype=torch.bool))
    return tsf.TreeSparseMetadata(
        row_ptr=torch.zeros(2, dtype=torch.int32), col_idx=torch.zeros(0, dtype=torch.int32),
        blk_type=torch.zeros(0, dtype=torch.int8), mixed_mask_payload=torch.zeros(0, dtype=torch.int32),
        mixed_mask_offset=torch.zeros(0, dtype=torch.int32), n_q_blocks=(t + bm - 1) // bm,
        n_tree_blocks=(t + bn - 1) // bn, block_m=bm, block_n=bn, prefix_len=p), mask


def _inputs(page_size=16, layout="NHD", dense=False, b=2, t=16, p=32):
    g = torch.Generator().manual_seed(0)
    q = torch.randn(b, 4, t, 64, generator=g).to(torch.bfloat16)
    k = torch.randn(b, 2, p + t, 64, generator=g).to(torch.bfloat16)
    v = torch.randn(b, 2, p + t, 64, generator=g).to(torch.bfloat16)
    cache, indptr, indices = configs.make_paged_kv(k, v, page_size, layout=layout, dense_table=dense)
    return q, cache, indptr, indices


def test_paged_rejects_small_or_odd_pages():
    q, _, _, _ = _inputs()
    meta, _ = _meta()
    for ps in (8, 24):
        cache = torch.zeros((6, 2, ps, 2, 64), dtype=torch.bfloat16)
        ind = torch.zeros(12, dtype=torch.int32)
        with pytest.raises(NotImplementedError):
            tsf.tree_sparse_attention_fwd_paged(q, cache, ind, meta, kv_len=48,
                                                kv_indptr=torch.tensor([0, 6, 12], dtype=torch.int32))


@pytest.mark.parametrize("change,exc", [
    (lambda a: a.update(cache=a["cache"][:, :1]), ValueError),                  # no V slot
    (lambda a: a.update(cache=a["cache"][..., :32]), ValueError),               # head_dim mismatch
    (lambda a: a.update(kv_layout="NDH"), ValueError),
    (lambda a: a.update(kv_indptr=a["kv_indptr"][:2]), ValueError),             # [B + 1] expected
    (lambda a: a.update(kv_indices=a["kv_indices"].long()), ValueError),        # int32 only
    (lambda a: a.update(kv_len=20), ValueError),                                # below prefix_len
    (lambda a: a.update(kv_indptr=None), ValueError),                           # 1-D list is no dense table
])
def test_paged_argument_errors(change, exc):
    q, cache, indptr, indices = _inputs()
    meta, _ = _meta()
    a = dict(cache=cache, kv_indices=indices, kv_indptr=indptr, kv_len=48, kv_layout="NHD")
    change(a)
    with pytest.raises(exc):
        tsf.tree_sparse_attention_fwd_paged(q, a["cache"], a["kv_indices"], meta, kv_len=a["kv_len"],
                                            kv_indptr=a["kv_indptr"], kv_layout=a["kv_layout"])


def test_paged_dense_table_too_short():
    q, cache, _, indices = _inputs(dense=True)
    meta, _ = _meta()
    with pytest.raises(ValueError):
        tsf.tree_sparse_attention_fwd_paged(q, cache, indices[:, :2], meta, kv_len=48)


def test_paged_requires_device_tensors():
    q, cache, indptr, indices = _inputs()
    meta, _ = _meta()
    with pytest.raises(ValueError, match="HIP device tensor"):
        tsf.tree_sparse_attention_fwd_paged(q, cache, indices, meta, kv_len=48, kv_indptr=indptr)
