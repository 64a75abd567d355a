"""Tree-sparse FlashAttention for MI355X: the metadata protocol and forward.

Drop-in for the reference module ``tree_sparse_flashattn.py`` (same public
names, argument meaning and errors).  Everything here is host plumbing around
libtsfa.so (hand-written HIP for gfx950): the metadata builder and the
forward run on the GPU; there is no CPU fallback.

Public API (reference citations):
  FULL_BLOCK, MIXED_BLOCK                  tree_sparse_flashattn.py:11-12
  TreeSparseMetadata                       tree_sparse_flashattn.py:15-41
  _pack_block_mask_to_int32                tree_sparse_flashattn.py:44-64
  prepare_tree_sparse_metadata             tree_sparse_flashattn.py:67-160
  block_sparse_tree_fwd_kernel[grid](...)  tree_sparse_flashattn.py:163-339
Extensions (no reference counterpart):
  BatchedTreeSparseMetadata / prepare_tree_sparse_metadata_batched: one tree
  per sequence (or one tree broadcast over the batch) in capacity layout,
  built without a host synchronisation; slice b is bit-identical to
  prepare_tree_sparse_metadata of tree b.
  tree_sparse_attention_fwd: allocate O and launch with either record.
  tree_sparse_attention_fwd(..., return_lse=True), tree_sparse_attention_bwd,
  tree_sparse_attention (autograd): the backward, which the reference lacks
  (README.md:198): dQ, dK, dV on HIP kernels from the forward's O and LSE.
  tree_sparse_attention_fwd_paged: the same forward over a paged K/V cache
  (FlashInfer's [pages, 2, page_size, Hkv, D] layout, benchmark.py:67-91)
  with per-sequence page lists, read in place.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import List, Optional

import torch

from tsfa import _lib

FULL_BLOCK = 0
MIXED_BLOCK = 1


@dataclass
class TreeSparseMetadata:
    """Compressed tree-block metadata for sparse verification attention.

    Attributes (tree_sparse_flashattn.py:15-41):
        row_ptr: CSR row pointer over Q blocks, int32 [n_q_blocks + 1].
        col_idx: CSR column indices of tree KV blocks, int32 [nnz_blocks].
        blk_type: FULL(0) or MIXED(1) per nnz block, int8 [nnz_blocks].
        mixed_mask_payload: packed MIXED bitsets, int32 [n_mixed * ceil(BM*BN/32)].
        mixed_mask_offset: payload offset per nnz block (0 for FULL), int32
            [nnz_blocks]; EMPTY when there is no MIXED block.
        n_q_blocks, n_tree_blocks, block_m, block_n, prefix_len: ints.
    """

    row_ptr: torch.Tensor
    col_idx: torch.Tensor
    blk_type: torch.Tensor
    mixed_mask_payload: torch.Tensor
    mixed_mask_offset: torch.Tensor
    n_q_blocks: int
    n_tree_blocks: int
    block_m: int
    block_n: int
    prefix_len: int


@dataclass
class BatchedTreeSparseMetadata:
    """Trees in capacity layout (cap = n_q_blocks*n_tree_blocks), on the device.

    row_ptr [S, n_q_blocks+1]; col_idx, blk_type, mixed_mask_offset [S, cap];
    mixed_mask_payload [S, cap*W]; counts [S, 2] int32 = (nnz, n_mixed) of
    each tree, left on the device: the forward reads only the entries below
    row_ptr[n_q_blocks], so building and using the record never waits for the
    host.  S is the batch (one tree per sequence) or 1 (one tree for every
    sequence).  ``nnz`` / ``n_mixed`` read the counts back on first use;
    ``sequence(b)`` returns the reference-shaped record of tree b.
    """

    row_ptr: torch.Tensor
    col_idx: torch.Tensor
    blk_type: torch.Tensor
    mixed_mask_payload: torch.Tensor
    mixed_mask_offset: torch.Tensor
    counts: torch.Tensor
    n_q_blocks: int
    n_tree_blocks: int
    block_m: int
    block_n: int
    prefix_len: int
    _host_counts: Optional[List[List[int]]] = field(default=None, repr=False, compare=False)

    @property
    def n_trees(self) -> int:
        return self.row_ptr.shape[0]

    @property
    def words_per_block(self) -> int:
        return (self.block_m * self.block_n + 31) // 32

    def _counts(self) -> List[List[int]]:
        if self._host_counts is None:
            self._host_counts = [[int(x) for x in row] for row in self.counts.cpu().tolist()]
        return self._host_counts

    @property
    def nnz(self) -> List[int]:
        return [c[0] for c in self._counts()]

    @property
    def n_mixed(self) -> List[int]:
        return [c[1] for c in self._counts()]

    def sequence(self, b: int) -> TreeSparseMetadata:
        nnz, nmx, w = self.nnz[b], self.n_mixed[b], self.words_per_block
        return TreeSparseMetadata(
            row_ptr=self.row_ptr[b],
            col_idx=self.col_idx[b, :nnz],
            blk_type=self.blk_type[b, :nnz],
            mixed_mask_payload=self.mixed_mask_payload[b, : nmx * w],
            mixed_mask_offset=self.mixed_mask_offset[b, :nnz] if nmx > 0 else self.mixed_mask_offset[b, :0],
            n_q_blocks=self.n_q_blocks,
            n_tree_blocks=self.n_tree_blocks,
            block_m=self.block_m,
            block_n=self.block_n,
            prefix_len=self.prefix_len,
        )


def _pack_block_mask_to_int32(mask_2d: torch.Tensor) -> torch.Tensor:
    """Pack a bool [BLOCK_M, BLOCK_N] block row-major into int32 words.

    Bit i of word w is flat[32w + i] (tree_sparse_flashattn.py:44-64); the
    result lives on the input's device: a CPU block is packed on the host
    (tsfa_pack_bits_host), a device block on its device (tsfa_pack_bits).
    """
    lib = _lib.load()
    flat = mask_2d.reshape(-1)
    if flat.dtype != torch.bool:
        flat = flat != 0
    flat = flat.contiguous().view(torch.uint8)
    n_bits = flat.numel()
    out = torch.zeros(((n_bits + 31) // 32,), dtype=torch.int32, device=flat.device)
    if not flat.is_cuda:
        _lib.check("_pack_block_mask_to_int32", lib.tsfa_pack_bits_host(_lib.ptr(flat), n_bits, _lib.ptr(out)))
        return out
    with torch.cuda.device(flat.device):
        _lib.check("_pack_block_mask_to_int32", lib.tsfa_pack_bits(_lib.ptr(flat), n_bits, _lib.ptr(out),
                                                                   _lib.stream_handle(flat.device)))
    return out


# validated geometry and buffer layout of metadata builds, by shape and block size
_META_GEOMETRY: dict = {}


def _meta_build(masks_u8: torch.Tensor, block_m: int, block_n: int, dev: torch.device):
    """tsfa_meta_build over [n_seq, q_len, q_len] uint8 masks on `dev` (a HIP
    device), or tsfa_meta_build_host when `dev` is the CPU."""
    lib = _lib.load()
    n_seq, q_len = masks_u8.shape[0], masks_u8.shape[1]
    geo_key = (n_seq, q_len, block_m, block_n, dev.type)
    geo = _META_GEOMETRY.get(geo_key)
    if geo is None:
        _lib.check("prepare_tree_sparse_metadata", lib.tsfa_meta_check_args(n_seq, q_len, block_m, block_n))
        nqb = (q_len + block_m - 1) // block_m
        ntb = (q_len + block_n - 1) // block_n
        words = (block_m * block_n + 31) // 32
        cap = nqb * ntb
        # one allocation holds the six outputs (256-byte aligned sections)
        # and, on a device, the build's workspace
        sections = ((n_seq * (nqb + 1), torch.int32), (n_seq * cap, torch.int32), (n_seq * cap, torch.int8),
                    (n_seq * cap * words, torch.int32), (n_seq * cap, torch.int32), (n_seq * 2, torch.int32))
        ws_bytes = 0 if dev.type == "cpu" else lib.tsfa_meta_workspace_bytes(n_seq, q_len, block_m, block_n)
        spans, at = [], 0
        for n, dt in sections:
            nbytes = n * (4 if dt == torch.int32 else 1)
            spans.append((at, at + nbytes, dt))
            at += (nbytes + 255) // 256 * 256
        geo = (nqb, ntb, words, cap, tuple(spans), at, ws_bytes)
        if len(_META_GEOMETRY) >= 64:
            _META_GEOMETRY.clear()
        _META_GEOMETRY[geo_key] = geo
    nqb, ntb, words, cap, spans, at, ws_bytes = geo
    buf = torch.empty((at + max(ws_bytes, 1),), dtype=torch.uint8, device=dev)
    views = [buf[a:b].view(dt) for a, b, dt in spans]
    row_ptr = views[0].view(n_seq, nqb + 1)
    col_idx, blk_type, offset = (views[i].view(n_seq, cap) for i in (1, 2, 4))
    payload = views[3].view(n_seq, cap * words)
    counts = views[5].view(n_seq, 2)
    if dev.type == "cpu":
        st = lib.tsfa_meta_build_host(_lib.ptr(masks_u8), masks_u8.stride(0), masks_u8.stride(1), n_seq, q_len,
                                      block_m, block_n, _lib.ptr(row_ptr), _lib.ptr(col_idx), _lib.ptr(blk_type),
                                      _lib.ptr(payload), _lib.ptr(offset), _lib.ptr(counts))
        _lib.check("prepare_tree_sparse_metadata", st)
        return row_ptr, col_idx, blk_type, payload, offset, counts, nqb, ntb
    ws = buf[at:]
    with torch.cuda.device(dev):
        st = lib.tsfa_meta_build(_lib.ptr(masks_u8), masks_u8.stride(0), masks_u8.stride(1), n_seq, q_len,
                                 block_m, block_n, _lib.ptr(row_ptr), _lib.ptr(col_idx), _lib.ptr(blk_type),
                                 _lib.ptr(payload), _lib.ptr(offset), _lib.ptr(counts), _lib.ptr(ws), ws_bytes,
                                 _lib.stream_handle(dev))
    _lib.check("prepare_tree_sparse_metadata", st)
    return row_ptr, col_idx, blk_type, payload, offset, counts, nqb, ntb


def _masks_u8(tree_masks: torch.Tensor) -> torch.Tensor:
    m = tree_masks
    if m.dtype != torch.bool:
        m = m != 0  # nonzero -> visible, NaN included (tree_sparse_flashattn.py:90)
    # the host builder reads rows at least q_len apart (an expanded mask with
    # row stride 0 is made dense first, as the reference's .contiguous()
    # does); the device builder reads any row stride
    if m.stride(-1) != 1 or (m.device.type == "cpu" and m.stride(-2) < m.shape[-1]):
        m = m.contiguous()
    return m.view(torch.uint8)


def prepare_tree_sparse_metadata(
    tree_mask: torch.Tensor,
    prefix_len: int,
    BLOCK_M: int,
    BLOCK_N: int,
) -> TreeSparseMetadata:
    """Generate CSR + tri-state metadata for block-sparse tree attention.

    Same contract as tree_sparse_flashattn.py:67-160: ``tree_mask`` is a
    [q_len, q_len] tensor of any dtype (nonzero = visible); ValueError for a
    non-square mask or non-positive block sizes.  The tensors come back on the
    mask's device: a CPU mask is processed on the host (tsfa_meta_build_host,
    no device needed, as the reference runs it), a device mask on its device.
    """
    if tree_mask.ndim != 2 or tree_mask.shape[0] != tree_mask.shape[1]:
        raise ValueError("tree_mask must be shape [q_len, q_len].")
    if BLOCK_M <= 0 or BLOCK_N <= 0:
        raise ValueError("BLOCK_M and BLOCK_N must be positive.")
    masks = _masks_u8(tree_mask).unsqueeze(0)
    row_ptr, col_idx, blk_type, payload, offset, counts, nqb, ntb = _meta_build(masks, BLOCK_M, BLOCK_N,
                                                                                tree_mask.device)
    nnz, n_mixed = (int(x) for x in counts[0].tolist())
    words = (BLOCK_M * BLOCK_N + 31) // 32
    return TreeSparseMetadata(
        row_ptr=row_ptr[0],
        col_idx=col_idx[0, :nnz],
        blk_type=blk_type[0, :nnz],
        mixed_mask_payload=payload[0, : n_mixed * words],
        mixed_mask_offset=offset[0, :nnz] if n_mixed > 0 else offset[0, :0],
        n_q_blocks=nqb,
        n_tree_blocks=ntb,
        block_m=BLOCK_M,
        block_n=BLOCK_N,
        prefix_len=prefix_len,
    )


def prepare_tree_sparse_metadata_batched(
    tree_masks: torch.Tensor,
    prefix_len: int,
    BLOCK_M: int,
    BLOCK_N: int,
) -> BatchedTreeSparseMetadata:
    """Metadata for [S, q_len, q_len] masks (one tree per sequence), or for one
    [q_len, q_len] mask shared by the whole batch (S = 1), in one launch and
    without a host synchronisation (the record stays in capacity layout).
    CPU masks are processed on the host and give a CPU record."""
    if tree_masks.ndim == 2:
        tree_masks = tree_masks.unsqueeze(0)
    if tree_masks.ndim != 3 or tree_masks.shape[1] != tree_masks.shape[2]:
        raise ValueError("tree_masks must be shape [batch, q_len, q_len] or [q_len, q_len].")
    if BLOCK_M <= 0 or BLOCK_N <= 0:
        raise ValueError("BLOCK_M and BLOCK_N must be positive.")
    masks = _masks_u8(tree_masks)
    row_ptr, col_idx, blk_type, payload, offset, counts, nqb, ntb = _meta_build(masks, BLOCK_M, BLOCK_N,
                                                                                tree_masks.device)
    return BatchedTreeSparseMetadata(
        row_ptr=row_ptr, col_idx=col_idx, blk_type=blk_type, mixed_mask_payload=payload,
        mixed_mask_offset=offset, counts=counts, n_q_blocks=nqb, n_tree_blocks=ntb, block_m=BLOCK_M,
        block_n=BLOCK_N, prefix_len=prefix_len)


def _workspace(workspace: Optional[torch.Tensor], nbytes: int, dev: torch.device) -> torch.Tensor:
    """The caller's workspace (a uint8 device tensor of at least ``nbytes``) or a new one."""
    if workspace is None:
        return torch.empty((max(nbytes, 1),), dtype=torch.uint8, device=dev)
    if workspace.device != dev or workspace.dtype != torch.uint8 or not workspace.is_contiguous():
        raise ValueError(f"workspace must be a contiguous uint8 tensor on {dev}")
    if workspace.numel() < nbytes:
        raise ValueError(f"workspace holds {workspace.numel()} bytes, the call needs {nbytes}")
    return workspace


def fwd_workspace_bytes(q: torch.Tensor, k: torch.Tensor, meta) -> int:
    """Bytes of the split-KV workspace tree_sparse_attention_fwd(q, k, v, meta) uses."""
    bsz, n_heads, q_len, head_dim = q.shape
    return int(_lib.load().tsfa_fwd_workspace_bytes_for_dtype(bsz, n_heads, k.shape[1], q_len, k.shape[2],
                                                              meta.prefix_len, head_dim, _lib.dtype_code(q.dtype)))


def _launch_fwd(q, k, v, o, row_ptr, col_idx, blk_type, payload, offset, meta_strides, strides, sm_scale,
                batch_size, num_heads, num_kv_heads, q_len, kv_len, prefix_len, n_q_blocks, n_tree_blocks,
                gqa_group_size, block_m, block_n, head_dim, lse=None, workspace=None):
    lib = _lib.load()
    for name, t in (("q", q), ("k", k), ("v", v), ("o", o)):
        if not t.is_cuda:
            raise ValueError(f"{name} must be a HIP device tensor")
    dev = q.device
    for name, t in (("row_ptr", row_ptr), ("col_idx", col_idx), ("blk_type", blk_type),
                    ("mixed_mask_payload", payload), ("mixed_mask_offset", offset)):
        if t.device != dev:
            raise ValueError(f"{name} must be on {dev} (move the metadata to the device first)")
    if not (q.dtype == k.dtype == v.dtype == o.dtype):
        raise NotImplementedError("q, k, v and o must share one dtype")
    dt = _lib.dtype_code(q.dtype)
    args = (batch_size, num_heads, num_kv_heads, q_len, kv_len, prefix_len, n_q_blocks, n_tree_blocks,
            gqa_group_size, block_m, block_n, head_dim, dt)
    _lib.check("block_sparse_tree_fwd_kernel", lib.tsfa_fwd_check_args(*args))
    ws_bytes = lib.tsfa_fwd_workspace_bytes_for_dtype(batch_size, num_heads, num_kv_heads, q_len, kv_len,
                                                      prefix_len, head_dim, dt)
    ws = _workspace(workspace, ws_bytes, dev)
    with torch.cuda.device(dev):
        if lse is None:
            st = lib.tsfa_fwd(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(o), _lib.ptr(row_ptr),
                              _lib.ptr(col_idx), _lib.ptr(blk_type), _lib.ptr(payload), _lib.ptr(offset),
                              _lib.i64_array(meta_strides), _lib.i64_array(strides), float(sm_scale), *args,
                              _lib.ptr(ws), ws_bytes, _lib.stream_handle(dev))
        else:
            st = lib.tsfa_fwd_lse(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(o), _lib.ptr(lse),
                                  _lib.ptr(row_ptr), _lib.ptr(col_idx), _lib.ptr(blk_type), _lib.ptr(payload),
                                  _lib.ptr(offset), _lib.i64_array(meta_strides), _lib.i64_array(strides),
                                  float(sm_scale), *args, _lib.ptr(ws), ws_bytes, _lib.stream_handle(dev))
    _lib.check("block_sparse_tree_fwd_kernel", st)
    return o


class _BlockSparseTreeFwdKernel:
    """``block_sparse_tree_fwd_kernel[grid](...)`` with the reference's arguments.

    Positional arguments follow tree_sparse_flashattn.py:164-199 (9 tensors,
    16 strides, sm_scale, 10 ints); BLOCK_M/BLOCK_N/BLOCK_D are keywords as in
    the reference.  ``grid`` and Triton launch options (num_warps,
    num_stages) are accepted and ignored: the HIP forward chooses its own
    split-KV decomposition.  The launch is asynchronous on the current stream
    of q's device.
    """

    def __getitem__(self, grid):
        def launch(q_ptr, k_ptr, v_ptr, o_ptr, row_ptr_ptr, col_idx_ptr, blk_type_ptr, mixed_mask_payload_ptr,
                   mixed_mask_offset_ptr, stride_qb, stride_qh, stride_qm, stride_qd, stride_kb, stride_kh,
                   stride_kn, stride_kd, stride_vb, stride_vh, stride_vn, stride_vd, stride_ob, stride_oh,
                   stride_om, stride_od, sm_scale, batch_size, num_heads, num_kv_heads, q_len, kv_len, prefix_len,
                   n_q_blocks, n_tree_blocks, gqa_group_size, *, BLOCK_M, BLOCK_N, BLOCK_D, num_warps=None,
                   num_stages=None, **_unused):
            if BLOCK_D != q_ptr.shape[-1]:
                raise ValueError(f"BLOCK_D ({BLOCK_D}) must equal head_dim ({q_ptr.shape[-1]})")
            # the reference addresses each operand by its base pointer and the
            # strides given here (tree_sparse_flashattn.py:174-189): the same
            # views of the tensors' storage
            qv = _strided(q_ptr, (batch_size, num_heads, q_len, BLOCK_D), (stride_qb, stride_qh, stride_qm, stride_qd))
            kv_shape = (batch_size, num_kv_heads, kv_len, BLOCK_D)
            kv_ = _strided(k_ptr, kv_shape, (stride_kb, stride_kh, stride_kn, stride_kd))
            vv = _strided(v_ptr, kv_shape, (stride_vb, stride_vh, stride_vn, stride_vd))
            ov = _strided(o_ptr, (batch_size, num_heads, q_len, BLOCK_D), (stride_ob, stride_oh, stride_om, stride_od))
            dp = _padded_dim(BLOCK_D)
            direct = dp == BLOCK_D and all(_layout_ok(t) for t in (qv, kv_, vv, ov))
            if direct:
                qc, kc, vc, oc = qv, kv_, vv, ov
            else:
                # head_dim zero-padded to a kernel width (zeros add nothing to
                # q.k and give zero columns of O) and layouts the kernel does
                # not address (d stride != 1, unaligned rows) copied
                qc, kc, vc = (_dense_padded(t, dp) for t in (qv, kv_, vv))
                oc = torch.empty((batch_size, num_heads, q_len, dp), dtype=ov.dtype, device=ov.device)
            strides = (*qc.stride(), *kc.stride(), *vc.stride(), *oc.stride())
            _launch_fwd(qc, kc, vc, oc, row_ptr_ptr, col_idx_ptr, blk_type_ptr, mixed_mask_payload_ptr,
                        mixed_mask_offset_ptr, (0, 0, 0, 0, 0), strides, sm_scale, batch_size, num_heads,
                        num_kv_heads, q_len, kv_len, prefix_len, n_q_blocks, n_tree_blocks, gqa_group_size,
                        BLOCK_M, BLOCK_N, dp)
            if not direct:
                ov.copy_(oc[..., :BLOCK_D])
            return o_ptr

        return launch

    def __call__(self, *args, **kwargs):
        raise TypeError("launch with block_sparse_tree_fwd_kernel[grid](...)")


block_sparse_tree_fwd_kernel = _BlockSparseTreeFwdKernel()


def _check_qkv(q: torch.Tensor, k: torch.Tensor, v: Optional[torch.Tensor], **same_as_q) -> None:
    """Shape checks the C-ABI cannot make (it sees strides only): q [B,Hq,T,D],
    k and v [B,Hkv,L,D] with Hq a multiple of Hkv, and each keyword tensor
    (out, dq, ...) of q's shape; ``dk``/``dv`` keywords must have k's shape.
    Raised before any launch (eagle_tree_sparse_bridge.py:84-87 asserts the
    same of its inputs)."""
    if q.dim() != 4 or k.dim() != 4:
        raise ValueError(f"q and k must be 4-D [B, H, L, D], got {tuple(q.shape)} and {tuple(k.shape)}")
    if v is not None and tuple(v.shape) != tuple(k.shape):
        raise ValueError(f"v shape {tuple(v.shape)} != k shape {tuple(k.shape)}")
    if k.shape[0] != q.shape[0]:
        raise ValueError(f"k batch {k.shape[0]} != q batch {q.shape[0]}")
    if k.shape[3] != q.shape[3]:
        raise ValueError(f"k head_dim {k.shape[3]} != q head_dim {q.shape[3]}")
    if k.shape[1] < 1 or q.shape[1] % k.shape[1]:
        raise ValueError(f"num_heads {q.shape[1]} must be a multiple of num_kv_heads {k.shape[1]}")
    for name, t in same_as_q.items():
        if t is None:
            continue
        want = k.shape if name in ("dk", "dv") else q.shape
        if tuple(t.shape) != tuple(want):
            raise ValueError(f"{name} shape {tuple(t.shape)} != {tuple(want)}")


# head_dim widths the kernels are built for; narrower dims are zero-padded
_KERNEL_DIMS = (64, 128, 256)


def _padded_dim(d: int) -> int:
    for w in _KERNEL_DIMS:
        if d <= w:
            return w
    raise NotImplementedError(f"head_dim {d} is above the widest kernel ({_KERNEL_DIMS[-1]})")


def _strided(t: torch.Tensor, size, stride) -> torch.Tensor:
    return torch.as_strided(t, size, [int(x) for x in stride])


def _layout_ok(t: torch.Tensor) -> bool:
    # what the kernels address directly: d stride 1, 16-byte aligned rows
    return t.stride(-1) == 1 and not any(st % 8 for st in t.stride()[:-1]) and t.data_ptr() % 16 == 0


def _dense_padded(t: torch.Tensor, width: int) -> torch.Tensor:
    if t.shape[-1] == width:
        return t.contiguous() if not _layout_ok(t) else t
    out = torch.zeros((*t.shape[:-1], width), dtype=t.dtype, device=t.device)
    out[..., : t.shape[-1]] = t
    return out


def _row_contig(t: torch.Tensor) -> torch.Tensor:
    if t.stride(-1) != 1 or any(s % 8 for s in t.stride()[:-1]) or t.data_ptr() % 16:
        return t.contiguous()
    return t


def _meta_arrays(meta, bsz: int):
    """The five metadata arrays and their per-sequence strides (0: one tree for all)."""
    tensors = (meta.row_ptr, meta.col_idx, meta.blk_type, meta.mixed_mask_payload, meta.mixed_mask_offset)
    if isinstance(meta, BatchedTreeSparseMetadata):
        if meta.n_trees not in (1, bsz):
            raise ValueError("batched metadata must have one tree per sequence, or one tree for all")
        if meta.n_trees > 1:
            return tensors, tuple(t.stride(0) for t in tensors)
    return tensors, (0, 0, 0, 0, 0)


def tree_sparse_attention_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, meta, *,
                              sm_scale: Optional[float] = None, out: Optional[torch.Tensor] = None,
                              return_lse: bool = False, workspace: Optional[torch.Tensor] = None):
    """O = tree-sparse attention of q [B,Hq,T,D] over k/v [B,Hkv,P+T,D].

    ``meta`` is a TreeSparseMetadata (one tree for the whole batch) or a
    BatchedTreeSparseMetadata (one tree per sequence, or one tree for every
    sequence), already on q's device.  With ``return_lse`` the result is
    ``(O, lse)``: lse [B, Hq, T] fp32 is the natural-log log-sum-exp of each
    row's visible scaled scores (-inf for a row with no visible key), what
    tree_sparse_attention_bwd needs.  ``workspace`` optionally supplies the
    split-KV partials buffer (uint8, ``fwd_workspace_bytes`` of the shape).
    """
    # repeated calls of one geometry skip the host checks the first call made
    # (the C entry point still validates every argument)
    key = _fwd_key(q, k, v, meta, out, return_lse)
    entry = _FWD_CALLS.get(key)
    if entry is not None:
        return _fwd_cached(entry, q, k, v, meta, sm_scale, out, return_lse, workspace)
    _check_qkv(q, k, v, out=out)
    q_in, k_in, v_in = q, k, v
    head_dim = q.shape[-1]
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(head_dim)
    if _padded_dim(head_dim) != head_dim:
        # head_dim below a kernel width: zero-padded copies (no change to q.k)
        dp = _padded_dim(head_dim)
        res = tree_sparse_attention_fwd(_dense_padded(q, dp), _dense_padded(k, dp), _dense_padded(v, dp), meta,
                                        sm_scale=sm_scale, return_lse=return_lse, workspace=workspace)
        o = res[0] if return_lse else res
        if out is None:
            out = o[..., :head_dim].contiguous()
        else:
            out.copy_(o[..., :head_dim])
        return (out, res[1]) if return_lse else out
    if out is not None and not _layout_ok(out):
        # an output the kernel cannot address (d stride != 1, unaligned rows)
        # is written through a dense temporary
        res = tree_sparse_attention_fwd(q, k, v, meta, sm_scale=sm_scale, return_lse=return_lse,
                                        workspace=workspace)
        out.copy_(res[0] if return_lse else res)
        return (out, res[1]) if return_lse else out
    q, k, v = _row_contig(q), _row_contig(k), _row_contig(v)
    bsz, n_heads, q_len, head_dim = q.shape
    _, n_kv_heads, kv_len, _ = k.shape
    if out is None:
        out = torch.empty_like(q)
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(head_dim)
    tensors, meta_strides = _meta_arrays(meta, bsz)
    strides = (*q.stride(), *k.stride(), *v.stride(), *out.stride())
    lse = torch.empty((bsz, n_heads, q_len), dtype=torch.float32, device=q.device) if return_lse else None
    _launch_fwd(q, k, v, out, *tensors, meta_strides, strides, sm_scale, bsz, n_heads, n_kv_heads, q_len,
                kv_len, meta.prefix_len, meta.n_q_blocks, meta.n_tree_blocks, n_heads // n_kv_heads,
                meta.block_m, meta.block_n, head_dim, lse=lse, workspace=workspace)
    if key is not None and q is q_in and k is k_in and v is v_in:
        # the geometry ran as given (no copies): remember its launch arguments
        if len(_FWD_CALLS) >= 64:
            _FWD_CALLS.clear()
        lib = _lib.load()
        _FWD_CALLS[key] = (
            _lib.i64_array(meta_strides), _lib.i64_array(strides),
            (bsz, n_heads, n_kv_heads, q_len, kv_len, meta.prefix_len, meta.n_q_blocks, meta.n_tree_blocks,
             n_heads // n_kv_heads, meta.block_m, meta.block_n, head_dim, _lib.dtype_code(q.dtype)),
            lib.tsfa_fwd_workspace_bytes_for_dtype(bsz, n_heads, n_kv_heads, q_len, kv_len, meta.prefix_len,
                                                   head_dim, _lib.dtype_code(q.dtype)),
            1.0 / math.sqrt(head_dim))
    return (out, lse) if return_lse else out


# launch arguments of forward geometries already validated, by _fwd_key
_FWD_CALLS: dict = {}


def reload_config() -> None:
    """Re-read the TSFA_* environment switches (the library reads them once)
    and forget launch arguments planned under the old ones."""
    _lib.check("tsfa_config_reload", _lib.load().tsfa_config_reload())
    _FWD_CALLS.clear()


def _fwd_key(q, k, v, meta, out, return_lse):
    """Everything a forward's validation and launch arguments depend on,
    pointers excepted (their 16-byte alignment included)."""
    if not (q.is_cuda and k.is_cuda and v.is_cuda) or (out is not None and not out.is_cuda):
        return None
    tensors = (meta.row_ptr, meta.col_idx, meta.blk_type, meta.mixed_mask_payload, meta.mixed_mask_offset)
    align = q.data_ptr() | k.data_ptr() | v.data_ptr() | (0 if out is None else out.data_ptr())
    return (q.shape, q.stride(), k.shape, k.stride(), v.shape, v.stride(), q.dtype, k.dtype, v.dtype,
            None if out is None else (out.shape, out.stride(), out.dtype), align & 15, q.device,
            tuple(t.device for t in tensors), type(meta), getattr(meta, "n_trees", 0),
            tuple(t.stride(0) for t in tensors) if isinstance(meta, BatchedTreeSparseMetadata) else None,
            meta.prefix_len, meta.n_q_blocks, meta.n_tree_blocks, meta.block_m, meta.block_n, return_lse)


def _fwd_cached(entry, q, k, v, meta, sm_scale, out, return_lse, workspace):
    meta_strides, strides, args, ws_bytes, default_scale = entry
    lib = _lib.load()
    dev = q.device
    if out is None:
        out = torch.empty_like(q)
    ws = _workspace(workspace, ws_bytes, dev)
    scale = default_scale if sm_scale is None else float(sm_scale)
    tensors = (meta.row_ptr, meta.col_idx, meta.blk_type, meta.mixed_mask_payload, meta.mixed_mask_offset)
    ptrs = (q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), *(t.data_ptr() for t in tensors))
    lse = torch.empty((args[0], args[1], args[3]), dtype=torch.float32, device=dev) if return_lse else None

    def launch():
        stream = _lib.stream_handle(dev)
        if return_lse:
            return lib.tsfa_fwd_lse(*ptrs[:4], lse.data_ptr(), *ptrs[4:], meta_strides, strides, scale, *args,
                                    ws.data_ptr(), ws_bytes, stream)
        return lib.tsfa_fwd(*ptrs, meta_strides, strides, scale, *args, ws.data_ptr(), ws_bytes, stream)

    # the device guard only when q is not on the current device (~1.2 us)
    if dev.index == torch.cuda.current_device():
        st = launch()
    else:
        with torch.cuda.device(dev):
            st = launch()
    _lib.check("block_sparse_tree_fwd_kernel", st)
    return (out, lse) if return_lse else out


def tree_sparse_attention_bwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, o: torch.Tensor,
                              lse: torch.Tensor, dout: torch.Tensor, meta, *, sm_scale: Optional[float] = None,
                              dq: Optional[torch.Tensor] = None, dk: Optional[torch.Tensor] = None,
                              dv: Optional[torch.Tensor] = None):
    """(dQ, dK, dV) of tree-sparse attention for the upstream gradient ``dout``.

    ``o`` and ``lse`` are the forward's outputs (tree_sparse_attention_fwd
    with return_lse=True) for the same q, k, v, meta and sm_scale.  dK / dV
    sum over the query heads of each kv head (GQA); rows with no visible key
    contribute nothing and get dQ = 0.  No counterpart in the reference, which
    has no backward (README.md:198).
    """
    _check_qkv(q, k, v, o=o, dout=dout, dq=dq, dk=dk, dv=dv)
    q, k, v, o, dout = (_row_contig(t) for t in (q, k, v, o, dout))
    bsz, n_heads, q_len, head_dim = q.shape
    _, n_kv_heads, kv_len, _ = k.shape
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(head_dim)
    if tuple(o.shape) != tuple(q.shape) or tuple(dout.shape) != tuple(q.shape):
        raise ValueError("o and dout must have q's shape")
    if tuple(v.shape) != tuple(k.shape):
        raise ValueError("k and v must have the same shape")
    if lse.dtype != torch.float32 or tuple(lse.shape) != (bsz, n_heads, q_len):
        raise ValueError(f"lse must be float32 [{bsz}, {n_heads}, {q_len}]")
    lse = lse.contiguous()
    dq = torch.empty_like(q) if dq is None else dq
    dk = torch.empty_like(k) if dk is None else dk
    dv = torch.empty_like(v) if dv is None else dv
    lib = _lib.load()
    tensors, meta_strides = _meta_arrays(meta, bsz)
    for name, t in (("q", q), ("k", k), ("v", v), ("o", o), ("lse", lse), ("dout", dout), ("dq", dq), ("dk", dk),
                    ("dv", dv)):
        if not t.is_cuda:
            raise ValueError(f"{name} must be a HIP device tensor")
        if t.device != q.device:
            raise ValueError(f"{name} must be on {q.device}")
    for name, t in zip(("row_ptr", "col_idx", "blk_type", "mixed_mask_payload", "mixed_mask_offset"), tensors):
        if t.device != q.device:
            raise ValueError(f"{name} must be on {q.device} (move the metadata to the device first)")
    if not (q.dtype == k.dtype == v.dtype == o.dtype == dout.dtype == dq.dtype == dk.dtype == dv.dtype):
        raise NotImplementedError("q, k, v, o, dout and the gradients must share one dtype")
    dt = _lib.dtype_code(q.dtype)
    args = (bsz, n_heads, n_kv_heads, q_len, kv_len, meta.prefix_len, meta.n_q_blocks, meta.n_tree_blocks,
            n_heads // n_kv_heads, meta.block_m, meta.block_n, head_dim, dt)
    _lib.check("tree_sparse_attention_bwd", lib.tsfa_fwd_check_args(*args))
    n_trees = bsz if any(meta_strides) else 1
    ws_bytes = lib.tsfa_bwd_workspace_bytes(bsz, n_heads, n_kv_heads, q_len, kv_len, meta.prefix_len, meta.block_m,
                                            meta.n_tree_blocks, head_dim, n_trees)
    if ws_bytes == 0 and bsz > 0 and q_len > 0:
        raise NotImplementedError("tree_sparse_attention_bwd: tree too large for the backward's tables")
    ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=q.device)
    strides = (*q.stride(), *k.stride(), *v.stride(), *o.stride(), *dout.stride(), *dq.stride(), *dk.stride(),
               *dv.stride())
    with torch.cuda.device(q.device):
        st = lib.tsfa_bwd(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(o), _lib.ptr(lse), _lib.ptr(dout),
                          _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv), *(_lib.ptr(t) for t in tensors),
                          _lib.i64_array(meta_strides), _lib.i64_array(strides), float(sm_scale), *args,
                          _lib.ptr(ws), ws_bytes, _lib.stream_handle(q.device))
    _lib.check("tree_sparse_attention_bwd", st)
    return dq, dk, dv


class TreeSparseAttentionFunction(torch.autograd.Function):
    """Differentiable tree-sparse attention: forward = tree_sparse_attention_fwd
    (saving O and the row LSE), backward = tree_sparse_attention_bwd."""

    @staticmethod
    def forward(ctx, q, k, v, meta, sm_scale):
        o, lse = tree_sparse_attention_fwd(q, k, v, meta, sm_scale=sm_scale, return_lse=True)
        ctx.save_for_backward(q, k, v, o, lse)
        ctx.meta = meta
        ctx.sm_scale = sm_scale
        return o

    @staticmethod
    def backward(ctx, dout):
        q, k, v, o, lse = ctx.saved_tensors
        dq, dk, dv = tree_sparse_attention_bwd(q, k, v, o, lse, dout, ctx.meta, sm_scale=ctx.sm_scale)
        return dq, dk, dv, None, None


def tree_sparse_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, meta,
                          sm_scale: Optional[float] = None) -> torch.Tensor:
    """tree_sparse_attention_fwd with autograd support (dQ, dK, dV on the HIP backward)."""
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(q.shape[-1])
    return TreeSparseAttentionFunction.apply(q, k, v, meta, sm_scale)


def tree_sparse_attention_fwd_paged(q: torch.Tensor, kv_cache: torch.Tensor, kv_indices: torch.Tensor, meta, *,
                                    kv_len: int, kv_indptr: Optional[torch.Tensor] = None,
                                    kv_layout: str = "NHD", sm_scale: Optional[float] = None,
                                    out: Optional[torch.Tensor] = None, return_lse: bool = False):
    """tree_sparse_attention_fwd with K/V read in place from a paged cache.

    kv_cache: [pages, 2, page_size, Hkv, D] (kv_layout "NHD": FlashInfer's
        default, the cache benchmark.py:67-91 builds) or [pages, 2, Hkv,
        page_size, D] ("HND"); slot 0 holds K, slot 1 V.  page_size must be
        a power of two >= 16.
    kv_indices / kv_indptr: FlashInfer's page lists -- sequence b's pages are
        kv_indices[kv_indptr[b]:kv_indptr[b + 1]] (int32, kv_indptr [B + 1]);
        without kv_indptr, kv_indices is a dense int32 [B, pages_per_seq]
        table.  Key j of sequence b is row j % page_size of its page
        j // page_size.
    kv_len: keys of every sequence (prefix_len + tree tokens).
    The metadata, scale and output are those of tree_sparse_attention_fwd;
    O equals tree_sparse_attention_fwd over the gathered [B, Hkv, kv_len, D]
    K/V bit for bit.  Page ids outside the cache and list positions outside
    kv_indices are clamped in the kernel (wrong O, never an invalid read).
    With ``return_lse`` the result is ``(O, lse)`` as in
    tree_sparse_attention_fwd.
    """
    if q.dim() != 4:
        raise ValueError(f"q must be 4-D [B, Hq, T, D], got {tuple(q.shape)}")
    if out is not None and tuple(out.shape) != tuple(q.shape):
        raise ValueError(f"out shape {tuple(out.shape)} != q shape {tuple(q.shape)}")
    q = _row_contig(q)
    bsz, n_heads, q_len, head_dim = q.shape
    if kv_cache.dim() != 5 or kv_cache.shape[1] != 2:
        raise ValueError("kv_cache must be [pages, 2, page_size, Hkv, D] (NHD) or [pages, 2, Hkv, page_size, D] (HND)")
    if kv_layout == "NHD":
        n_pages, _, page_size, n_kv_heads, kv_dim = kv_cache.shape
        cache_strides = tuple(kv_cache.stride())
    elif kv_layout == "HND":
        n_pages, _, n_kv_heads, page_size, kv_dim = kv_cache.shape
        sp, ss, sh, sr, sd = kv_cache.stride()
        cache_strides = (sp, ss, sr, sh, sd)
    else:
        raise ValueError(f"kv_layout must be 'NHD' or 'HND', got {kv_layout!r}")
    if kv_dim != head_dim:
        raise ValueError(f"kv_cache head_dim {kv_dim} != q head_dim {head_dim}")
    if n_kv_heads <= 0 or n_heads % n_kv_heads:
        raise ValueError("num_heads must be a multiple of the cache's kv heads")
    if page_size < 16 or page_size & (page_size - 1):
        raise NotImplementedError(f"page_size must be a power of two >= 16, got {page_size}")
    if kv_indices.dtype != torch.int32 or (kv_indptr is not None and kv_indptr.dtype != torch.int32):
        raise ValueError("kv_indices and kv_indptr must be int32")
    if kv_len < meta.prefix_len:
        raise ValueError("kv_len must be >= prefix_len")
    pages_per_seq = -(-kv_len // page_size)
    if kv_indptr is None:
        if kv_indices.dim() != 2 or kv_indices.shape[0] != bsz or kv_indices.shape[1] < pages_per_seq:
            raise ValueError(f"a dense page table must be [{bsz}, >= {pages_per_seq}] int32")
        if kv_indices.stride(1) != 1:
            kv_indices = kv_indices.contiguous()
        pt_stride = kv_indices.stride(0)
    else:
        if kv_indptr.dim() != 1 or kv_indptr.numel() != bsz + 1:
            raise ValueError(f"kv_indptr must be int32 [{bsz + 1}]")
        kv_indptr, kv_indices = kv_indptr.contiguous(), kv_indices.contiguous().view(-1)
        pt_stride = 0
    if kv_indices.numel() == 0 and bsz > 0 and kv_len > 0:
        raise ValueError("kv_indices is empty")
    if out is None:
        out = torch.empty_like(q)
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(head_dim)
    tensors, meta_strides = _meta_arrays(meta, bsz)

    lib = _lib.load()
    for name, t in (("q", q), ("kv_cache", kv_cache), ("o", out), ("kv_indices", kv_indices)):
        if not t.is_cuda:
            raise ValueError(f"{name} must be a HIP device tensor")
    dev = q.device
    for name, t in (("kv_cache", kv_cache), ("kv_indices", kv_indices), ("kv_indptr", kv_indptr),
                    ("row_ptr", tensors[0]), ("col_idx", tensors[1]), ("blk_type", tensors[2]),
                    ("mixed_mask_payload", tensors[3]), ("mixed_mask_offset", tensors[4])):
        if t is not None and t.device != dev:
            raise ValueError(f"{name} must be on {dev}")
    if not (q.dtype == kv_cache.dtype == out.dtype):
        raise NotImplementedError("q, kv_cache and o must share one dtype")
    dt = _lib.dtype_code(q.dtype)
    args = (bsz, n_heads, n_kv_heads, q_len, kv_len, meta.prefix_len, meta.n_q_blocks, meta.n_tree_blocks,
            n_heads // n_kv_heads, meta.block_m, meta.block_n, head_dim, dt)
    _lib.check("tree_sparse_attention_fwd_paged", lib.tsfa_fwd_check_args(*args))
    ws_bytes = lib.tsfa_fwd_workspace_bytes_for_dtype(bsz, n_heads, n_kv_heads, q_len, kv_len, meta.prefix_len,
                                                      head_dim, dt)
    ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=dev)
    lse = torch.empty((bsz, n_heads, q_len), dtype=torch.float32, device=dev) if return_lse else None
    with torch.cuda.device(dev):
        st = lib.tsfa_fwd_paged(
            _lib.ptr(q), _lib.ptr(kv_cache), _lib.ptr(kv_indptr), _lib.ptr(kv_indices), kv_indices.numel(),
            pt_stride, n_pages, page_size, _lib.ptr(out), _lib.ptr(lse), *(_lib.ptr(t) for t in tensors),
            _lib.i64_array(meta_strides), _lib.i64_array(q.stride()), _lib.i64_array(cache_strides),
            _lib.i64_array(out.stride()), float(sm_scale), *args, _lib.ptr(ws), ws_bytes, _lib.stream_handle(dev))
    _lib.check("tree_sparse_attention_fwd_paged", st)
    return (out, lse) if return_lse else out
