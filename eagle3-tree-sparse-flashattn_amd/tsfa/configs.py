"""Named verification workloads and their seeded synthetic inputs.

Shared input recipe: Q, K, V ~ N(0, 1) drawn in float32 on the CPU from a
seeded ``torch.Generator`` (seed 42 as in benchmark.py:154) and cast to the
workload dtype, so every consumer sees identical values; the softmax scale is
1/sqrt(head_dim) (eagle_tree_sparse_bridge.py:116).  Tree masks come from the
seeded generators in ``tsfa.trees``.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

from . import trees


@dataclass(frozen=True)
class Workload:
    name: str
    batch: int
    q_heads: int
    kv_heads: int
    head_dim: int
    prefix_len: int
    tree_len: int
    dtype: torch.dtype
    block_m: int
    block_n: int
    tree_kind: str            # random | eagle | kary | depth_limited
    tree_args: dict = field(default_factory=dict)
    per_sequence: bool = False  # one tree per batch element
    description: str = ""

    @property
    def kv_len(self) -> int:
        return self.prefix_len + self.tree_len

    @property
    def group(self) -> int:
        return self.q_heads // self.kv_heads

    def kv_bytes(self) -> int:
        """Algorithmic K+V bytes of one forward call (each byte once)."""
        es = torch.tensor([], dtype=self.dtype).element_size()
        return 2 * self.batch * self.kv_heads * self.kv_len * self.head_dim * es

    def with_blocks(self, block_m: int, block_n: int) -> "Workload":
        d = dict(self.__dict__)
        d.update(block_m=block_m, block_n=block_n, name=f"{self.name}-bm{block_m}-bn{block_n}")
        return Workload(**d)


WORKLOADS = {
    w.name: w
    for w in [
        Workload("tiny-random-tree-fp32", 1, 4, 4, 64, 32, 128, torch.float32, 64, 64, "random",
                 description="CPU-runnable case: random parents, fp32"),
        Workload("llama3-8b-eagle64-p4096", 1, 32, 8, 128, 4096, 64, torch.bfloat16, 16, 64, "eagle",
                 {"depth": 6, "topk": 8},
                 description="Llama-3-8B attention shape, 4k prefix, 64-node EAGLE tree"),
        Workload("batched-decode-b16-p2048", 16, 32, 8, 128, 2048, 64, torch.bfloat16, 16, 64, "eagle",
                 {"depth": 5, "topk": 6}, per_sequence=True,
                 description="16 sequences, shared 2k prefix length, own 64-node EAGLE tree each"),
        Workload("wide-tree-1024-p16384", 1, 32, 8, 128, 16384, 1024, torch.bfloat16, 64, 64, "kary",
                 {"arity": 4},
                 description="4-ary BFS tree of 1024 nodes behind a 16k prefix"),
        Workload("llama3-70b-b4-p32768", 4, 64, 8, 128, 32768, 256, torch.float16, 64, 64, "depth_limited",
                 {"max_depth": 10}, per_sequence=True,
                 description="Llama-3-70B head layout, 32k prefix, 256-node random trees of depth <= 10"),
    ]
}

HEADLINE = "llama3-8b-eagle64-p4096"


def make_parents(w: Workload, seq: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng([seed, seq])
    if w.tree_kind == "random":
        return trees.random_parents(w.tree_len, rng)
    if w.tree_kind == "eagle":
        return trees.eagle_parents(w.tree_len, w.tree_args["depth"], w.tree_args["topk"], rng)
    if w.tree_kind == "kary":
        return trees.kary_bfs_parents(w.tree_len, w.tree_args["arity"])
    if w.tree_kind == "depth_limited":
        return trees.depth_limited_parents(w.tree_len, w.tree_args["max_depth"], rng)
    raise ValueError(f"unknown tree kind {w.tree_kind}")


def make_tree_mask(w: Workload, seed: int = 42) -> torch.Tensor:
    """[T, T] bool (shared tree) or [B, T, T] bool (per-sequence trees), on the CPU."""
    if not w.per_sequence:
        return torch.from_numpy(trees.ancestor_mask(make_parents(w, 0, seed)))
    return torch.from_numpy(np.stack([trees.ancestor_mask(make_parents(w, b, seed)) for b in range(w.batch)]))


def make_qkv(w: Workload, seed: int = 42, device="cpu"):
    """Q [B,Hq,T,D], K/V [B,Hkv,P+T,D] in the workload dtype on ``device``."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((w.batch, w.q_heads, w.tree_len, w.head_dim), generator=g, dtype=torch.float32)
    k = torch.randn((w.batch, w.kv_heads, w.kv_len, w.head_dim), generator=g, dtype=torch.float32)
    v = torch.randn((w.batch, w.kv_heads, w.kv_len, w.head_dim), generator=g, dtype=torch.float32)
    return tuple(x.to(w.dtype).to(device) for x in (q, k, v))


def make_paged_kv(k: torch.Tensor, v: torch.Tensor, page_size: int, *, layout: str = "NHD", seed=None,
                  spare_pages: int = 0, dense_table: bool = False):
    """K/V [B,Hkv,L,D] laid into FlashInfer's paged cache, as benchmark.py:67-91 builds it.

    Returns (cache, kv_indptr, kv_indices): cache [pages, 2, page_size, Hkv, D]
    ("NHD") or [pages, 2, Hkv, page_size, D] ("HND"), K in slot 0 and V in
    slot 1, rows past L in a sequence's last page zero.  Sequence b owns
    ceil(L / page_size) pages; with ``seed`` the pages are scattered over the
    pool in a seeded random order (plus ``spare_pages`` never referenced),
    otherwise sequence b holds pages b*n .. b*n + n - 1 as in the reference.
    kv_indptr is None and kv_indices a [B, n] table with ``dense_table``.
    """
    bsz, hkv, kv_len, d = k.shape
    n = -(-kv_len // page_size)
    total = bsz * n + spare_pages
    if seed is None:
        order = torch.arange(total, dtype=torch.int64)
    else:
        order = torch.randperm(total, generator=torch.Generator().manual_seed(seed))
    ids = order[: bsz * n].view(bsz, n)
    shape = (total, 2, page_size, hkv, d) if layout == "NHD" else (total, 2, hkv, page_size, d)
    cache = torch.zeros(shape, dtype=k.dtype, device=k.device)
    pad = n * page_size - kv_len
    for slot, x in ((0, k), (1, v)):
        xs = torch.nn.functional.pad(x, (0, 0, 0, pad))  # [B, Hkv, n*ps, D]
        xs = xs.view(bsz, hkv, n, page_size, d)
        xs = xs.permute(0, 2, 3, 1, 4) if layout == "NHD" else xs.permute(0, 2, 1, 3, 4)
        cache[ids.reshape(-1).to(k.device), slot] = xs.reshape(bsz * n, *shape[2:])
    kv_indices = ids.to(torch.int32).to(k.device)
    if dense_table:
        return cache, None, kv_indices
    kv_indptr = (torch.arange(bsz + 1, dtype=torch.int32) * n).to(k.device)
    return cache, kv_indptr, kv_indices.reshape(-1).contiguous()
