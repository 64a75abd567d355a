"""Seeded draft-tree generators and ancestor masks.

A draft tree is a parent array in topological order (``parents[0] == -1`` is
the root, ``parents[i] < i``).  Its verification mask is
``mask[i, j] = 1`` iff ``j == i`` or ``j`` is an ancestor of ``i`` -- the
"ancestor-visible, cross-branch-invisible" tree mask the reference's README
describes (README.md:150-151) and that EAGLE verification feeds to
``prepare_tree_sparse_metadata``.
"""

from __future__ import annotations

import numpy as np


def ancestor_mask(parents) -> np.ndarray:
    """[n, n] bool: row i has i and every ancestor of i set."""
    parents = np.asarray(parents, dtype=np.int64)
    n = parents.size
    mask = np.zeros((n, n), dtype=bool)
    for i in range(n):
        p = int(parents[i])
        if p >= 0:
            if p >= i:
                raise ValueError("parents must be in topological order (parent < child)")
            mask[i] = mask[p]
        mask[i, i] = True
    return mask


def depths(parents) -> np.ndarray:
    parents = np.asarray(parents, dtype=np.int64)
    d = np.zeros(parents.size, dtype=np.int64)
    for i in range(1, parents.size):
        d[i] = d[parents[i]] + 1
    return d


def random_parents(n: int, rng: np.random.Generator) -> np.ndarray:
    """parent[i] uniform over the earlier nodes; node 0 is the root."""
    parents = np.full(n, -1, dtype=np.int64)
    for i in range(1, n):
        parents[i] = rng.integers(0, i)
    return parents


def depth_limited_parents(n: int, max_depth: int, rng: np.random.Generator) -> np.ndarray:
    """Random parents among earlier nodes whose depth is below ``max_depth``."""
    parents = np.full(n, -1, dtype=np.int64)
    d = np.zeros(n, dtype=np.int64)
    eligible = [0]
    for i in range(1, n):
        p = eligible[int(rng.integers(0, len(eligible)))]
        parents[i] = p
        d[i] = d[p] + 1
        if d[i] < max_depth:
            eligible.append(i)
    return parents


def kary_bfs_parents(n: int, arity: int) -> np.ndarray:
    """Complete ``arity``-ary tree in breadth-first order, truncated to n nodes."""
    parents = np.full(n, -1, dtype=np.int64)
    parents[1:] = (np.arange(1, n) - 1) // arity
    return parents


def eagle_parents(n_keep: int, depth: int, topk: int, rng: np.random.Generator,
                  score_floor: float = 1e-3) -> np.ndarray:
    """EAGLE-style dynamic draft tree.

    Level by level (``depth`` levels below the root), the ``topk`` best nodes
    of the previous level are each expanded into ``topk`` children whose edge
    scores are log-uniform on [score_floor, 1).  A node's score is the
    cumulative log-score of its path, so it is strictly below its parent's and
    keeping the ``n_keep`` best nodes overall yields an ancestor-closed tree.
    The kept nodes are ordered by (depth, score descending), which is
    topological.
    """
    lo = np.log(score_floor)
    par = [-1]
    lvl = [0]
    cum = [0.0]
    frontier = [0]
    for level in range(1, depth + 1):
        cand = []
        for p in frontier:
            edge = rng.uniform(lo, 0.0, size=topk)
            for e in edge:
                par.append(p)
                lvl.append(level)
                cum.append(cum[p] + float(e))
                cand.append(len(par) - 1)
        cand.sort(key=lambda i: -cum[i])
        frontier = cand[:topk]
    order = sorted(range(len(par)), key=lambda i: (-cum[i], lvl[i], i))[:n_keep]
    order.sort(key=lambda i: (lvl[i], -cum[i], i))
    remap = {old: new for new, old in enumerate(order)}
    parents = np.full(len(order), -1, dtype=np.int64)
    for new, old in enumerate(order):
        parents[new] = -1 if par[old] < 0 else remap[par[old]]
    return parents
