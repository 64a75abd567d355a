"""CPU oracle for the tree-sparse attention path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, and only as the
checker (or as the timed CPU baseline).  The product path in
``eagle3-tree-sparse-flashattn_amd/`` never imports it and has no CPU fallback.

Modules:
  meta_oracle  numpy restatement of the metadata protocol
               (tree_sparse_flashattn.py:11-160).
  attn_oracle  fp32 torch restatement of the dense+mask attention
               (benchmark.py:8-35) plus an fp64 brute-force loop for tiny
               shapes.
"""
