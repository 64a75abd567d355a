"""Host-side support package of the MI355X tree-sparse attention build.

  _lib     ctypes binding of libtsfa.so (C ABI: include/tsfa.h)
  build    hipcc recipe that produces libtsfa.so in-tree
  trees    seeded draft-tree generators and ancestor masks
  configs  named verification workloads and their synthetic inputs
"""
