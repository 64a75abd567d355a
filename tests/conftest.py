"""pytest configuration: the `gpu` marker and import paths.

The package directory (eagle3-tree-sparse-flashattn_amd/) is put on sys.path
the way a user of the reference puts the reference checkout on it, so the
drop-in modules import under the reference's names.
"""

import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "eagle3-tree-sparse-flashattn_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X) and the built libtsfa.so")
