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


# The library reads its TSFA_* environment switches once; tests that switch
# them through monkeypatch (setenv, delenv, and the restore at teardown) make
# it read them again.
import pytest  # noqa: E402

_mp_setenv, _mp_delenv, _mp_undo = pytest.MonkeyPatch.setenv, pytest.MonkeyPatch.delenv, pytest.MonkeyPatch.undo


def _reload_config():
    try:
        import tree_sparse_flashattn as tsf
        tsf.reload_config()
    except Exception:  # library not built (or host-only): nothing to reload
        pass


def _setenv(self, name, value, prepend=None):
    _mp_setenv(self, name, value, prepend)
    if str(name).startswith("TSFA_"):
        _reload_config()


def _delenv(self, name, raising=True):
    _mp_delenv(self, name, raising)
    if str(name).startswith("TSFA_"):
        _reload_config()


def _undo(self):
    touched = any(str(getattr(entry, "name", entry[1] if isinstance(entry, tuple) else "")).startswith("TSFA_")
                  for entry in getattr(self, "_setitem", []))
    _mp_undo(self)
    if touched:
        _reload_config()


pytest.MonkeyPatch.setenv = _setenv
pytest.MonkeyPatch.delenv = _delenv
pytest.MonkeyPatch.undo = _undo
