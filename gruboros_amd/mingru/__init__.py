"""Drop-in for the reference package `mingru` (mingru/__init__.py:1-2).

Put this directory's parent (gruboros_amd/) on sys.path, or alias it, so
that `from mingru.minLM import minLM` resolves here; see
gruboros_amd.mingru.install_alias().
"""
from .minGRU import MinGRU, minGRU  # noqa: F401


def install_alias():
    """Make `import mingru`, `mingru.minGRU` and `mingru.minLM` resolve to this package."""
    import importlib
    import sys

    _g = importlib.import_module(__name__ + ".minGRU")
    _l = importlib.import_module(__name__ + ".minLM")

    pkg = sys.modules[__name__]
    sys.modules.setdefault("mingru", pkg)
    sys.modules.setdefault("mingru.minGRU", _g)
    sys.modules.setdefault("mingru.minLM", _l)
    return pkg
