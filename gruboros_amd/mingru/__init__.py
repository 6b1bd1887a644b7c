"""Drop-in for the reference package `mingru` (mingru/__init__.py:1-2).

Put this directory's parent (gruboros_amd/) on sys.path, or alias it, so
that `from mingru.minLM import minLM` resolves here; see
gruboros_amd.mingru.install_alias().
"""
from . import _defaults
from .minGRU import MinGRU, minGRU  # noqa: F401


def set_default_compute_dtype(dtype):
    """Activation dtype of every minLM built without compute_dtype (None: the
    parameters' dtype, as in the reference). torch.bfloat16 is the MI355X
    training configuration; this lets an unchanged caller (reference
    train.py) train in it."""
    _defaults.COMPUTE_DTYPE = dtype


def install_alias(compute_dtype=None):
    """Make `import mingru`, `mingru.minGRU` and `mingru.minLM` resolve to this
    package; compute_dtype (e.g. torch.bfloat16) sets the default activation
    dtype of minLM (set_default_compute_dtype)."""
    import importlib
    import sys

    if compute_dtype is not None:
        set_default_compute_dtype(compute_dtype)
    _g = importlib.import_module(__name__ + ".minGRU")
    _l = importlib.import_module(__name__ + ".minLM")

    pkg = sys.modules[__name__]
    sys.modules.setdefault("mingru", pkg)
    sys.modules.setdefault("mingru.minGRU", _g)
    sys.modules.setdefault("mingru.minLM", _l)
    return pkg
