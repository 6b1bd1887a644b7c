"""gruboros_amd — MI355X-native minGRU / minLM training hot path.

Modules:
  _lib     ctypes binding of libmingru_hip.so (C ABI in include/mingru_hip.h)
  scan     autograd Functions: fused gate math + associative scan
  mingru   drop-in mirror of the reference package (minGRU, minLM)
"""
from .build import LIB_PATH  # noqa: F401

__version__ = "0.1.0"
