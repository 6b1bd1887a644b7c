"""The C-ABI library loads, exports every symbol include/*.h declares, and
rejects bad arguments with an error code and message (no GPU work needed:
argument checks run before anything is enqueued)."""
import ctypes
import glob
import os
import re

import pytest

from gruboros_amd import _lib
from gruboros_amd.build import LIB_PATH

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names.update(re.findall(r"\b(mg_\w+)\s*\(", text))
    return sorted(names)


@pytest.fixture(scope="module")
def L():
    if not os.path.exists(LIB_PATH):
        pytest.fail(f"{LIB_PATH} not built (run __graft_entry__.build())")
    return _lib.lib()


def test_every_declared_symbol_is_exported(L):
    names = declared_symbols()
    assert "mg_scan_fwd" in names and "mg_version" in names
    for n in names:
        assert hasattr(L, n), f"{n} declared in include/ but not exported"
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature in gruboros_amd/_lib.py"


def test_version_and_queries(L):
    assert L.mg_version() >= 100
    # ticket counters per chain and direction (rounded to 256 B) + one 8-byte
    # look-back word per (tile, channel) for the forward (128-step tiles) and
    # the backward (64-step tiles)
    assert L.mg_scan_workspace_bytes(2, 300, 64) == 256 + (3 + 5) * 2 * 64 * 8
    assert L.mg_scan_workspace_bytes(16, 8192, 2048) == 4096 + (64 + 128) * 16 * 2048 * 8


def _fwd(L, **kw):
    args = dict(in_dtype=1, hidden=16, gate=16, in_sb=1024, in_ld=64, h0=None, out_dtype=1, h=16, out_sb=512,
                out_ld=64, h_last=None, ckpt=None, B=2, T=8, Di=64, ws=16, wsb=1 << 20, stream=None)
    args.update(kw)
    return L.mg_scan_fwd(*args.values())


def test_argument_errors(L):
    assert _fwd(L, Di=62) == 1
    assert "multiple of 4" in L.mg_last_error().decode()
    assert _fwd(L, T=0) == 1
    assert _fwd(L, wsb=8) == 3
    assert "workspace" in L.mg_last_error().decode()
    assert _fwd(L, in_dtype=7) == 2
    assert _fwd(L, hidden=None) == 1
    assert _fwd(L, in_ld=66) == 1
    assert _fwd(L, hidden=18) == 1  # misaligned
    assert _fwd(L, out_dtype=1, in_dtype=0) == 2  # f32 -> bf16 not offered
    # every argument valid, but the workspace was never initialised
    assert _fwd(L) == 3
    assert "not initialised" in L.mg_last_error().decode()
    assert L.mg_scan_workspace_init(None, 1 << 20, 2, 8, 64, None) == 3
    assert L.mg_scan_workspace_init(16, 8, 2, 8, 64, None) == 3
    assert L.mg_scan_workspace_init(16, 1 << 20, 2, 8, 62, None) == 1


def test_decode_argument_errors(L):
    import ctypes

    eps = ctypes.c_float(1e-7)
    # batch above 8, a dimension that is not a multiple of 8, a width over the LDS staging
    assert L.mg_decode_mingru(9, 64, None, None, 0, 16, None, 16, 16, 16, 16, eps, None) == 1
    assert L.mg_decode_mingru(1, 60, None, None, 0, 16, None, 16, 16, 16, 16, eps, None) == 1
    assert L.mg_decode_ff(8, 64, 8192, 16, 16, 16, 16, 16, 16, 16, 16, eps, None) == 1
    assert L.mg_decode_mingru(1, 64, 16, None, 256, None, None, 16, 16, 16, 16, eps, None) == 1  # no embedding
    assert L.mg_decode_head(1, 64, 0, 16, None, 16, 16, 16, eps, None) == 1
    # the norm prologue reads 16-byte groups of x / emb / norm weight and 8 bytes of pending:
    # misaligned pointers are refused before any launch
    assert L.mg_decode_mingru(1, 64, None, None, 0, 20, None, 16, 16, 16, 16, eps, None) == 1  # x_in
    assert L.mg_decode_mingru(1, 64, None, None, 0, 16, 20, 16, 16, 16, 16, eps, None) == 1  # pending
    assert L.mg_decode_mingru(1, 64, 16, 24, 256, None, None, 16, 16, 16, 16, eps, None) == 1  # emb
    assert L.mg_decode_ff(1, 64, 256, 24, 16, 16, 16, 16, 16, 16, 16, eps, None) == 1  # x
    assert L.mg_decode_head(1, 64, 256, 16, None, 24, 16, 16, eps, None) == 1  # norm weight
    assert b"aligned" in L.mg_last_error()


def test_product_refuses_cpu_tensors():
    import torch
    from gruboros_amd.scan import gate_scan

    x = torch.zeros(1, 4, 8)
    with pytest.raises(RuntimeError, match="GPU only"):
        gate_scan(x, x)
