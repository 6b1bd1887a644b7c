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
    assert L.mg_version() == 206  # 0.2.6: the ABI of include/mingru_hip.h
    # a 256-byte header, ticket counters per chain and direction (rounded to
    # 256 B) + one 8-byte look-back word per (tile, channel) for the forward
    # (128-step tiles) and the backward (64-step tiles)
    assert L.mg_scan_workspace_bytes(2, 300, 64) == 256 + 256 + (3 + 5) * 2 * 64 * 8
    assert L.mg_scan_workspace_bytes(16, 8192, 2048) == 256 + 4096 + (64 + 128) * 16 * 2048 * 8


def _fwd(L, **kw):
    args = dict(in_dtype=1, hidden=16, gate=16, in_sb=1024, in_ld=64, h0=None, out_dtype=1, h=16, out_sb=512,
                out_ld=64, h_last=None, ckpt=None, B=2, T=8, Di=64, ws=16, wsb=1 << 20, stream=None)
    args.update(kw)
    return L.mg_scan_fwd(*args.values())


def test_poll_and_noalloc_check_argument_errors(L):
    # rejected before any HIP call (no GPU needed)
    assert L.mg_scan_workspace_poll(None, None, None) == 1
    assert "bad workspace" in L.mg_last_error().decode()
    assert L.mg_scan_workspace_poll(16, None, None) == 1
    assert "host word" in L.mg_last_error().decode()


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
    # (a workspace that was never initialised is refused by the kernel itself, on the
    # device: tests/test_scan_gpu.py::test_workspace_errors_end_the_kernel)
    assert L.mg_scan_workspace_init(None, 1 << 20, 2, 8, 64, None) == 3
    assert L.mg_scan_workspace_init(16, 8, 2, 8, 64, None) == 3
    assert L.mg_scan_workspace_init(16, 1 << 20, 2, 8, 62, None) == 1
    assert L.mg_scan_workspace_check(None, None) == 1
    assert L.mg_scan_workspace_set_max_polls(None, 5, None) == 1
    assert L.mg_scan_workspace_set_max_polls(16, 0, None) == 1
    # backward output strides are checked like the inputs'
    bwd = dict(in_dtype=1, hidden=16, gate=16, in_sb=1024, in_ld=64, h0=None, out_dtype=1, h=16, out_sb=512,
               out_ld=64, ckpt=None, dh=16, g_sb=512, g_ld=64, dh_last=None, dhid=16, dgat=16, d_sb=512, d_ld=66,
               dh0=None, B=2, T=8, Di=64, ws=16, wsb=1 << 20, stream=None)
    assert L.mg_scan_bwd(*bwd.values()) == 1 and b"dhidden" in L.mg_last_error()


def test_embedding_bwd_argument_errors(L):
    e = dict(ids=16, dx=16, ldx=64, N=100, D=64, V=256, dw=16, ldw=64, ws=16, wsb=1 << 24, stream=None)
    # (every call below fails its checks before any launch)
    for bad in ({"V": 0}, {"V": 513}, {"D": 62}, {"ldx": 62}, {"ldw": 32}, {"N": 0}, {"ids": None}, {"dx": 8},
                {"ws": None}):
        args = {**e, **bad}
        rc = L.mg_embedding_bwd(*args.values())
        assert rc in (1, 3), (bad, rc)
    assert L.mg_embedding_bwd(*{**e, "wsb": 64}.values()) == 3 and b"workspace" in L.mg_last_error()
    assert L.mg_embedding_bwd(*{**e, "V": 513}.values()) == 1 and b"V=513" in L.mg_last_error()
    assert L.mg_embedding_bwd_workspace_bytes(16384, 1024, 256) >= (256 + 256) * 1024 * 4 + 16384 * 4


def test_wgrad_pair_argument_errors(L):
    """Every call here fails validation before any launch (fake, aligned pointers)."""
    fake = ctypes.c_void_p(1 << 20)
    ws = 1 << 30
    ok = dict(dy0=fake, ld_dy0=1024, x0=fake, ld_x0=4096, M0=1024, N0=4096, dw0=fake, ldc0=4096,
              dy1=fake, ld_dy1=4096, x1=fake, ld_x1=1024, M1=4096, N1=1024, dw1=fake, ldc1=1024, K=16376, flags=0,
              ws=fake, wsb=ws, stream=None)

    def call(**kw):
        a = dict(ok, **kw)
        return L.mg_gemm_wgrad_pair(*a.values())

    assert L.mg_gemm_wgrad_pair_workspace_bytes(1024, 4096, 4096, 1024, 16376, 0) == 2 * 2 * 1024 * 4096 * 4
    assert call(flags=4) == 1                      # hi/lo is not a weight-gradient flag
    assert call(dy1=None) == 1
    assert call(M0=-256) == 1
    assert call(ld_dy0=1000) == 1                  # below M0
    assert call(ldc1=1020) == 1                    # below N1
    assert call(ld_x0=4100) == 1                   # not a multiple of 8
    assert call(x1=ctypes.c_void_p((1 << 20) + 8)) == 1   # misaligned
    assert call(wsb=1024) == 3                     # workspace too small
    assert call(K=1 << 20) == 1                    # operands over 2 GiB
    assert b"mg_gemm_wgrad_pair" in L.mg_last_error()


def test_hilo_and_norm_argument_errors(L):
    # hi/lo products need K-contiguous operands and K >= 1; rows must hold 2K values
    g = dict(al=0, A=16, lda=128, bl=0, B=16, ldb=128, M=64, N=64, K=64, epi=0, bias=None, aux=None, ldaux=0,
             cd=0, C=16, ldc=64, flags=4, ws=None, wsb=0, stream=None)
    assert L.mg_gemm(*{**g, "al": 1}.values()) == 1 and b"K-contiguous" in L.mg_last_error()
    assert L.mg_gemm(*{**g, "K": 0}.values()) == 1
    assert L.mg_gemm(*{**g, "lda": 64}.values()) == 1 and b"leading dimension" in L.mg_last_error()
    assert L.mg_gemm(*{**g, "flags": 64}.values()) == 1
    assert L.mg_split_hilo(16, 8, 4, 6, 16, 16, None) == 1  # cols % 4
    assert L.mg_split_hilo(16, 8, 4, 8, 16, 8, None) == 1   # ldo < 2 cols
    assert L.mg_split_hilo(20, 8, 4, 8, 16, 16, None) == 1  # x misaligned
    eps = ctypes.c_float(1e-7)
    n = dict(x=16, ddt=0, delta=None, w=16, x_out=None, ydt=1, y=16, y_lo=None, ldy=60, rstd=None, N=4, D=64, eps=eps,
             stream=None)
    assert L.mg_add_rmsnorm_fwd(*n.values()) == 1 and b"ldy" in L.mg_last_error()
    assert L.mg_add_rmsnorm_fwd(*{**n, "ldy": 128, "ydt": 0, "y_lo": 16}.values()) == 2  # lo needs a bf16 y


def test_decode_argument_errors(L):
    import ctypes

    eps = ctypes.c_float(1e-7)
    # batch above 8, a dimension that is not a multiple of 8, a width over the LDS staging
    assert L.mg_decode_mingru(9, 64, None, None, 0, 16, None, 16, 16, 16, 16, eps, None) == 1
    assert L.mg_decode_mingru(1, 60, None, None, 0, 16, None, 16, 16, 16, 16, eps, None) == 1
    assert L.mg_decode_ff(8, 64, 8200, 16, 16, 16, 16, 16, 16, 16, 16, eps, None) == 1
    assert L.mg_decode_mingru_expanded(1, 64, 8200, None, None, 0, 16, None, 16, 16, 16, 16, eps, None) == 1
    assert L.mg_decode_mingru_expanded(1, 64, 100, None, None, 0, 16, None, 16, 16, 16, 16, eps, None) == 1
    assert L.mg_decode_mingru_expanded(1, 64, 96, None, None, 0, 16, None, None, 16, 16, 16, eps, None) == 1  # h_out
    assert L.mg_decode_to_out(1, 64, 8200, None, None, 0, 16, None, 16, 16, 16, None) == 1
    assert L.mg_decode_to_out(1, 64, 96, None, None, 0, 16, None, 24, 16, 16, None) == 1  # h misaligned
    assert L.mg_decode_to_out(1, 64, 96, None, None, 0, 16, None, 16, 16, None, None) == 1  # x_out
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
    # the fp32 and float16 steps: exactly one of x_out / h_out, Di == D without h_out, the fp32
    # staged-row limit at batch 5-8 (4096), 16-byte fp32 pending
    assert L.mg_decode_mingru_f32(1, 64, 64, None, None, 0, 16, None, 16, 16, 16, 16, 16, eps, None) == 1
    assert L.mg_decode_mingru_f32(1, 64, 64, None, None, 0, 16, None, None, None, 16, 16, 16, eps, None) == 1
    assert L.mg_decode_mingru_f32(1, 64, 96, None, None, 0, 16, None, 16, None, 16, 16, 16, eps, None) == 1
    assert b"h_out" in L.mg_last_error()
    assert L.mg_decode_ff_f32(5, 64, 4104, 16, 16, 16, 16, 16, 16, 16, 16, eps, None) == 1
    assert L.mg_decode_to_out_f32(8, 64, 8192, None, None, 0, 16, None, 16, 16, 16, None) == 1
    assert L.mg_decode_mingru_f32(1, 64, 64, None, None, 0, 16, 24, 16, None, 16, 16, 16, eps, None) == 1  # pending
    assert L.mg_decode_mingru_f16(1, 64, 64, None, None, 0, 16, None, 16, 16, 16, 16, 16, eps, None) == 1
    assert L.mg_decode_ff_f16(9, 64, 256, 16, 16, 16, 16, 16, 16, 16, 16, eps, None) == 1
    assert L.mg_decode_head_f16(1, 64, 0, 16, None, 16, 16, 16, eps, None) == 1


def test_scaled_norm_bwd_argument_errors(L):
    # mg_add_rmsnorm_bwd_scaled: the scale is a 4-byte-aligned device float (NULL: 1); the
    # other checks are mg_add_rmsnorm_bwd's, which forwards to it
    args = dict(xn=16, w=16, rstd=16, dydt=1, dy=16, scale=None, dres=None, dx=16, dddt=0, dd=None, dw=16, N=4, D=64,
                ws=None, wsb=0, stream=None)
    assert L.mg_add_rmsnorm_bwd_scaled(*{**args, "scale": 18}.values()) == 1
    assert b"dy_scale" in L.mg_last_error()
    assert L.mg_add_rmsnorm_bwd_scaled(*args.values()) == 3  # no workspace
    assert L.mg_add_rmsnorm_bwd(16, 16, 16, 1, 16, None, 16, 0, None, 16, 4, 62, None, 0, None) == 1  # D % 4


def test_product_refuses_cpu_tensors():
    import torch
    from gruboros_amd.scan import gate_scan

    x = torch.zeros(1, 4, 8)
    with pytest.raises(RuntimeError, match="GPU only"):
        gate_scan(x, x)
