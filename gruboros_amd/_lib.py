"""ctypes binding of libmingru_hip.so (declarations: include/mingru_hip.h).

The library is required: there is no fallback path. Loading it after
``import torch`` makes it share torch's HIP runtime, so torch streams and
device pointers can be passed straight through.
"""
import ctypes
import os

import torch  # noqa: F401  (loads the HIP runtime the library binds to)

from .build import LIB_PATH

MG_F32 = 0
MG_BF16 = 1
MG_ERR_STALL = 5

_c_int, _c_i64, _c_size, _vp, _fp = (ctypes.c_int, ctypes.c_int64, ctypes.c_size_t, ctypes.c_void_p,
                                     ctypes.c_void_p)

# name -> (restype, argtypes); mirrors include/mingru_hip.h
SIGNATURES = {
    "mg_version": (_c_int, []),
    "mg_last_error": (ctypes.c_char_p, []),
    "mg_scan_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int]),
    "mg_scan_workspace_init": (_c_int, [_vp, _c_size, _c_int, _c_int, _c_int, _vp]),
    "mg_scan_workspace_set_max_polls": (_c_int, [_vp, ctypes.c_uint32, _vp]),
    "mg_scan_workspace_check": (_c_int, [_vp, _vp]),
    "mg_scan_workspace_poll": (_c_int, [_vp, _vp, _vp]),
    "mg_scan_fwd_noalloc_check": (_c_int, [_vp]),
    "mg_decode_mingru": (_c_int, [_c_int, _c_int, _vp, _vp, _c_int, _vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_float,
                                  _vp]),
    "mg_decode_mingru_expanded": (_c_int, [_c_int, _c_int, _c_int, _vp, _vp, _c_int, _vp, _vp, _vp, _vp, _vp, _vp,
                                           ctypes.c_float, _vp]),
    "mg_decode_to_out": (_c_int, [_c_int, _c_int, _c_int, _vp, _vp, _c_int, _vp, _vp, _vp, _vp, _vp, _vp]),
    "mg_decode_ff": (_c_int, [_c_int, _c_int, _c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_float, _vp]),
    "mg_decode_head": (_c_int, [_c_int, _c_int, _c_int, _vp, _vp, _vp, _vp, _vp, ctypes.c_float, _vp]),
    "mg_decode_mingru_f32": (_c_int, [_c_int, _c_int, _c_int, _vp, _vp, _c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                      ctypes.c_float, _vp]),
    "mg_decode_to_out_f32": (_c_int, [_c_int, _c_int, _c_int, _vp, _vp, _c_int, _vp, _vp, _vp, _vp, _vp, _vp]),
    "mg_decode_ff_f32": (_c_int, [_c_int, _c_int, _c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_float,
                                  _vp]),
    "mg_decode_head_f32": (_c_int, [_c_int, _c_int, _c_int, _vp, _vp, _vp, _vp, _vp, ctypes.c_float, _vp]),
    "mg_decode_mingru_f16": (_c_int, [_c_int, _c_int, _c_int, _vp, _vp, _c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                      ctypes.c_float, _vp]),
    "mg_decode_to_out_f16": (_c_int, [_c_int, _c_int, _c_int, _vp, _vp, _c_int, _vp, _vp, _vp, _vp, _vp, _vp]),
    "mg_decode_ff_f16": (_c_int, [_c_int, _c_int, _c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_float,
                                  _vp]),
    "mg_decode_head_f16": (_c_int, [_c_int, _c_int, _c_int, _vp, _vp, _vp, _vp, _vp, ctypes.c_float, _vp]),
    "mg_scan_ckpt_elems": (_c_size, [_c_int, _c_int, _c_int]),
    "mg_scan_fwd_noalloc_max_bytes": (_c_size, []),
    "mg_scan_fwd_noalloc": (_c_int, [_c_int, _vp, _vp, _c_i64, _c_i64, _fp, _c_int, _vp, _c_i64, _c_i64, _fp, _fp,
                                     _c_int, _c_int, _c_int, _vp]),
    "mg_scan_fwd_residual": (_c_int, [_c_int, _vp, _vp, _c_i64, _c_i64, _fp, _fp, _fp, _c_i64, _c_i64, _fp, _fp,
                                      _c_int, _c_int, _c_int, _vp, _c_size, _vp]),
    "mg_scan_fwd": (_c_int, [_c_int, _vp, _vp, _c_i64, _c_i64, _fp, _c_int, _vp, _c_i64, _c_i64, _fp, _fp,
                             _c_int, _c_int, _c_int, _vp, _c_size, _vp]),
    "mg_scan_bwd": (_c_int, [_c_int, _vp, _vp, _c_i64, _c_i64, _fp, _c_int, _vp, _c_i64, _c_i64, _fp,
                             _vp, _c_i64, _c_i64, _fp, _vp, _vp, _c_i64, _c_i64, _fp, _c_int, _c_int, _c_int, _vp,
                             _c_size, _vp]),
    "mg_add_rmsnorm_fwd": (_c_int, [_fp, _c_int, _vp, _fp, _fp, _c_int, _vp, _vp, _c_i64, _fp, _c_i64, _c_int,
                                    ctypes.c_float, _vp]),
    "mg_split_hilo": (_c_int, [_fp, _c_i64, _c_i64, _c_int, _vp, _c_i64, _vp]),
    "mg_split_limbs": (_c_int, [_fp, _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_int, _vp, _c_i64, _vp]),
    "mg_round_bf16_sr": (_c_int, [_fp, _c_i64, _vp, ctypes.c_uint32, _vp]),
    "mg_add_rmsnorm_bwd_workspace_bytes": (_c_size, [_c_i64, _c_int]),
    "mg_add_rmsnorm_bwd": (_c_int, [_fp, _fp, _fp, _c_int, _vp, _fp, _fp, _c_int, _vp, _fp, _c_i64, _c_int, _vp,
                                    _c_size, _vp]),
    "mg_add_rmsnorm_bwd_scaled": (_c_int, [_fp, _fp, _fp, _c_int, _vp, _vp, _fp, _fp, _c_int, _vp, _fp, _c_i64, _c_int,
                                          _vp, _c_size, _vp]),
    "mg_cross_entropy_partials": (_c_int, [_c_i64]),
    "mg_cross_entropy_fwd_bwd": (_c_int, [_c_int, _vp, _vp, _c_int, _vp, _fp, _vp, _c_i64, _c_int, ctypes.c_float,
                                          _vp]),
    "mg_sf_adamw_chunk_elems": (_c_i64, []),
    "mg_sf_adamw_step": (_c_int, [_vp, _c_int, _c_i64] + [ctypes.c_float] * 8 + [_vp]),
    "mg_logits_cross_entropy_partials": (_c_int, [_c_i64]),
    "mg_logits_cross_entropy": (_c_int, [_vp, _c_i64, _vp, _c_i64, _vp, _vp, _c_i64, _fp, _vp, _c_int, _c_int, _c_int,
                                         ctypes.c_float, _vp]),
    "mg_column_sum_workspace_bytes": (_c_size, [_c_i64, _c_int]),
    "mg_column_sum": (_c_int, [_c_int, _vp, _c_i64, _c_i64, _c_int, _fp, _vp, _c_size, _vp]),
    "mg_ff_bias_bwd_workspace_bytes": (_c_size, [_c_i64, _c_int, _c_int]),
    "mg_ff_bias_bwd": (_c_int, [_c_int, _vp, _c_i64, _vp, _c_i64, _vp, _c_i64, _fp, _c_i64, _c_int, _vp, _c_i64, _fp,
                                _c_int, _vp, _c_size, _vp]),
    "mg_gelu_bwd": (_c_int, [_c_int, _vp, _c_i64, _vp, _c_i64, _vp, _c_i64, _fp, _c_i64, _c_int, _vp, _c_size, _vp]),
    "mg_embedding_bwd_workspace_bytes": (_c_size, [_c_i64, _c_int, _c_int]),
    "mg_embedding_bwd": (_c_int, [_vp, _fp, _c_i64, _c_i64, _c_int, _c_int, _fp, _c_i64, _vp, _c_size, _vp]),
    "mg_gemm": (_c_int, [_c_int, _vp, _c_i64, _c_int, _vp, _c_i64, _c_int, _c_int, _c_int, _c_int, _fp, _vp, _c_i64,
                         _c_int, _vp, _c_i64, _c_int, _vp, _c_size, _vp]),
    "mg_gemm_hilo_prefix": (_c_int, [_vp, _c_i64, _vp, _c_i64, _c_int, _c_int, _c_int, _c_int, _vp, _c_i64, _vp]),
    "mg_gemm_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int]),
    "mg_gemm_wgrad_pair": (_c_int, [_vp, _c_i64, _vp, _c_i64, _c_int, _c_int, _fp, _c_i64,
                                    _vp, _c_i64, _vp, _c_i64, _c_int, _c_int, _fp, _c_i64, _c_int, _c_int,
                                    _vp, _c_size, _vp]),
    "mg_gemm_wgrad_pair_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int]),
}

_LIB = None


class MingruHipError(RuntimeError):
    pass


def lib():
    """The loaded library; raises if it has not been built."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise MingruHipError(
                f"{LIB_PATH} is missing: build it with `python -m gruboros_amd.build` "
                "(or __graft_entry__.build()). There is no non-HIP fallback.")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def check(rc: int, what: str = "") -> None:
    if rc != 0:
        msg = lib().mg_last_error().decode(errors="replace")
        raise MingruHipError(f"{what or 'libmingru_hip'} failed (code {rc}): {msg}")


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return MG_F32
    if dt == torch.bfloat16:
        return MG_BF16
    raise MingruHipError(f"unsupported dtype {dt}: the MI355X kernels take float32 and bfloat16 "
                         "(cast a float16 model with .to(torch.bfloat16) instead)")


# Pointer and stream arguments go to the library as plain integers (every one is
# declared c_void_p, which takes an int; None is NULL): the per-call cost of
# building ctypes objects and torch.cuda.Stream wrappers is measurable at the
# ~20 k library calls of a [1, 2048]-chunk optimizer step of a 79-layer model.
_raw_stream = torch._C._cuda_getCurrentRawStream


def ptr(t):
    return None if t is None else t.data_ptr()


def raw_stream(device: torch.device) -> int:
    """Handle of the current HIP stream of a CUDA device (0 for the null stream)."""
    return _raw_stream(device.index)


def stream_of(t: torch.Tensor) -> int:
    return _raw_stream(t.device.index)


def require_cuda(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise MingruHipError(
                "libmingru_hip kernels run on the GPU only; got a tensor on "
                f"{t.device}. There is no CPU path in the product; the CPU restatement "
                "of the reference lives in oracle/ for tests.")
