"""bf16 MFMA matrix products of libmingru_hip.so (mg_gemm) for the nn.Linear
layers of the hot path (reference mingru/minGRU.py:45,71; mingru/minLM.py:17-23,
:75,:138): forward Y = X W^T (+ bias, + GELU), and the backward products
dX = dY W and dW = dY^T X (fp32, optionally accumulated).

All tensors are CUDA bf16 (fp32 for bias, dW and fp32 outputs), 2-D with a
unit inner stride; the functions launch on torch's current stream.
"""
import torch

from . import _lib

KCONTIG, MNCONTIG = 0, 1
EPI_NONE, EPI_BIAS, EPI_BIAS_GELU, EPI_GELU_GRAD = 0, 1, 2, 3
FLAG_ACCUMULATE, FLAG_DETERMINISTIC, FLAG_HILO, FLAG_STOCHASTIC = 1, 2, 4, 8


def _rows(t, name):
    if t.dim() != 2 or t.stride(1) != 1:
        raise _lib.MingruHipError(f"{name}: expected a 2-D tensor with unit inner stride, got "
                                  f"shape {tuple(t.shape)} strides {t.stride()}")
    return t.stride(0)


def spans_ok(rows, ld):
    """Whether a bf16 operand of `rows` rows at row stride `ld` fits mg_gemm's
    buffer ranges (under 2 GiB, with 256 rows of slack)."""
    return (rows + 256) * ld * 2 < (1 << 31)


def _row_step(n, *row_bytes):
    """Rows per launch for a row-parallel product over n rows: every operand
    (row_bytes: its bytes per row) then spans under 2 GiB, mg_gemm's buffer
    range (with its 256 rows of slack); a multiple of 256 rows."""
    r = ((1 << 31) - 1) // max(max(row_bytes), 1) - 257
    r = max(256, r // 256 * 256)
    return n if n <= r else r


def fits(a, w):
    """Whether linear_fwd(a, w) and linear_dx(a, w) (with a GELU pre-activation
    of a's rows) meet mg_gemm's rules: bf16 2-D tensors with unit inner
    stride, a's and both of w's dimensions and the row strides multiples of
    8, 16-byte aligned, every operand under 2 GiB."""
    return all(t.dtype == torch.bfloat16 and t.dim() == 2 and t.stride(1) == 1 and t.stride(0) % 8 == 0
               and t.data_ptr() % 16 == 0 for t in (a, w)) and a.shape[1] % 8 == 0 and \
        w.shape[0] % 8 == 0 and w.shape[1] % 8 == 0 and spans_ok(a.shape[0], max(a.stride(0), *w.shape)) and \
        spans_ok(w.shape[0], w.stride(0))


# Split-K partial buffers, one per (device, stream), grown on demand.
_WORKSPACES = {}
# mg_gemm_workspace_bytes by (layouts, shape, epilogue, output dtype, flags): a pure function
# of its arguments, asked once per shape instead of once per call.
_WS_BYTES = {}


def _workspace(device, nbytes):
    key = (device.index, _lib.raw_stream(device))
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws


def gemm(a, a_layout, b, b_layout, M, N, K, out, *, epilogue=EPI_NONE, bias=None, aux=None, accumulate=False,
         deterministic=None, hilo=False, stochastic=False):
    """out[M, N] (=|+=) epilogue(sum_k A(m, k) B(k, n)); see include/mingru_hip.h (mg_gemm).
    Results repeat bit for bit. deterministic (default: torch.are_deterministic_algorithms_enabled())
    also rules out the split along K, so the sum order depends only on K. hilo: A and B rows are
    [hi (K) | lo (K)] bf16 pairs and the product is fp32-accurate (three MFMA passes). stochastic: a bf16
    out is rounded stochastically (a gradient)."""
    if deterministic is None:
        deterministic = torch.are_deterministic_algorithms_enabled()
    flags = (FLAG_ACCUMULATE if accumulate else 0) | (FLAG_DETERMINISTIC if deterministic else 0) | \
        (FLAG_HILO if hilo else 0) | (FLAG_STOCHASTIC if stochastic else 0)
    _lib.require_cuda(a, b, out)
    if a.dtype != torch.bfloat16 or b.dtype != torch.bfloat16:
        raise _lib.MingruHipError(f"mg_gemm operands must be bfloat16 (got {a.dtype}, {b.dtype})")
    lda, ldb, ldc = _rows(a, "A"), _rows(b, "B"), _rows(out, "C")
    ldaux = _rows(aux, "aux") if aux is not None else 0
    if bias is not None and (bias.dtype != torch.float32 or not bias.is_contiguous()):
        raise _lib.MingruHipError("mg_gemm bias must be contiguous float32")
    L = _lib.lib()
    cd = _lib.dtype_code(out.dtype)
    wkey = (a_layout, b_layout, M, N, K, epilogue, cd, flags)
    wsb = _WS_BYTES.get(wkey)
    if wsb is None:
        wsb = _WS_BYTES[wkey] = L.mg_gemm_workspace_bytes(a_layout, b_layout, M, N, K, epilogue, cd, flags)
    ws = _workspace(out.device, wsb) if wsb else None
    rc = L.mg_gemm(a_layout, _lib.ptr(a), lda, b_layout, _lib.ptr(b), ldb, M, N, K, epilogue,
                   _lib.ptr(bias) if bias is not None else None, _lib.ptr(aux) if aux is not None else None, ldaux,
                   cd, _lib.ptr(out), ldc, flags, _lib.ptr(ws), ws.numel() if ws is not None else 0,
                   _lib.stream_of(out))
    _lib.check(rc, "mg_gemm")
    return out


def linear_fwd(x, w, bias=None, *, gelu_pre=None, out_dtype=torch.bfloat16):
    """x [N, in] bf16, w [out, in] bf16 -> x w^T (+ bias) [N, out].
    gelu_pre: if given ([N, out] bf16), receives x w^T + bias and the result is gelu of it."""
    n, k = x.shape
    o = w.shape[0]
    y = torch.empty(n, o, device=x.device, dtype=out_dtype)
    if gelu_pre is not None:
        epi = EPI_BIAS_GELU
    else:
        epi = EPI_BIAS if bias is not None else EPI_NONE
    step = _row_step(n, 2 * x.stride(0), o * y.element_size(), 2 * o if gelu_pre is not None else 0)
    for r0 in range(0, n, step):
        r1 = min(n, r0 + step)
        gemm(x[r0:r1], KCONTIG, w, KCONTIG, r1 - r0, o, k, y[r0:r1], epilogue=epi, bias=bias,
             aux=gelu_pre[r0:r1] if gelu_pre is not None else None)
    return y


def hilo_prefix_fits(x_pair, w_pair, K, hilo_cols):
    """Whether linear_fwd_hilo_prefix takes these operands (mg_gemm_hilo_prefix's rules)."""
    N = w_pair.shape[0]
    return (K % 128 == 0 and hilo_cols % 256 == 0 and 0 < hilo_cols < N and N % 8 == 0 and
            all(t.dtype == torch.bfloat16 and t.stride(1) == 1 and t.stride(0) % 8 == 0 and t.stride(0) >= 2 * K and
                t.data_ptr() % 16 == 0 for t in (x_pair, w_pair)) and
            spans_ok(x_pair.shape[0], x_pair.stride(0)) and spans_ok(N, w_pair.stride(0)))


def linear_fwd_hilo_prefix(x_pair, w_pair, out, K, hilo_cols):
    """out[N, O] (bf16) = x w^T from hi/lo pairs x_pair [N, 2K], w_pair [O, 2K]: columns below
    hilo_cols to fp32 accuracy, the rest from the hi halves alone, in one launch
    (mg_gemm_hilo_prefix)."""
    L = _lib.lib()
    _lib.check(L.mg_gemm_hilo_prefix(_lib.ptr(x_pair), _rows(x_pair, "x_pair"), _lib.ptr(w_pair), _rows(w_pair, "w_pair"),
                                     x_pair.shape[0], w_pair.shape[0], K, hilo_cols, _lib.ptr(out), _rows(out, "out"),
                                     _lib.stream_of(out)), "mg_gemm_hilo_prefix")
    return out


def split_hilo(x, out=None):
    """fp32 [rows, cols] (unit inner stride) -> bf16 [rows, 2 cols] = [bf16(x) | bf16(x - bf16(x))]
    (mg_split_hilo), the operand form of hilo products."""
    rows, cols = x.shape
    if out is None:
        out = torch.empty(rows, 2 * cols, dtype=torch.bfloat16, device=x.device)
    L = _lib.lib()
    _lib.check(L.mg_split_hilo(_lib.ptr(x), _rows(x, "x"), rows, cols, _lib.ptr(out), _rows(out, "out"),
                               _lib.stream_of(x)), "mg_split_hilo")
    return out


def round_bf16_sr(x, salt=0x3c1d):
    """fp32 tensor (contiguous, numel % 4 == 0) -> bf16, rounded stochastically (mg_round_bf16_sr)."""
    out = torch.empty(x.shape, dtype=torch.bfloat16, device=x.device)
    _lib.check(_lib.lib().mg_round_bf16_sr(_lib.ptr(x), x.numel(), _lib.ptr(out), salt, _lib.stream_of(x)),
               "mg_round_bf16_sr")
    return out


def linear_fwd_hilo(x_pair, w_pair, out, K, bias=None):
    """out[N, O] = x w^T (+ bias, fp32 [O]) to fp32 accuracy from hi/lo pairs: x_pair [N, 2K],
    w_pair [O, 2K] (bf16); out bf16 or fp32, any row stride."""
    n, o = x_pair.shape[0], w_pair.shape[0]
    step = _row_step(n, 2 * x_pair.stride(0), out.stride(0) * out.element_size())
    for r0 in range(0, n, step):
        r1 = min(n, r0 + step)
        gemm(x_pair[r0:r1], KCONTIG, w_pair, KCONTIG, r1 - r0, o, K, out[r0:r1], hilo=True,
             epilogue=EPI_BIAS if bias is not None else EPI_NONE, bias=bias)
    return out


# limb patterns of mg_split_limbs (2 bits per segment: 0 h, 1 m, 2 l): a product of an operand
# split with LIMBS_A and one split with LIMBS_B over the 6-fold K sums hh + mh + hm + mm + lh + hl
LIMBS_A = 0 | 1 << 2 | 0 << 4 | 1 << 6 | 2 << 8 | 0 << 10   # h m h m l h
LIMBS_B = 0 | 0 << 2 | 1 << 4 | 1 << 6 | 0 << 8 | 2 << 10   # h h m m h l


def split_limbs(x, pattern, stack_rows):
    """fp32 x [rows, cols] (unit inner stride) -> its six bf16 limb segments (mg_split_limbs):
    [rows, 6 cols] side by side (stack_rows False: a K-contiguous operand over 6 cols) or
    [6 rows, cols] stacked (stack_rows True: an MN-contiguous operand over 6 rows)."""
    rows, cols = x.shape
    out = torch.empty((6 * rows, cols) if stack_rows else (rows, 6 * cols), dtype=torch.bfloat16, device=x.device)
    _lib.check(_lib.lib().mg_split_limbs(_lib.ptr(x), _rows(x, "x"), rows, cols, pattern, 6, int(stack_rows),
                                         _lib.ptr(out), out.stride(0), _lib.stream_of(x)), "mg_split_limbs")
    return out


def linear_dx(dy, w, *, gelu_pre=None, out_dtype=torch.bfloat16, stochastic=False):
    """dy [N, out] bf16, w [out, in] bf16 -> dy w [N, in] (bf16 or fp32); times gelu'(gelu_pre) when given
    (then rounded stochastically); stochastic: a plain bf16 result rounded stochastically."""
    n, o = dy.shape
    k = w.shape[1]
    dx = torch.empty(n, k, device=dy.device, dtype=out_dtype)
    step = _row_step(n, 2 * dy.stride(0), k * dx.element_size(), 2 * k if gelu_pre is not None else 0)
    for r0 in range(0, n, step):
        r1 = min(n, r0 + step)
        gemm(dy[r0:r1], KCONTIG, w, MNCONTIG, r1 - r0, k, o, dx[r0:r1],
             epilogue=EPI_GELU_GRAD if gelu_pre is not None else EPI_NONE,
             aux=gelu_pre[r0:r1] if gelu_pre is not None else None,
             stochastic=stochastic and gelu_pre is None and out_dtype == torch.bfloat16)
    return dx


def linear_dw_pair(dy0, x0, dy1, x1, deterministic=None, out0=None, out1=None, accumulate=False):
    """(dy0^T x0, dy1^T x1), fp32, over the same rows: the FeedForward's two weight gradients in one
    K-split launch (mg_gemm_wgrad_pair; each product alone where the pair does not apply). Operands
    over 2 GiB go through linear_dw one product at a time. accumulate: added into out0 and out1
    (both given, fp32 contiguous) instead of written."""
    n = dy0.shape[0]
    if deterministic is None:
        deterministic = torch.are_deterministic_algorithms_enabled()
    if dy1.shape[0] != n or x0.shape[0] != n or x1.shape[0] != n:
        raise _lib.MingruHipError("linear_dw_pair: the four operands must have the same number of rows")
    if accumulate and (out0 is None or out1 is None):
        raise _lib.MingruHipError("linear_dw_pair: accumulate needs both outputs")
    if _row_step(n, 2 * dy0.stride(0), 2 * x0.stride(0), 2 * dy1.stride(0), 2 * x1.stride(0)) < n:
        return (linear_dw(dy0, x0, out=out0, accumulate=accumulate, deterministic=deterministic),
                linear_dw(dy1, x1, out=out1, accumulate=accumulate, deterministic=deterministic))
    _lib.require_cuda(dy0, x0, dy1, x1)
    if any(t.dtype != torch.bfloat16 for t in (dy0, x0, dy1, x1)):
        raise _lib.MingruHipError("linear_dw_pair operands must be bfloat16")
    (m0, n0), (m1, n1) = (dy0.shape[1], x0.shape[1]), (dy1.shape[1], x1.shape[1])
    if out0 is None:
        out0 = torch.empty(m0, n0, device=dy0.device, dtype=torch.float32)
    if out1 is None:
        out1 = torch.empty(m1, n1, device=dy0.device, dtype=torch.float32)
    flags = (FLAG_DETERMINISTIC if deterministic else 0) | (FLAG_ACCUMULATE if accumulate else 0)
    L = _lib.lib()
    wsb = L.mg_gemm_wgrad_pair_workspace_bytes(m0, n0, m1, n1, n, flags)
    ws = _workspace(out0.device, wsb) if wsb else None
    rc = L.mg_gemm_wgrad_pair(_lib.ptr(dy0), _rows(dy0, "dy0"), _lib.ptr(x0), _rows(x0, "x0"), m0, n0,
                              _lib.ptr(out0), _rows(out0, "out0"), _lib.ptr(dy1), _rows(dy1, "dy1"), _lib.ptr(x1),
                              _rows(x1, "x1"), m1, n1, _lib.ptr(out1), _rows(out1, "out1"), n, flags, _lib.ptr(ws),
                              ws.numel() if ws is not None else 0, _lib.stream_of(out0))
    _lib.check(rc, "mg_gemm_wgrad_pair")
    return out0, out1


def linear_dw(dy, x, out=None, accumulate=False, deterministic=None):
    """dy [N, out] bf16, x [N, in] bf16 -> dy^T x [out, in] fp32 (written, or added when accumulate)."""
    n, o = dy.shape
    k = x.shape[1]
    if out is None:
        out = torch.empty(o, k, device=dy.device, dtype=torch.float32)
    # over 2 GiB of rows: the sum along rows in blocks, each added to the last
    step = _row_step(n, 2 * dy.stride(0), 2 * x.stride(0))
    for r0 in range(0, n, step):
        r1 = min(n, r0 + step)
        gemm(dy[r0:r1], MNCONTIG, x[r0:r1], MNCONTIG, o, k, r1 - r0, out, accumulate=accumulate or r0 > 0,
             deterministic=deterministic)
    return out
