"""Autograd Functions over the fused residual-add + RMSNorm kernels
(mg_add_rmsnorm_fwd / mg_add_rmsnorm_bwd).

Reference semantics: torch.nn.RMSNorm(dim) as used by mingru/minLM.py:67,
:69, :74 (eps=None -> float32 machine epsilon) and the residual adds at
mingru/minLM.py:125 and :130. The residual stream is kept in fp32; the
normalized output is produced in the activation dtype, optionally (bf16) as
a hi/lo pair [N, 2D] = [bf16(y) | bf16(y - bf16(y))] whose hi half is the
usual output: the operand of the fp32-accurate products (gemm HILO).
Weights of any floating dtype are accepted (a model cast with
.to(torch.bfloat16), as reference generate.py:140-142 does); the kernels read
them as fp32.
"""
import ctypes

import torch

from ._lib import check, dtype_code, lib, ptr, require_cuda, stream_of

FP32_EPS = float(torch.finfo(torch.float32).eps)


def _rows(t):
    D = t.shape[-1]
    return t.numel() // D, D


def _fwd(x, delta, w, out_dtype, with_lo=False):
    """Returns (x_out, y, rstd, pair): pair is the [..., 2D] hi/lo buffer
    (y is its first half) when with_lo, else None."""
    N, D = _rows(x)
    pair = None
    if with_lo:
        pair = torch.empty(*x.shape[:-1], 2 * D, dtype=torch.bfloat16, device=x.device)
        y = pair[..., :D]
    else:
        y = torch.empty(x.shape, dtype=out_dtype, device=x.device)
    rstd = torch.empty(N, dtype=torch.float32, device=x.device)
    x_out = torch.empty_like(x) if delta is not None else None
    rc = lib().mg_add_rmsnorm_fwd(ptr(x), dtype_code(delta.dtype) if delta is not None else 0, ptr(delta), ptr(w),
                                  ptr(x_out), dtype_code(y.dtype), ptr(y),
                                  ctypes.c_void_p(pair.data_ptr() + 2 * D) if with_lo else None,
                                  2 * D if with_lo else D, ptr(rstd), N, D, FP32_EPS, stream_of(x))
    check(rc, "mg_add_rmsnorm_fwd")
    return x_out, y, rstd, pair


def _bwd(xn, w, rstd, dy, dres, want_dx, delta_dtype, want_ddelta, dy_scale=None):
    """dy_scale: an optional fp32 device scalar dy is multiplied by as it is loaded."""
    N, D = _rows(xn)
    dev = xn.device
    if dy is None:
        dy = torch.zeros(xn.shape, dtype=torch.float32, device=dev)
    elif not dy.is_contiguous():
        dy = dy.contiguous()
    if dres is not None:
        dres = dres.to(torch.float32).contiguous()
    dx = torch.empty(xn.shape, dtype=torch.float32, device=dev) if want_dx else None
    ddelta = torch.empty(xn.shape, dtype=delta_dtype, device=dev) if want_ddelta else None
    dw = torch.empty(D, dtype=torch.float32, device=dev)
    L = lib()
    wsb = L.mg_add_rmsnorm_bwd_workspace_bytes(N, D)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    if dy_scale is not None:
        dy_scale = dy_scale.detach().to(device=dev, dtype=torch.float32).reshape(1)
    rc = L.mg_add_rmsnorm_bwd_scaled(ptr(xn), ptr(w), ptr(rstd), dtype_code(dy.dtype), ptr(dy), ptr(dy_scale),
                                     ptr(dres), ptr(dx), dtype_code(delta_dtype) if want_ddelta else 0,
                                     ptr(ddelta), ptr(dw), N, D, ptr(ws), wsb, stream_of(xn))
    check(rc, "mg_add_rmsnorm_bwd")
    return dx, ddelta, dw


class RMSNormResidualFn(torch.autograd.Function):
    """(x, rmsnorm(x) * w) for an fp32 x that also continues as the residual
    stream: the gradient reaching x through the residual joins the norm's
    gradient inside the backward kernel instead of in a separate add."""

    @staticmethod
    def forward(ctx, x, w, out_dtype, with_lo):
        _, y, rstd, pair = _fwd(x, None, w, out_dtype, with_lo)
        ctx.save_for_backward(x, w, rstd)
        ctx.set_materialize_grads(False)
        if pair is not None:
            ctx.mark_non_differentiable(pair)
        return x.view_as(x), y, pair

    @staticmethod
    def backward(ctx, dx_res, dy, _dpair):
        x, w, rstd = ctx.saved_tensors
        if dx_res is None and dy is None:
            return None, None, None, None
        dx, _, dw = _bwd(x, w, rstd, dy, dx_res, ctx.needs_input_grad[0], None, False)
        return dx, (dw if ctx.needs_input_grad[1] else None), None, None


class RMSNormFn(torch.autograd.Function):
    """y = x * w / sqrt(mean(x^2) + eps) over the last dim; x fp32, y in out_dtype."""

    @staticmethod
    def forward(ctx, x, w, out_dtype):
        _, y, rstd, _ = _fwd(x, None, w, out_dtype)
        ctx.save_for_backward(x, w, rstd)
        return y

    @staticmethod
    def backward(ctx, dy):
        x, w, rstd = ctx.saved_tensors
        dx, _, dw = _bwd(x, w, rstd, dy, None, ctx.needs_input_grad[0], None, False)
        return dx, (dw if ctx.needs_input_grad[1] else None), None


class AddRMSNormFn(torch.autograd.Function):
    """(x + delta, rmsnorm(x + delta) * w): the residual add fused with the next norm."""

    @staticmethod
    def forward(ctx, x, delta, w, out_dtype, with_lo):
        x_out, y, rstd, pair = _fwd(x, delta, w, out_dtype, with_lo)
        ctx.save_for_backward(x_out, w, rstd)
        ctx.delta_dtype = delta.dtype
        ctx.set_materialize_grads(False)  # an unused x_out (the final norm's) gets no zero tensor
        if pair is not None:
            ctx.mark_non_differentiable(pair)
        return x_out, y, pair

    @staticmethod
    def backward(ctx, dx_out, dy, _dpair):
        xn, w, rstd = ctx.saved_tensors
        if dx_out is None and dy is None:
            return None, None, None, None, None
        want_dx, want_dd = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        dx, dd, dw = _bwd(xn, w, rstd, dy, dx_out, want_dx, ctx.delta_dtype, want_dd)
        return dx, dd, (dw if ctx.needs_input_grad[2] else None), None, None


def _check(x, w, delta=None):
    """Validates the operands; returns the weight as fp32 (a cast that autograd
    differentiates, for models whose parameters are bf16 or fp16)."""
    require_cuda(x, w, delta)
    if x.dtype != torch.float32:
        raise ValueError(f"the residual stream must be float32, got {x.dtype}")
    if not w.is_floating_point() or w.dim() != 1 or w.shape[0] != x.shape[-1]:
        raise ValueError(f"weight must be a floating [{x.shape[-1]}] vector, got {w.dtype} {tuple(w.shape)}")
    if delta is not None and delta.shape != x.shape:
        raise ValueError(f"delta {tuple(delta.shape)} must match x {tuple(x.shape)}")
    return w if w.dtype == torch.float32 else w.float()


def _lo_ok(out_dtype, with_lo):
    if with_lo and out_dtype != torch.bfloat16:
        raise ValueError("the hi/lo pair output needs a bfloat16 output")
    return with_lo


def rms_norm(x, w, out_dtype=None):
    """RMSNorm of an fp32 tensor over its last dim with fp32 epsilon; output in out_dtype."""
    w = _check(x, w)
    return RMSNormFn.apply(x.contiguous(), w, out_dtype or x.dtype)


def rms_norm_residual(x, w, out_dtype=None, with_lo=False):
    """Returns (x, rms_norm(x, w), pair) where the first output carries x on as
    the residual stream (one backward kernel for both uses of x); pair is the
    hi/lo buffer when with_lo (bf16 output; the second output is its hi half),
    else None."""
    w = _check(x, w)
    out_dtype = out_dtype or x.dtype
    return RMSNormResidualFn.apply(x.contiguous(), w, out_dtype, _lo_ok(out_dtype, with_lo))


def add_rms_norm(x, delta, w, out_dtype=None, with_lo=False):
    """Returns (x + delta, rms_norm(x + delta, w), pair); x fp32, delta fp32 or
    bf16; pair as in rms_norm_residual."""
    w = _check(x, w, delta)
    out_dtype = out_dtype or x.dtype
    return AddRMSNormFn.apply(x.contiguous(), delta.contiguous(), w, out_dtype, _lo_ok(out_dtype, with_lo))
