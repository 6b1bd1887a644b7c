"""Block-level autograd functions of the bf16 minLM training path.

Reference mingru/minLM.py:107-149: per layer
    x = minGRU(RMSNorm(x)) + x        (:119-125)
    x = FeedForward(RMSNorm(x)) + x   (:127-130)
then the final RMSNorm, the logits and the cross-entropy (:137-149).

Here each of those three pieces is one torch.autograd.Function (bf16
activations over fp32 master weights):

  MinGRUBlock   x1 = x + pending; n = RMSNorm(x1) as a hi/lo pair;
                hg = [n W_h^T (fp32-accurate) | n W_g^T]; h = scan(hg) in fp32;
                expansion 1: the scan writes x2 = x1 + h itself (h is kept only as
                fp32 checkpoints); else out = to_out(h) (fp32-accurate).
  FFBlock       x2 = x1 + out (or x2 as given); n2 = RMSNorm(x2);
                pending = FeedForward(n2) (bf16).
  FinalNormCE   embed = RMSNorm(x + pending); mean cross-entropy of
                embed W_out^T (streaming loss kernel).

Why blocks rather than one Function per op: every gradient a block stores
in bf16 (dlogits, the input-gradient products, dgate/dhidden, dpre, the
FeedForward output's gradient) is rounded stochastically by the kernel that
writes it. An autograd boundary at a bf16 tensor would instead cast its
incoming gradient to bf16 with round-to-nearest, whose errors at a near-
uniform softmax repeat across the rows of a label and add up in the weight
gradients (measured on the fp64 restatement: 4-7% at the cfg3 row count
against 0.5% with stochastic rounding). The gradients crossing block boundaries
are the fp32 residual stream's, the fp32 minGRU output's, and the bf16
FeedForward output's (stochastically rounded by the next block's norm).
"""
import torch

from . import _lib
from . import gemm
from .linear import bf16_copy, bf16_pair, column_sum, gelu_backward, gelu_backward_bias_grads, grad_target
from .norm import FP32_EPS  # noqa: F401  (the kernels' eps; norm._fwd passes it)
from .norm import _bwd as _norm_bwd
from .norm import _fwd as _norm_fwd
from .scan import _launch_bwd as _scan_bwd
from .scan import _launch_fwd as _scan_fwd
from .scan import _launch_fwd_residual as _scan_fwd_res

BF16 = torch.bfloat16

# The FeedForward's two weight gradients in one K-split launch
# (mg_gemm_wgrad_pair) instead of one launch each; likewise to_out's and
# to_hidden_and_gate's (expansion != 1).
FF_DW_PAIR = True

# At expansion 1 the scan adds its state to the residual stream itself
# (mg_scan_fwd_residual) and keeps h only as fp32 checkpoints for the backward;
# False: the scan writes h and the FeedForward's norm adds it.
SCAN_RESIDUAL = True

# The FeedForward backward's GELU backward and both bias gradients in one launch
# (mg_ff_bias_bwd); False: mg_gelu_bwd and mg_column_sum separately.
FF_BIAS_BWD_FUSED = True

# to_hidden_and_gate's forward as one launch (mg_gemm_hilo_prefix: the hidden
# half's tiles hi/lo, the gate half's plain) instead of two.
HG_ONE_LAUNCH = True


def _f32(b):
    """A bias as the fp32 contiguous vector the GEMM epilogue adds."""
    return b if b.dtype == torch.float32 and b.is_contiguous() else b.float().contiguous()


class MinGRUBlock(torch.autograd.Function):
    """(x, pending) -> (x_next, out, h_last); see the module docstring.

    x: fp32 [B, T, D] residual stream; pending: bf16 [B, T, D] (the previous
    FeedForward's output, not yet added) or None; w_norm fp32 [D]; w_hg fp32
    master [2 Di, D]; h0 fp32 [B, Di] or None; w_to fp32 master [D, Di] or None.
    Without to_out (expansion 1): x_next = x + pending + h (the scan adds its
    state to the residual stream) and out is None. With it: x_next = x + pending
    and out = to_out(h), fp32 [B, T, D]. h_last fp32 [B, 1, Di]."""

    @staticmethod
    def forward(ctx, x, pending, w_norm, w_hg, h0, w_to):
        ctx.set_materialize_grads(False)
        B, T, D = x.shape
        N, Di = B * T, w_hg.shape[0] // 2
        ctx.w_hg, ctx.w_to = w_hg, w_to  # for their .grad (weight gradients added in place, grad_target)
        x2 = x.reshape(N, D)
        p2 = pending.reshape(N, D) if pending is not None else None
        x_out, n, rstd, pair = _norm_fwd(x2, p2, w_norm, BF16, with_lo=True)
        xn = x_out if x_out is not None else x2
        whp, whb = bf16_pair(w_hg), bf16_copy(w_hg)
        hg = torch.empty(N, 2 * Di, dtype=BF16, device=x.device)
        if HG_ONE_LAUNCH and gemm.hilo_prefix_fits(pair, whp, D, Di):
            gemm.linear_fwd_hilo_prefix(pair, whp, hg, D, Di)                   # minGRU.py:45, both halves
        else:
            gemm.linear_fwd_hilo(pair, whp[:Di], hg[:, :Di], D)                # minGRU.py:45, hidden half
            gemm.gemm(n, gemm.KCONTIG, whb[Di:], gemm.KCONTIG, N, Di, D, hg[:, Di:])  # gate half
        hg3 = hg.view(B, T, 2 * Di)
        if w_to is None and SCAN_RESIDUAL:
            # minGRU.py:47-69 and the residual add of minLM.py:125 in one pass; the
            # backward rebuilds h from the fp32 checkpoints
            x2, h_last, ckpt = _scan_fwd_res(hg3[..., :Di], hg3[..., Di:], h0, xn.view(B, T, D))
            ctx.save_for_backward(xn, w_norm, rstd, pair, hg, None, h0, whb, ckpt)
            ctx.dims = (B, T, D, Di)
            ctx.has_pending, ctx.has_to, ctx.res = pending is not None, False, True
            return x2, None, h_last
        h, h_last, _ = _scan_fwd(hg3[..., :Di], hg3[..., Di:], h0, torch.float32)   # minGRU.py:47-69
        saved = [xn, w_norm, rstd, pair, hg, h, h0, whb]
        if w_to is not None:                                                   # minGRU.py:71
            h_pair = gemm.split_hilo(h.view(N, Di))
            out = torch.empty(N, D, dtype=torch.float32, device=x.device)
            gemm.linear_fwd_hilo(h_pair, bf16_pair(w_to), out, Di)
            out = out.view(B, T, D)
            saved += [h_pair, bf16_copy(w_to)]
        else:
            out = h
        ctx.save_for_backward(*saved)
        ctx.dims = (B, T, D, Di)
        ctx.has_pending, ctx.has_to, ctx.res = pending is not None, w_to is not None, False
        x1 = x_out.view(B, T, D) if x_out is not None else x.view_as(x)
        return x1, out, h_last

    @staticmethod
    def backward(ctx, dx1, dout, dh_last):
        B, T, D, Di = ctx.dims
        N = B * T
        saved = ctx.saved_tensors
        xn, w_norm, rstd, pair, hg, h, h0, whb = saved[:8]
        ckpt = None
        dev = xn.device
        dW_to = None
        if ctx.res:
            # x_next = x1 + h: h and the residual get the same gradient
            ckpt = saved[8]
            dh = dx1
        elif dout is None:
            dh = None
        elif ctx.has_to:
            h_pair, wtb = saved[8:10]
            dob = gemm.round_bf16_sr(dout.reshape(N, D).contiguous().float())
            dh = gemm.linear_dx(dob, wtb, out_dtype=torch.float32).view(B, T, Di)
            if ctx.needs_input_grad[5] and not (FF_DW_PAIR and ctx.needs_input_grad[3]):
                g_to = grad_target(ctx.w_to)
                if g_to is not None:
                    gemm.linear_dw(dob, h_pair[:, :Di], out=g_to, accumulate=True)
                else:
                    dW_to = gemm.linear_dw(dob, h_pair[:, :Di])
        else:
            dh = dout.float()
        dhg = torch.empty(N, 2 * Di, dtype=BF16, device=dev)
        hg3, dhg3 = hg.view(B, T, 2 * Di), dhg.view(B, T, 2 * Di)
        want_dh0 = h0 is not None and ctx.needs_input_grad[4]
        if dh is None and dh_last is None:
            dhg.zero_()
            dh0 = torch.zeros_like(h0) if want_dh0 else None
        else:
            dh0 = _scan_bwd(hg3[..., :Di], hg3[..., Di:], h0, h, ckpt, dh, dh_last, dhg3[..., :Di], dhg3[..., Di:],
                            want_dh0)
        dn = gemm.linear_dx(dhg, whb, stochastic=True)             # bf16, stochastically rounded
        dW_hg = None
        if ctx.needs_input_grad[3]:
            g_hg = grad_target(ctx.w_hg)
            if ctx.has_to and dout is not None and ctx.needs_input_grad[5] and FF_DW_PAIR:
                # to_out's and to_hidden_and_gate's weight gradients in one launch
                g_to = grad_target(ctx.w_to)
                if g_to is not None and g_hg is not None:
                    gemm.linear_dw_pair(dob, h_pair[:, :Di], dhg, pair[:, :D], out0=g_to, out1=g_hg, accumulate=True)
                else:
                    dW_to, dW_hg = gemm.linear_dw_pair(dob, h_pair[:, :Di], dhg, pair[:, :D])
            elif g_hg is not None:
                gemm.linear_dw(dhg, pair[:, :D], out=g_hg, accumulate=True)
            else:
                dW_hg = gemm.linear_dw(dhg, pair[:, :D])
        dres = dx1.reshape(N, D) if dx1 is not None else None
        dx, dpend, dw_norm = _norm_bwd(xn, w_norm, rstd, dn, dres, True, BF16, ctx.has_pending)
        return (dx.view(B, T, D), dpend.view(B, T, D) if dpend is not None else None,
                dw_norm if ctx.needs_input_grad[2] else None, dW_hg,
                dh0.reshape(h0.shape) if dh0 is not None else None, dW_to)


class FFBlock(torch.autograd.Function):
    """(x1, out) -> (x2 = x1 + out, pending = FeedForward(RMSNorm(x2))).

    x1 fp32 [B, T, D]; out fp32 [B, T, D] (the minGRU branch), or None when
    x1 already holds it (then x2 is x1, returned as is); FeedForward =
    Linear(D, F) -> GELU -> Linear(F, D) (reference mingru/minLM.py:17-23)
    with fp32 masters; pending bf16. Forward and backward products run on
    mg_gemm: the first with the bias + GELU epilogue (pre-activation and
    activation written in one pass), the second with the bias epilogue."""

    @staticmethod
    def forward(ctx, x1, out, w_norm, w1, b1, w2, b2):
        ctx.set_materialize_grads(False)
        B, T, D = x1.shape
        N = B * T
        ctx.w1, ctx.w2 = w1, w2  # for their .grad (weight gradients added in place, grad_target)
        x2, n2, rstd, _ = _norm_fwd(x1.reshape(N, D), out.reshape(N, D) if out is not None else None, w_norm, BF16)
        ctx.has_out = out is not None
        if x2 is None:
            x2 = x1.reshape(N, D)
        w1b, w2b = bf16_copy(w1), bf16_copy(w2)
        pre = torch.empty(N, w1.shape[0], dtype=BF16, device=x1.device)
        act = gemm.linear_fwd(n2, w1b, _f32(b1), gelu_pre=pre)   # pre = n2 W1^T + b1, act = gelu(pre)
        pend = gemm.linear_fwd(act, w2b, _f32(b2))                # act W2^T + b2
        ctx.save_for_backward(x2, w_norm, rstd, n2, pre, act, w1b, w2b)
        ctx.dims = (B, T, D)
        return (x2.view(B, T, D) if ctx.has_out else x1), pend.view(B, T, D)

    @staticmethod
    def backward(ctx, dx2, dpend):
        B, T, D = ctx.dims
        N = B * T
        x2, w_norm, rstd, n2, pre, act, w1b, w2b = ctx.saved_tensors
        dres = dx2.reshape(N, D) if dx2 is not None else None
        dW1 = db1 = dW2 = db2 = None
        if dpend is None:
            dn2 = torch.zeros(N, D, dtype=torch.float32, device=x2.device)
        else:
            dp = dpend.reshape(N, D)
            if dp.dtype != BF16 or not dp.is_contiguous():
                dp = dp.to(BF16).contiguous()
            dact = gemm.linear_dx(dp, w2b, stochastic=True)            # bf16, stochastically rounded
            if FF_BIAS_BWD_FUSED:
                dpre, db1, db2 = gelu_backward_bias_grads(dact, pre, dp)  # dpre bf16, stochastically rounded
            else:
                (dpre, db1), db2 = gelu_backward(dact, pre), column_sum(dp)
            dn2 = gemm.linear_dx(dpre, w1b, stochastic=True)           # bf16, stochastically rounded
            g1, g2 = grad_target(ctx.w1), grad_target(ctx.w2)
            if FF_DW_PAIR and g1 is not None and g2 is not None:
                gemm.linear_dw_pair(dp, act, dpre, n2, out0=g2, out1=g1, accumulate=True)  # into .grad
            elif FF_DW_PAIR:
                dW2, dW1 = gemm.linear_dw_pair(dp, act, dpre, n2)     # one launch for both weight gradients
            else:
                if g2 is not None:
                    gemm.linear_dw(dp, act, out=g2, accumulate=True)
                else:
                    dW2 = gemm.linear_dw(dp, act)
                if g1 is not None:
                    gemm.linear_dw(dpre, n2, out=g1, accumulate=True)
                else:
                    dW1 = gemm.linear_dw(dpre, n2)
        # x2 = x1 + out: both inputs get the same gradient, written once and returned for both
        # (the consumer, MinGRUBlock.backward, only reads them)
        dx1, _, dw_norm = _norm_bwd(x2, w_norm, rstd, dn2, dres, True, torch.float32, False)
        return dx1.view(B, T, D), (dx1.view(B, T, D) if ctx.has_out else None), dw_norm, dW1, db1, dW2, db2


class FinalNormCE(torch.autograd.Function):
    """mean CE(RMSNorm(x + pending) W_out^T, labels) (reference mingru/minLM.py:137-149)
    for V <= 256 classes on the streaming loss kernel (logits never in memory).
    x fp32 [B, T, D], pending bf16 [B, T, D] or None, labels int64 [B, T]."""

    @staticmethod
    def forward(ctx, x, pending, w_norm, w_out, labels):
        B, T, D = x.shape
        N = B * T
        V = w_out.shape[0]
        x2 = x.reshape(N, D)
        x_out, embed, rstd, _ = _norm_fwd(x2, pending.reshape(N, D) if pending is not None else None, w_norm, BF16)
        xn = x_out if x_out is not None else x2
        wob = bf16_copy(w_out)
        L = _lib.lib()
        dl = torch.empty(N, V, dtype=BF16, device=x.device)
        part = torch.empty(L.mg_logits_cross_entropy_partials(N), dtype=torch.float32, device=x.device)
        lab = labels.reshape(-1).contiguous()
        _lib.check(L.mg_logits_cross_entropy(_lib.ptr(embed), embed.stride(0), _lib.ptr(wob), wob.stride(0),
                                             _lib.ptr(lab), _lib.ptr(dl), V, _lib.ptr(part), None, N, D, V, 1.0 / N,
                                             _lib.stream_of(embed)), "mg_logits_cross_entropy")
        ctx.save_for_backward(xn, w_norm, rstd, embed, dl, wob)
        ctx.dims = (B, T, D)
        ctx.has_pending = pending is not None
        return part.sum() / N

    @staticmethod
    def backward(ctx, g):
        B, T, D = ctx.dims
        xn, w_norm, rstd, embed, dl, wob = ctx.saved_tensors
        de = gemm.linear_dx(dl, wob, out_dtype=torch.float32)         # fp32, unscaled
        dW = gemm.linear_dw(dl, embed) if ctx.needs_input_grad[3] else None
        if dW is not None:
            dW.mul_(g)  # upstream scale (1 / grad_accum in the reference loop), in fp32; no host sync
        # de's scale by g is the norm backward's, as it loads de (the same fp32 products)
        dx, dpend, dw_norm = _norm_bwd(xn, w_norm, rstd, de, None, True, BF16, ctx.has_pending, dy_scale=g)
        return (dx.view(B, T, D), dpend.view(B, T, D) if dpend is not None else None,
                dw_norm if ctx.needs_input_grad[2] else None, dW, None)


def supported(model):
    """Whether the block path applies: bf16 activations over fp32 masters, no
    conv, no dropout, a loss head the streaming kernel takes, and widths every
    product and kernel of the blocks takes (D, Di = D * expansion and the
    FeedForward's F multiples of 8; mg_gemm's N and K, the scan's Di % 4)."""
    D = model.dim
    V = model.to_logits.weight.shape[0]
    return (all(conv is None and dropout is None for conv, _, _, _, _, dropout in model.layers)
            and model.token_emb.weight.dtype == torch.float32 and D % 8 == 0 and V % 8 == 0 and V <= 256
            and all(gru.to_hidden_and_gate.weight.shape[0] % 16 == 0 and ff[0].weight.shape[0] % 8 == 0
                    for _, _, gru, _, ff, _ in model.layers))
