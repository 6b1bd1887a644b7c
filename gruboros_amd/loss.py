"""Loss head: logits projection + mean cross-entropy (reference
mingru/minLM.py:138, :146-149). For bf16 embeddings and V <= 256 classes the
logits product, log-softmax, loss and logits gradient are one kernel
(mg_logits_cross_entropy) and the fp32 logits never reach memory; otherwise
the logits are formed first and mg_cross_entropy_fwd_bwd does the rest in one
pass.
"""
import torch

from . import gemm
from ._lib import check, dtype_code, lib, ptr, require_cuda, stream_of
from .linear import _mm_f32, bf16_copy, f32_linear, f32_linear_applies


def _ce(logits2d, labels1d, grad_dtype):
    N, V = logits2d.shape
    L = lib()
    P = L.mg_cross_entropy_partials(N)
    dl = torch.empty(N, V, dtype=grad_dtype, device=logits2d.device)
    part = torch.empty(P, dtype=torch.float32, device=logits2d.device)
    rc = L.mg_cross_entropy_fwd_bwd(dtype_code(logits2d.dtype), ptr(logits2d), ptr(labels1d), dtype_code(grad_dtype),
                                    ptr(dl), ptr(part), None, N, V, 1.0 / N, stream_of(logits2d))
    check(rc, "mg_cross_entropy_fwd_bwd")
    return part.sum() / N, dl


class LogitsCrossEntropy(torch.autograd.Function):
    """mean_n CE(embed_n @ W^T, label_n); embed bf16 [N, D], W fp32 master [V, D]."""

    @staticmethod
    def forward(ctx, embed, w, wb, labels):
        N, D = embed.shape
        V = wb.shape[0]
        if V <= 256 and V % 8 == 0 and D % 8 == 0:
            L = lib()
            dl = torch.empty(N, V, dtype=torch.bfloat16, device=embed.device)
            part = torch.empty(L.mg_logits_cross_entropy_partials(N), dtype=torch.float32, device=embed.device)
            rc = L.mg_logits_cross_entropy(ptr(embed), embed.stride(0), ptr(wb), wb.stride(0), ptr(labels), ptr(dl),
                                           V, ptr(part), None, N, D, V, 1.0 / N, stream_of(embed))
            check(rc, "mg_logits_cross_entropy")
            loss = part.sum() / N
        else:
            logits = _mm_f32(embed, wb.t())               # [N, V] fp32
            loss, dl = _ce(logits, labels, torch.bfloat16)
        ctx.save_for_backward(embed, wb, dl)
        return loss

    @staticmethod
    def backward(ctx, g):
        embed, wb, dl = ctx.saved_tensors
        dl = dl * g  # upstream gradient (1/grad_accum in the reference loop); stays bf16
        de = torch.mm(dl, wb) if ctx.needs_input_grad[0] else None
        dw = gemm.linear_dw(dl, embed) if ctx.needs_input_grad[1] else None
        return de, dw, None, None


class CrossEntropyFromLogits(torch.autograd.Function):
    """mean_n CE(logits_n, label_n) for fp32 logits [N, V] (the fp32 path)."""

    @staticmethod
    def forward(ctx, logits, labels):
        loss, dl = _ce(logits, labels, torch.float32)
        ctx.save_for_backward(dl)
        return loss

    @staticmethod
    def backward(ctx, g):
        (dl,) = ctx.saved_tensors
        return dl * g, None


def logits_cross_entropy(embed, to_logits, labels):
    """Mean cross-entropy of to_logits(embed) against labels (int64), like
    F.cross_entropy(logits.transpose(1, 2), labels) in the reference."""
    require_cuda(embed, labels)
    D = embed.shape[-1]
    e2 = embed.reshape(-1, D)
    lab = labels.reshape(-1).contiguous()
    w = to_logits.weight
    if embed.dtype == torch.bfloat16 and w.dtype == torch.float32:
        return LogitsCrossEntropy.apply(e2.contiguous(), w, bf16_copy(w), lab)
    if f32_linear_applies(e2, w):
        logits = f32_linear(e2, w)  # the fp32 path: the logits product on mg_gemm over bf16 limbs
    else:
        logits = torch.nn.functional.linear(e2.to(w.dtype), w)  # (parameters cast to another dtype: product in it)
    return CrossEntropyFromLogits.apply(logits.float().contiguous(), lab)
