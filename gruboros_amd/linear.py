"""Linear layers in the activation dtype with fp32 master weights.

The reference trains nn.Linear layers in fp32 (mingru/minGRU.py:40-41,
mingru/minLM.py:17-23, :75). Here, for bf16 activations, each weight keeps
a bf16 copy next to its fp32 master:
  * the copy is written by the fused optimizer step together with the
    master (no separate cast pass per forward), and is re-made from the
    master whenever the master's version counter shows an in-place change
    made by anything else (load_state_dict, the gossip blend of reference
    gossip/evolutionary_node.py:267-296, optimizer.eval()/train());
  * the backward produces the weight gradient directly in fp32 (bf16 x bf16
    GEMM with fp32 output), so no cast of the gradient either.
With fp32 activations this is plain F.linear.
"""
import torch
import torch.nn.functional as F

_MM_OUT_DTYPE = None  # whether torch.mm(..., out_dtype=float32) works for bf16 on this build


def _mm_f32(a, b):
    """a @ b with bf16 inputs and an fp32 result."""
    global _MM_OUT_DTYPE
    if _MM_OUT_DTYPE is None:
        try:
            torch.mm(a[:1, :1], b[:1, :1], out_dtype=torch.float32)
            _MM_OUT_DTYPE = True
        except (RuntimeError, TypeError):
            _MM_OUT_DTYPE = False
    if _MM_OUT_DTYPE:
        return torch.mm(a, b, out_dtype=torch.float32)
    return torch.mm(a, b).float()


def bf16_copy(w):
    """The bf16 copy of fp32 parameter w, re-made if w changed in place."""
    cache = getattr(w, "_mg_bf16", None)
    if cache is None or cache[0] != w._version or cache[1].device != w.device or cache[1].shape != w.shape:
        cache = (w._version, w.detach().to(torch.bfloat16))
        w._mg_bf16 = cache
    return cache[1]


class BF16Linear(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w, b, wb):
        bb = b.to(torch.bfloat16) if b is not None else None
        y = F.linear(x, wb, bb)
        ctx.save_for_backward(x, wb)
        ctx.has_bias = b is not None
        return y

    @staticmethod
    def backward(ctx, dy):
        x, wb = ctx.saved_tensors
        out_f, in_f = wb.shape
        dy2 = dy.reshape(-1, out_f)
        dx = dw = db = None
        if ctx.needs_input_grad[0]:
            dx = torch.mm(dy2, wb).reshape(*dy.shape[:-1], in_f)
        if ctx.needs_input_grad[1]:
            dw = _mm_f32(dy2.t(), x.reshape(-1, in_f))
        if ctx.has_bias and ctx.needs_input_grad[2]:
            db = dy2.sum(0, dtype=torch.float32)
        return dx, dw, db, None


def linear(x, layer):
    """layer(x) in x's dtype: fp32 -> F.linear; bf16 -> BF16Linear over the cached bf16 weight."""
    w, b = layer.weight, layer.bias
    if x.dtype == w.dtype:
        return F.linear(x, w, b)
    if x.dtype != torch.bfloat16 or w.dtype != torch.float32:
        raise TypeError(f"unsupported linear: activations {x.dtype}, weight {w.dtype}")
    return BF16Linear.apply(x, w, b, bf16_copy(w))
