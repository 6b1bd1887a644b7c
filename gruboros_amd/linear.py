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
With fp32 activations and fp32 weights (the reference's own precision: an
unchanged train.py, cfg1's single layer) every product runs on mg_gemm over
three-limb bf16 splits, fp32-accurate on MFMA: F32Linear.

Two products are computed to fp32 accuracy from bf16 hi/lo pairs (mg_gemm
HILO: A_hi B_hi + A_lo B_hi + A_hi B_lo on MFMA): the hidden half of
to_hidden_and_gate (reference mingru/minGRU.py:45) and to_out (:71). The
reference's g(x) has a kink at 0 (g' jumps from 1/4 to 1), so a bf16-rounded
pre-activation that lands on the wrong side of 0 changes that element's
gradient by 75%; measured on the fp64 restatement at the cfg3 model size,
bf16-rounded inputs and weights there alone move the to_hidden_and_gate and
norm-weight gradients by ~3% (norm-relative), the accurate products bring
every gradient to ~1.3%. The gate half has no kink and stays a plain bf16
product.
"""
import torch
import torch.nn.functional as F

from . import gemm
from ._lib import check, dtype_code, lib, ptr, stream_of

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


# Weight gradients added into an existing .grad by the product itself (gradient
# accumulation over micro-steps or TBPTT chunks: every backward after the first)
# instead of autograd adding the product's fresh result; see grad_target.
ACCUMULATE_IN_PLACE = True


def grad_target(w):
    """w.grad, when this backward may add w's gradient into it directly and give autograd none:
    the engine will run w's AccumulateGrad (a .backward() that accumulates, not
    torch.autograd.grad), w.grad exists as an fp32 contiguous tensor of w's shape, and w has no
    gradient hooks. Else None (the gradient is returned to autograd as usual). Called from a
    backward."""
    if not ACCUMULATE_IN_PLACE or not isinstance(w, torch.Tensor) or not w.requires_grad:
        return None
    g = w.grad
    if (g is None or g.dtype != torch.float32 or g.shape != w.shape or not g.is_contiguous() or
            g.device != w.device or w._backward_hooks or getattr(w, "_post_accumulate_grad_hooks", None)):
        return None
    try:
        if not torch._C._will_engine_execute_node(torch.autograd.graph.get_gradient_edge(w).node):
            return None
    except (RuntimeError, AttributeError):
        return None
    return g


def _dw_ok(dy2, x2):
    """Shapes the MFMA weight-gradient product takes (mg_gemm, both operands MN-contiguous)."""
    return (dy2.dtype == torch.bfloat16 and x2.dtype == torch.bfloat16 and dy2.stride(1) == 1 and x2.stride(1) == 1
            and dy2.shape[1] % 8 == 0 and x2.shape[1] % 8 == 0 and dy2.stride(0) % 8 == 0 and x2.stride(0) % 8 == 0
            and dy2.data_ptr() % 16 == 0 and x2.data_ptr() % 16 == 0
            and gemm.spans_ok(dy2.shape[0], dy2.stride(0)) and gemm.spans_ok(x2.shape[0], x2.stride(0)))


def column_sum(x2):
    """fp32 column sums of a 2-D fp32/bf16 tensor with unit inner stride (mg_column_sum)."""
    N, C = x2.shape
    if C % 8 or x2.stride(1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        return x2.sum(0, dtype=torch.float32)
    L = lib()
    out = torch.empty(C, dtype=torch.float32, device=x2.device)
    ws = torch.empty(L.mg_column_sum_workspace_bytes(N, C), dtype=torch.uint8, device=x2.device)
    check(L.mg_column_sum(dtype_code(x2.dtype), ptr(x2), x2.stride(0), N, C, ptr(out), ptr(ws), ws.numel(),
                          stream_of(x2)), "mg_column_sum")
    return out


def _gelu_grad_f32(pre):
    """gelu'(x) = Phi(x) + x phi(x) in fp32 (exact erf form of nn.GELU())."""
    x = pre.float()
    return 0.5 * (1.0 + torch.erf(x * 0.7071067811865476)) + x * torch.exp(-0.5 * x * x) * 0.3989422804014327


def gelu_backward(dh, pre, want_bias_grad=True):
    """(bf16(dh * gelu'(pre)) rounded stochastically, its fp32 column sums) for a bf16 or fp32
    dh and bf16 pre, [N, C] (mg_gelu_bwd). Widths the kernel does not take (C % 8) run as
    torch elementwise ops in fp32, rounded to nearest."""
    N, C = pre.shape
    if C % 8 or C < 8 or pre.stride(1) != 1 or dh.stride(1) != 1 or pre.stride(0) % 8 or dh.stride(0) % 8:
        d = dh.float() * _gelu_grad_f32(pre)
        return d.to(pre.dtype), (d.sum(0) if want_bias_grad else None)
    L = lib()
    dpre = torch.empty_like(pre)
    db = torch.empty(C, dtype=torch.float32, device=pre.device) if want_bias_grad else None
    ws = torch.empty(L.mg_column_sum_workspace_bytes(N, C) if want_bias_grad else 16, dtype=torch.uint8,
                     device=pre.device)
    check(L.mg_gelu_bwd(dtype_code(dh.dtype), ptr(dh), dh.stride(0), ptr(pre), pre.stride(0), ptr(dpre),
                        dpre.stride(0), ptr(db), N, C, ptr(ws), ws.numel(), stream_of(pre)), "mg_gelu_bwd")
    return dpre, db


def bf16_copy(w, dense=False):
    """The bf16 copy of fp32 parameter w, re-made if w changed in place. Where w has a current
    hi/lo pair (bf16_pair) and `dense` is false, its hi half (a [rows, cols] view with row
    stride 2 cols); dense: a contiguous copy (the fused optimizer step keeps the pair current
    and drops this copy, which is then re-made from w on its next use)."""
    pair = getattr(w, "_mg_pair", None)
    if not dense and pair is not None and pair[0] == w._version and pair[1].device == w.device and \
            pair[1].shape == (w.shape[0], 2 * w.shape[1]):
        return pair[1][:, :w.shape[1]]
    cache = getattr(w, "_mg_bf16", None)
    if cache is None or cache[0] != w._version or cache[1].device != w.device or cache[1].shape != w.shape:
        cache = (w._version, w.detach().to(torch.bfloat16))
        w._mg_bf16 = cache
    return cache[1]


def bf16_pair(w):
    """The hi/lo pair [rows, 2 cols] of fp32 parameter w (gemm.split_hilo), re-made if w
    changed in place. The fused optimizer step rewrites it together with w (it changes w
    through a raw pointer, which torch's version counter does not see), or drops it where it
    cannot."""
    cache = getattr(w, "_mg_pair", None)
    if cache is None or cache[0] != w._version or cache[1].device != w.device or \
            cache[1].shape != (w.shape[0], 2 * w.shape[1]):
        cache = (w._version, gemm.split_hilo(w.detach()))
        w._mg_pair = cache
    return cache[1]


class HiddenGateProjection(torch.autograd.Function):
    """hg = [n W_hidden^T | n W_gate^T] (reference mingru/minGRU.py:45) in bf16, its hidden
    half computed to fp32 accuracy from the hi/lo pairs of n and W_hidden.

    n: [N, D] bf16, the hi half of `pair` ([N, 2D], from the norm kernel); w: fp32 master
    [2 Di, D] with its pair and bf16 copy. Backward: dn = dhg W (bf16), dW = dhg^T n (fp32)."""

    @staticmethod
    def forward(ctx, n, pair, w, w_pair, wb):
        N, D = n.shape
        Di = w.shape[0] // 2
        hg = torch.empty(N, 2 * Di, dtype=torch.bfloat16, device=n.device)
        gemm.linear_fwd_hilo(pair, w_pair[:Di], hg[:, :Di], D)
        gemm.gemm(n, gemm.KCONTIG, wb[Di:], gemm.KCONTIG, N, Di, D, hg[:, Di:])
        ctx.save_for_backward(n, wb)
        return hg

    @staticmethod
    def backward(ctx, dhg):
        n, wb = ctx.saved_tensors
        dhg = dhg.contiguous()
        dn = torch.mm(dhg, wb) if ctx.needs_input_grad[0] else None
        dw = None
        if ctx.needs_input_grad[2]:
            dw = gemm.linear_dw(dhg, n) if _dw_ok(dhg, n) else _mm_f32(dhg.t(), n)
        return dn, None, dw, None, None


def hidden_gate_projection(n, pair, layer):
    """to_hidden_and_gate(n) with the accurate hidden half; n [..., D] bf16 (hi half of pair).
    Widths mg_gemm does not take (D or Di not a multiple of 8) run the hidden half as an
    fp32 torch product of hi + lo (the same fp32-accurate value) and the gate half in bf16."""
    w = layer.weight
    shape = n.shape
    D, Di = shape[-1], w.shape[0] // 2
    if D % 8 or Di % 8:
        x32 = pair[..., :D].float() + pair[..., D:].float()
        x32 = n.float() + (x32 - n.float()).detach()  # value hi + lo, gradient to n
        hidden = F.linear(x32, w[:Di]).to(torch.bfloat16)
        gate = linear(n, _RowSlice(layer, Di))
        return torch.cat([hidden, gate], dim=-1)
    hg = HiddenGateProjection.apply(n.reshape(-1, shape[-1]), pair.reshape(-1, 2 * shape[-1]), w, bf16_pair(w),
                                    bf16_copy(w))
    return hg.view(*shape[:-1], w.shape[0])


class AccurateLinearF32(torch.autograd.Function):
    """y = x W^T to fp32 accuracy (hi/lo products) for an fp32 x [N, K] and fp32 master W;
    y fp32. Backward: dx = dy W in fp32, dW = dy^T x on bf16 operands (fp32 result)."""

    @staticmethod
    def forward(ctx, x, w, w_pair, wb):
        N, K = x.shape
        x_pair = gemm.split_hilo(x)
        y = torch.empty(N, w.shape[0], dtype=torch.float32, device=x.device)
        gemm.linear_fwd_hilo(x_pair, w_pair, y, K)
        ctx.save_for_backward(x_pair, wb)
        return y

    @staticmethod
    def backward(ctx, dy):
        x_pair, wb = ctx.saved_tensors
        K = wb.shape[1]
        dyb = dy.to(torch.bfloat16).contiguous()
        dx = gemm.linear_dx(dyb, wb, out_dtype=torch.float32) if ctx.needs_input_grad[0] else None
        dw = None
        if ctx.needs_input_grad[1]:
            xh = x_pair[:, :K]
            dw = gemm.linear_dw(dyb, xh) if _dw_ok(dyb, xh) else _mm_f32(dyb.t(), xh)
        return dx, dw, None, None


class _RowSlice:
    """rows [r0:] of a bias-free linear layer's weight, as `linear` takes a layer."""

    def __init__(self, layer, r0):
        self.weight, self.bias = layer.weight[r0:], None


def accurate_linear_f32(x, layer):
    """layer(x) (no bias) for an fp32 x, to fp32 accuracy on MFMA; fp32 output. Widths
    mg_gemm does not take (either dimension of the weight not a multiple of 8) run as an
    fp32 torch product."""
    w = layer.weight
    shape = x.shape
    if w.shape[0] % 8 or w.shape[1] % 8:
        return F.linear(x, w)
    y = AccurateLinearF32.apply(x.reshape(-1, shape[-1]).contiguous(), w, bf16_pair(w), bf16_copy(w))
    return y.view(*shape[:-1], w.shape[0])


class F32Linear(torch.autograd.Function):
    """y = x W^T (+ b) for fp32 x [N, K] and fp32 W [O, K] (reference nn.Linear in fp32:
    mingru/minGRU.py:40-41,45,71; minLM.py:17-23,75,138), all three products on MFMA to
    fp32 accuracy: each fp32 operand is split into three bf16 limbs (h + m + l == x,
    mg_split_limbs) and one plain bf16 product over the 6-fold reduction sums the six limb
    products through 2^-16 (hh, mh, hm, mm, lh, hl; the dropped ones are below 2^-24).
    Forward y = x W^T (+ b in the epilogue); backward dx = dy W (dy's limbs side by side,
    W's stacked), dW = dy^T x (both stacked along the rows, so no transposes and no
    padding), db = column sums of dy. The limbs are formed per call, so nothing cached can
    go stale when W changes.
    (Two limbs, x = hi + lo to 2^-16, are not enough here: the reference's g(x) has a kink
    at 0, and at cfg1's size a 4e-6 product error moves ~10 hidden pre-activations across
    it, 8e-4 on dx and dW.)"""

    @staticmethod
    def forward(ctx, x, w, b):
        y = gemm.linear_fwd(gemm.split_limbs(x, gemm.LIMBS_A, False), gemm.split_limbs(w.detach(), gemm.LIMBS_B, False),
                            b.detach().contiguous() if b is not None else None, out_dtype=torch.float32)
        ctx.save_for_backward(x, w)
        ctx.has_bias = b is not None
        return y

    @staticmethod
    def backward(ctx, dy):
        x, w = ctx.saved_tensors
        dy = dy.contiguous()
        dx = dw = db = None
        if ctx.needs_input_grad[0]:
            dx = gemm.linear_dx(gemm.split_limbs(dy, gemm.LIMBS_A, False), gemm.split_limbs(w.detach(), gemm.LIMBS_B, True),
                                out_dtype=torch.float32)
        if ctx.needs_input_grad[1]:
            dw = gemm.linear_dw(gemm.split_limbs(dy, gemm.LIMBS_A, True), gemm.split_limbs(x, gemm.LIMBS_B, True))
        if ctx.has_bias and ctx.needs_input_grad[2]:
            db = column_sum(dy)
        return dx, dw, db


def f32_linear_applies(x, w):
    """Whether F32Linear takes x [.., K] and w [O, K]: fp32 CUDA tensors, O and K multiples of 8."""
    return x.is_cuda and x.dtype == torch.float32 and w.dtype == torch.float32 and w.dim() == 2 and \
        w.shape[0] % 8 == 0 and w.shape[1] % 8 == 0


def f32_linear(x, w, b=None):
    """x W^T (+ b) for fp32 x and W on F32Linear, x of any leading shape."""
    shape = x.shape
    y = F32Linear.apply(x.reshape(-1, shape[-1]).contiguous(), w, b)
    return y.view(*shape[:-1], w.shape[0])


class BF16Linear(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w, b, wb):
        bb = bf16_copy(b) if b is not None else None
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
            x2 = x.reshape(-1, in_f)
            dw = gemm.linear_dw(dy2, x2) if _dw_ok(dy2, x2) else _mm_f32(dy2.t(), x2)
        if ctx.has_bias and ctx.needs_input_grad[2]:
            db = column_sum(dy2)
        return dx, dw, db, None


def linear(x, layer):
    """layer(x) in x's dtype: fp32 activations and weights on the GPU -> F32Linear (mg_gemm
    hi/lo, fp32-accurate); other equal dtypes, or widths F32Linear does not take -> F.linear;
    bf16 activations over fp32 masters -> BF16Linear over the cached bf16 weight; parameters
    in another dtype (a model cast to float16) -> the product in the parameters' dtype, the
    result back in x's."""
    w, b = layer.weight, layer.bias
    if x.dtype == w.dtype:
        if f32_linear_applies(x, w):
            return f32_linear(x, w, b)
        return F.linear(x, w, b)
    if x.dtype == torch.bfloat16 and w.dtype == torch.float32:
        return BF16Linear.apply(x, w, b, bf16_copy(w))
    return F.linear(x.to(w.dtype), w, b).to(x.dtype)


def gelu_backward_bias_grads(dh, pre, dy):
    """(dpre, db1, db2) of the FeedForward backward in one launch (mg_ff_bias_bwd): dpre =
    bf16(dh * gelu'(pre)) rounded stochastically with its fp32 column sums db1 (as
    gelu_backward), and db2 = the fp32 column sums of dy (as column_sum). dh bf16 or fp32 and
    pre bf16 [N, F], dy bf16 [N, D]; widths the kernels do not take fall back to the two
    separate calls."""
    N, C1 = pre.shape
    C2 = dy.shape[1]
    if (C1 % 8 or C2 % 8 or dy.dtype != torch.bfloat16 or pre.stride(1) != 1 or dh.stride(1) != 1 or
            dy.stride(1) != 1 or pre.stride(0) % 8 or dh.stride(0) % 8 or dy.stride(0) % 8 or dy.data_ptr() % 16):
        dpre, db1 = gelu_backward(dh, pre)
        return dpre, db1, column_sum(dy)
    L = lib()
    dpre = torch.empty_like(pre)
    db1 = torch.empty(C1, dtype=torch.float32, device=pre.device)
    db2 = torch.empty(C2, dtype=torch.float32, device=pre.device)
    wsb = L.mg_ff_bias_bwd_workspace_bytes(N, C1, C2)
    ws = torch.empty(wsb, dtype=torch.uint8, device=pre.device)
    check(L.mg_ff_bias_bwd(dtype_code(dh.dtype), ptr(dh), dh.stride(0), ptr(pre), pre.stride(0), ptr(dpre),
                           dpre.stride(0), ptr(db1), N, C1, ptr(dy), dy.stride(0), ptr(db2), C2, ptr(ws), wsb,
                           stream_of(pre)), "mg_ff_bias_bwd")
    return dpre, db1, db2


# Where the GELU of the FeedForward runs (measured on MI355X, 16384 x 1024
# activations, F = 4096):
#   forward: mg_gemm with the bias + GELU epilogue (its GELU from a bf16
#     table), 154 us, against 175 us for hipBLASLt's x W1^T + b1 and torch's
#     GELU pass; the second product on mg_gemm too;
#   backward: hipBLASLt's dY W2 and mg_gelu_bwd (fused with the first bias
#     gradient), 208 us against 244 us for mg_gemm's GELU-gradient epilogue
#     plus a column sum (that epilogue's VALU work runs after the tile's MFMA
#     loop with nothing to overlap it).
# Both fused forms are exact and tested.
FUSED_GELU_FORWARD = True
FUSED_GELU_BACKWARD = False


class BF16FeedForward(torch.autograd.Function):
    """Linear -> GELU -> Linear (reference mingru/minLM.py:17-23) in bf16 with
    fp32 weight gradients. Forward: mg_gemm with the bias + GELU epilogue
    (keeping bf16(x W1^T + b1) for the backward) and the bias epilogue, or
    (FUSED_GELU_FORWARD off, or widths mg_gemm does not take) hipBLASLt (via
    torch) and a GELU pass. Backward: either mg_gemm's GELU-gradient
    epilogue on dY W2 or hipBLASLt's dY W2 and mg_gelu_bwd; weight gradients
    on mg_gemm, bias gradients on mg_column_sum / mg_gelu_bwd."""

    @staticmethod
    def forward(ctx, x, w1, b1, w2, b2, w1b, w2b, b1b, b2b):
        shape = x.shape
        x2 = x.reshape(-1, shape[-1])
        if not x2.is_contiguous():
            x2 = x2.contiguous()
        if FUSED_GELU_FORWARD and gemm.fits(x2, w1b):
            pre = torch.empty(x2.shape[0], w1b.shape[0], device=x.device, dtype=torch.bfloat16)
            h = gemm.linear_fwd(x2, w1b, b1.detach().float().contiguous(), gelu_pre=pre)
        else:
            pre = F.linear(x2, w1b, b1b)
            h = F.gelu(pre)
        if FUSED_GELU_FORWARD and gemm.fits(h, w2b):
            y = gemm.linear_fwd(h, w2b, b2.detach().float().contiguous())
        else:
            y = F.linear(h, w2b, b2b)
        ctx.save_for_backward(x2, pre, h, w1b, w2b)
        return y.view(*shape[:-1], w2b.shape[0])

    @staticmethod
    def backward(ctx, dy):
        x2, pre, h, w1b, w2b = ctx.saved_tensors
        dy2 = dy.reshape(-1, dy.shape[-1])
        if dy2.dtype != torch.bfloat16:
            dy2 = dy2.to(torch.bfloat16)
        if not dy2.is_contiguous():
            dy2 = dy2.contiguous()
        if FUSED_GELU_BACKWARD and gemm.fits(dy2, w2b):
            dpre = gemm.linear_dx(dy2, w2b, gelu_pre=pre)
            db1 = column_sum(dpre)
        else:
            dpre, db1 = gelu_backward(torch.mm(dy2, w2b), pre)
        dw2 = gemm.linear_dw(dy2, h) if _dw_ok(dy2, h) else _mm_f32(dy2.t(), h)
        db2 = column_sum(dy2)
        dx = torch.mm(dpre, w1b).view(*dy.shape[:-1], w1b.shape[1])
        dw1 = gemm.linear_dw(dpre, x2) if _dw_ok(dpre, x2) else _mm_f32(dpre.t(), x2)
        return dx, dw1, db1, dw2, db2, None, None, None, None


def feed_forward(x, ff):
    """ff = nn.Sequential(Linear, GELU, Linear) applied to x in x's dtype."""
    l1, l2 = ff[0], ff[2]
    if x.dtype == l1.weight.dtype:
        return linear(F.gelu(linear(x, l1)), l2)
    if x.dtype != torch.bfloat16 or l1.weight.dtype != torch.float32:
        return l2(F.gelu(l1(x.to(l1.weight.dtype)))).to(x.dtype)  # parameters cast to another dtype
    if l1.bias is None or l2.bias is None:
        raise TypeError("the bf16 feed-forward needs both biases (reference mingru/minLM.py:17-23)")
    return BF16FeedForward.apply(x, l1.weight, l1.bias, l2.weight, l2.bias, bf16_copy(l1.weight),
                                 bf16_copy(l2.weight), bf16_copy(l1.bias), bf16_copy(l2.bias))
