"""Drop-in mirror of the reference's mingru/minGRU.py on MI355X kernels.

Same class name, constructor, parameter names/shapes and forward signature as
the reference (mingru/minGRU.py:33-76); the parallel and the single-step
paths both run through the fused gate-math + scan kernel
(libmingru_hip.so: mg_scan_fwd / mg_scan_bwd). g, log_g and
heinsen_associative_scan_log stay importable as in the reference
(:16-28).
"""
import torch
import torch.nn.functional as F
from torch.nn import Identity, Linear, Module

from ..linear import accurate_linear_f32, hidden_gate_projection
from ..linear import linear as _linear
from ..scan import gate_scan_packed


def exists(v):
    return v is not None


def default(v, d):
    return v if exists(v) else d


def heinsen_associative_scan_log(log_coeffs, log_values):
    """Reference mingru/minGRU.py:16-20, kept as an importable utility (eager torch).
    The module's own forward does not use it: its scan runs in the fused kernel."""
    a_star = log_coeffs.cumsum(dim=1)
    log_h0_plus_b_star = (log_values - a_star).logcumsumexp(dim=1)
    log_h = a_star + log_h0_plus_b_star
    return log_h.exp()


def g(x):
    """Reference mingru/minGRU.py:24-25."""
    return torch.where(x >= 0, x + 0.5, x.sigmoid())


def log_g(x):
    """Reference mingru/minGRU.py:27-28."""
    return torch.where(x >= 0, (F.relu(x) + 0.5).log(), -F.softplus(-x))


class minGRU(Module):
    """Reference mingru/minGRU.py:33-76.

    forward(x [B,T,D], prev_hidden [B,1,Di] | None, return_next_prev_hidden)
    -> out [B,T,D] (x's dtype) or (out, next_prev_hidden [B,1,Di]).

    next_prev_hidden is the fp32 scan state after the last step (the
    reference returns out[:, -1:], a view in out's dtype; with fp32
    activations the two are equal). prev_hidden must be >= 0 as in the
    reference, which takes its log.
    """

    def __init__(self, dim, expansion_factor=1., proj_out=None):
        super().__init__()
        dim_inner = int(dim * expansion_factor)
        proj_out = default(proj_out, expansion_factor != 1.)
        self.to_hidden_and_gate = Linear(dim, dim_inner * 2, bias=False)
        self.to_out = Linear(dim_inner, dim, bias=False) if proj_out else Identity()

    def forward(self, x, prev_hidden=None, return_next_prev_hidden=False):
        hg = _linear(x, self.to_hidden_and_gate)          # :45 (chunk is implicit: [hidden | gate])
        out, next_prev_hidden = gate_scan_packed(hg, prev_hidden)   # :47-69
        if isinstance(self.to_out, Linear):
            out = _linear(out, self.to_out)                # :71
        if not return_next_prev_hidden:
            return out
        return out, next_prev_hidden

    def block_forward(self, n, pair, prev_hidden=None):
        """The minLM block's call (reference mingru/minLM.py:121-123): returns
        (out, next_prev_hidden) with `out` in fp32 when the activations are
        bf16, so the residual stream receives the scan state unrounded.

        pair: the hi/lo buffer of the normalized input n (bf16 activations over
        fp32 master weights) or None. With it, the hidden half of the projection
        and to_out are fp32-accurate products (see gruboros_amd.linear)."""
        if pair is not None:
            hg = hidden_gate_projection(n, pair, self.to_hidden_and_gate)
        else:
            hg = _linear(n, self.to_hidden_and_gate)
        out_dtype = torch.float32 if hg.dtype == torch.bfloat16 else None
        out, next_prev_hidden = gate_scan_packed(hg, prev_hidden, out_dtype)
        if isinstance(self.to_out, Linear):
            if pair is not None:
                out = accurate_linear_f32(out, self.to_out)
            else:
                out = _linear(out.to(n.dtype), self.to_out)
        return out, next_prev_hidden


MinGRU = minGRU
