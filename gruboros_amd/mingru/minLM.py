"""Drop-in mirror of the reference's mingru/minLM.py on MI355X kernels.

Same constructor, module tree, parameter names/shapes/registration order,
initialisation and forward signature as the reference
(mingru/minLM.py:17-206), so state dicts, checkpoints, optimizer parameter
indices and the TBPTT caller (train.py:783-809) carry over unchanged.

Compute: parameters stay fp32 masters; activations run in `compute_dtype`
(default: the process default set by gruboros_amd.mingru.set_default_compute_dtype
or install_alias(compute_dtype=...), else the parameters' dtype; bfloat16 for
the MI355X training configuration) with the residual stream kept in fp32. The
minGRU scan runs in the fused HIP kernel. A model whose parameters were cast
to bfloat16 (reference generate.py:140-142) runs its activations in bf16; one
cast to float16 (generate.py:143-144) runs its products in float16 and the
kernels (norm, scan) in fp32.
"""
import math

import torch
import torch.nn.functional as F
from torch import nn
from torch.nn import Module, ModuleList, RMSNorm

from .. import blocks, decode
from .. import scan as scan_errors
from ..embed import embedding
from ..linear import feed_forward
from ..linear import linear as _linear
from ..loss import logits_cross_entropy
from ..norm import add_rms_norm, rms_norm, rms_norm_residual
from ..scan import _prep_h0
from . import _defaults
from .minGRU import minGRU


def exists(v):
    return v is not None


def default(v, d):
    return v if exists(v) else d


def FeedForward(dim, mult=4):
    """Reference mingru/minLM.py:17-23."""
    dim_inner = int(dim * mult)
    return nn.Sequential(
        nn.Linear(dim, dim_inner),
        nn.GELU(),
        nn.Linear(dim_inner, dim)
    )


class CausalDepthWiseConv1d(Module):
    """Reference mingru/minLM.py:27-39 (only built when enable_conv=True; eager torch)."""

    def __init__(self, dim, kernel_size):
        super().__init__()
        self.kernel_size = kernel_size
        self.net = nn.Sequential(
            nn.Conv1d(dim, dim, kernel_size=kernel_size, groups=dim),
            nn.Conv1d(dim, dim, kernel_size=1)
        )

    def forward(self, x):
        x = x.transpose(1, 2)
        x = F.pad(x, (self.kernel_size - 1, 0), value=0.)
        x = self.net(x)
        return x.transpose(1, 2)


def _ff(x, ff):
    return feed_forward(x, ff)


class minLM(Module):
    """Reference mingru/minLM.py:43-206.

    decode_kernels: one-token calls under no_grad (the generation loop) run on the decode
    kernels when they apply (gruboros_amd.decode.forward_one); False keeps them on the
    parallel path."""

    decode_kernels = True

    def __init__(
        self,
        *,
        num_tokens,
        dim,
        depth,
        ff_mult=4,
        expansion=1.5,
        conv_kernel_size=3,
        use_lstm=None,  # kept for backward compatibility, ignored (as in the reference)
        enable_conv=False,
        dropout=0.,
        compute_dtype=None,
    ):
        super().__init__()
        self.token_emb = nn.Embedding(num_tokens, dim)
        self.layers = ModuleList([])
        for _ in range(depth):
            self.layers.append(ModuleList([
                CausalDepthWiseConv1d(dim, conv_kernel_size) if enable_conv else None,
                RMSNorm(dim),
                minGRU(dim, expansion_factor=expansion),
                RMSNorm(dim),
                FeedForward(dim, mult=ff_mult),
                nn.Dropout(dropout) if dropout > 0. else None
            ]))
        self.norm = RMSNorm(dim)
        self.to_logits = nn.Linear(dim, num_tokens, bias=False)
        self.can_cache = not enable_conv
        self.dim = dim
        self.depth = depth
        self.compute_dtype = compute_dtype
        self._initialize_weights()

    def forward(self, x, return_loss=False, return_prev_hiddens=False, prev_hiddens=None):
        """Reference mingru/minLM.py:86-155."""
        if x.is_cuda:
            # a look-back error reported since the last step raises here; then
            # the workspaces are polled again (asynchronously, no host sync)
            scan_errors.surface_errors(x.device)
        if return_loss:
            x, labels = x[:, :-1], x[:, 1:]
        if exists(prev_hiddens) and not return_loss:
            x = x[:, -1:]  # single-step decoding (reference :101-102; per-token ops commute with the slice)
        if self.decode_kernels and not return_loss and x.is_cuda and x.shape[1] == 1 and \
                not torch.is_grad_enabled():
            # a one-token call of the generation loop (reference generate.py:199-203) runs on
            # the decode kernels (one captured HIP graph per batch size) where they apply
            out = decode.forward_one(self, x, prev_hiddens)
            if out is not None:
                return out if return_prev_hiddens else out[0]

        cd, accurate = self._dtypes()
        if accurate and blocks.supported(self):
            # bf16 training path: block-level autograd functions (gruboros_amd.blocks)
            xs, pending, next_prev_hiddens = self._trunk_blocks(x, prev_hiddens)
            if return_loss:
                loss = blocks.FinalNormCE.apply(xs, pending, self.norm.weight, self.to_logits.weight, labels)
                return (loss, next_prev_hiddens) if return_prev_hiddens else loss
            if pending is None:
                embed = rms_norm(xs, self.norm.weight, cd)
            else:
                _, embed, _ = add_rms_norm(xs, pending, self.norm.weight, cd)
            logits = _linear(embed, self.to_logits)
            return (logits, next_prev_hiddens) if return_prev_hiddens else logits

        embed, next_prev_hiddens = self._trunk(x, prev_hiddens)

        if not return_loss:
            logits = _linear(embed, self.to_logits)
            if not return_prev_hiddens:
                return logits
            return logits, next_prev_hiddens

        # reference: F.cross_entropy(to_logits(embed).transpose(1, 2), labels)
        loss = logits_cross_entropy(embed, self.to_logits, labels)

        if not return_prev_hiddens:
            return loss
        return loss, next_prev_hiddens

    def logits_and_hiddens(self, ids, prev_hiddens=None):
        """Logits for every position of `ids` and the next prev_hiddens
        (reference mingru/minLM.py:97-138, the body shared by all forward modes)."""
        cd, accurate = self._dtypes()
        if accurate and blocks.supported(self):
            xs, pending, hiddens = self._trunk_blocks(ids, prev_hiddens)
            _, embed, _ = add_rms_norm(xs, pending, self.norm.weight, cd)
            return _linear(embed, self.to_logits), hiddens
        embed, hiddens = self._trunk(ids, prev_hiddens)
        return _linear(embed, self.to_logits), hiddens

    def _dtypes(self):
        """(activation dtype of the kernels, whether the bf16 path over fp32 masters applies)."""
        param_dtype = self.token_emb.weight.dtype
        cd = default(self.compute_dtype, default(_defaults.COMPUTE_DTYPE, param_dtype))
        if param_dtype not in (torch.float32, torch.bfloat16):
            cd = torch.float32  # float16 parameters: products in float16 (linear.linear), kernels in fp32
        elif param_dtype == torch.bfloat16:
            cd = torch.bfloat16
        return cd, cd == torch.bfloat16 and param_dtype == torch.float32

    def _trunk_blocks(self, ids, prev_hiddens):
        """Embedding and the blocks (reference :97-135) as block-level autograd
        functions: returns (x, pending, next_prev_hiddens), x the fp32 residual
        stream and pending the last FeedForward output, not yet added."""
        x = embedding(ids, self.token_emb.weight).float()
        prev_hiddens = iter(default(prev_hiddens, []))
        next_prev_hiddens = []
        pending = None
        for _, norm, mingru, ff_norm, ff, _ in self.layers:
            B, T, _ = x.shape
            w_hg = mingru.to_hidden_and_gate.weight
            h0 = _prep_h0(next(prev_hiddens, None), B, w_hg.shape[0] // 2, x.device)
            w_to = mingru.to_out.weight if isinstance(mingru.to_out, nn.Linear) else None
            x, out, h_last = blocks.MinGRUBlock.apply(x, pending, norm.weight, w_hg, h0, w_to)
            next_prev_hiddens.append(h_last)
            x, pending = blocks.FFBlock.apply(x, out, ff_norm.weight, ff[0].weight, ff[0].bias, ff[2].weight,
                                              ff[2].bias)
        return x, pending, next_prev_hiddens

    def _trunk(self, ids, prev_hiddens):
        """Embedding, blocks and final norm (reference :97-137) op by op:
        (embed, next_prev_hiddens)."""
        x = embedding(ids, self.token_emb.weight)
        cd, accurate = self._dtypes()
        x = x.float()  # fp32 residual stream

        next_prev_hiddens = []
        prev_hiddens = iter(default(prev_hiddens, []))

        # Pre-norm blocks with each residual add fused into the norm that
        # follows it (reference :107-135): n is the normalized input of the
        # next branch, x the fp32 residual stream, pending the branch output
        # still to be added to x.
        n = None
        pending = None
        for conv, norm, mingru, ff_norm, ff, dropout in self.layers:
            if exists(conv):
                if pending is not None:
                    x, pending = x + pending.float(), None
                x = conv(x) + x
            if pending is None:
                x, n, pair = rms_norm_residual(x, norm.weight, cd, with_lo=accurate)
            else:
                x, n, pair = add_rms_norm(x, pending, norm.weight, cd, with_lo=accurate)

            prev_hidden = next(prev_hiddens, None)
            min_gru_out, next_prev_hidden = mingru.block_forward(n, pair, prev_hidden)
            next_prev_hiddens.append(next_prev_hidden)

            x, n2, _ = add_rms_norm(x, min_gru_out, ff_norm.weight, cd)
            pending = _ff(n2, ff)

            if exists(dropout):
                x, pending = dropout(x + pending.float()), None

        if pending is None:
            embed = rms_norm(x, self.norm.weight, cd)
        else:
            _, embed, _ = add_rms_norm(x, pending, self.norm.weight, cd)
        return embed, next_prev_hiddens

    def _initialize_weights(self):
        """Reference mingru/minLM.py:157-206: N(0, 0.02/sqrt(dim)) for the embedding,
        the logits head, every to_hidden_and_gate and every first FF linear;
        zeros for to_out and the second FF linear (weight and bias), so each
        block starts as the identity. FF[0].bias keeps nn.Linear's default.
        The normal draws happen in the reference's order, so a seeded
        construction reproduces its parameters."""
        std = 0.02 / math.sqrt(self.dim)

        def normal(t):
            nn.init.normal_(t, mean=0.0, std=std)

        normal(self.token_emb.weight)
        normal(self.to_logits.weight)
        for layer in self.layers:
            gru, ff = layer[2], layer[4]
            normal(gru.to_hidden_and_gate.weight)
            if isinstance(gru.to_out, nn.Linear):
                nn.init.zeros_(gru.to_out.weight)
            normal(ff[0].weight)
            nn.init.zeros_(ff[2].weight)
            nn.init.zeros_(ff[2].bias)
