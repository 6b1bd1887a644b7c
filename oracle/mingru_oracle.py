"""CPU oracle for the minGRU / minLM training hot path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only as the checker or as the timed CPU baseline.
The product (gruboros_amd) never calls it.

Two kinds of function live here:

* Restatements of the reference, op for op, in a caller-chosen dtype
  (float64 for the parity oracle, float32 for "the reference's own
  precision" and for the CPU baseline). Each cites the reference line it
  follows (paths relative to the reference tree).
* Independent evaluations of the same mathematics used to pin the
  restatements: a brute-force linear recurrence (float64 numpy), the
  textbook cumulative log-add-exp (numpy.logaddexp.accumulate), and the
  closed-form adjoint of the scan. The tests compare the restatements with
  these, so a dropped term, wrong sign or shifted index in either shows up.

Pins (see tests/test_oracle.py): g/log_g and the gate math against closed
forms and branch special cases; the scan against the linear recurrence,
logaddexp.accumulate and invariants (convexity bounds, constant input,
geometric closed form, chunked == unchunked, T one-step updates == scan);
the backward against torch.autograd.gradcheck and the closed form; RMSNorm
against torch.nn.functional.rms_norm; the loss against
torch.nn.functional.cross_entropy; the causal convolution against torch.nn.Conv1d. Parity of the seeded initialisation
order (mingru/minLM.py:157-206) is not pinned: tests share one state dict
between the oracle and the product instead.
"""
import math

import numpy as np
import torch
import torch.nn.functional as F

FP32_EPS = float(torch.finfo(torch.float32).eps)


# --------------------------------------------------------------------------- gate math

def g(x):
    """mingru/minGRU.py:24-25."""
    return torch.where(x >= 0, x + 0.5, x.sigmoid())


def log_g(x):
    """mingru/minGRU.py:27-28."""
    return torch.where(x >= 0, (F.relu(x) + 0.5).log(), -F.softplus(-x))


def heinsen_associative_scan_log(log_coeffs, log_values):
    """mingru/minGRU.py:16-20 (scan along dim 1)."""
    a_star = log_coeffs.cumsum(dim=1)
    log_h0_plus_b_star = (log_values - a_star).logcumsumexp(dim=1)
    log_h = a_star + log_h0_plus_b_star
    return log_h.exp()


def mingru_scan(hidden, gate, prev_hidden=None):
    """minGRU.forward after the projection, mingru/minGRU.py:43-69 (to_out excluded).

    hidden, gate: [B, T, Di]; prev_hidden: [B, 1, Di] or None.
    Returns (out [B, T, Di], next_prev_hidden [B, 1, Di]) in the inputs' dtype.
    """
    seq_len = hidden.shape[1]
    if seq_len == 1:                                           # :47-52
        hid = g(hidden)
        gt = gate.sigmoid()
        out = torch.lerp(prev_hidden, hid, gt) if prev_hidden is not None else hid * gt
    else:                                                      # :53-67
        log_coeffs = -F.softplus(gate)
        log_z = -F.softplus(-gate)
        log_tilde_h = log_g(hidden)
        log_values = log_z + log_tilde_h
        if prev_hidden is not None:
            log_values = torch.cat((prev_hidden.log(), log_values), dim=1)
            log_coeffs = F.pad(log_coeffs, (0, 0, 1, 0))
        out = heinsen_associative_scan_log(log_coeffs, log_values)
        out = out[:, -seq_len:]
    next_prev_hidden = out[:, -1:]                             # :69
    return out, next_prev_hidden


# --------------------------------------------------------------------------- independent pins

def _np_sigmoid(x):
    return np.where(x >= 0, 1.0 / (1.0 + np.exp(-np.abs(x))), np.exp(-np.abs(x)) / (1.0 + np.exp(-np.abs(x))))


def np_g(x):
    """Closed form of g: x + 1/2 for x >= 0, logistic sigmoid for x < 0."""
    return np.where(x >= 0, x + 0.5, _np_sigmoid(x))


def np_g_prime(x):
    """d g / dx as autograd of the reference's log_g sees it (relu'(0) = 0)."""
    s = _np_sigmoid(x)
    return np.where(x > 0, 1.0, np.where(x == 0, 0.0, s * (1.0 - s)))


def linear_recurrence(hidden, gate, h0=None):
    """Brute-force float64 h_t = (1 - z_t) h_{t-1} + z_t g(hidden_t), z = sigmoid(gate).

    numpy arrays [B, T, Di]; h0 [B, Di] or None (zero state). Returns h [B, T, Di].
    """
    hidden = np.asarray(hidden, dtype=np.float64)
    gate = np.asarray(gate, dtype=np.float64)
    B, T, Di = hidden.shape
    z = _np_sigmoid(gate)
    a = _np_sigmoid(-gate)
    b = z * np_g(hidden)
    h = np.zeros((B, Di)) if h0 is None else np.asarray(h0, dtype=np.float64).reshape(B, Di).copy()
    out = np.empty((B, T, Di))
    for t in range(T):
        h = a[:, t] * h + b[:, t]
        out[:, t] = h
    return out


def logaddexp_scan(hidden, gate, h0=None):
    """Textbook evaluation of the same recurrence in log space with numpy's
    cumulative logaddexp: log h_t = A_t + logaddexp_{k<=t}(log b_k - A_k),
    A_t = sum_{k<=t} log a_k, with log h0 as an extra leading term."""
    hidden = np.asarray(hidden, dtype=np.float64)
    gate = np.asarray(gate, dtype=np.float64)
    la = -np.logaddexp(0.0, gate)                       # log(1 - sigmoid(gate))
    lb = -np.logaddexp(0.0, -gate) + np.log(np_g(hidden))
    if h0 is not None:
        B, _, Di = hidden.shape
        lh0 = np.log(np.asarray(h0, dtype=np.float64).reshape(B, 1, Di))
        la = np.concatenate([np.zeros_like(lh0), la], axis=1)
        lb = np.concatenate([lh0, lb], axis=1)
    A = np.cumsum(la, axis=1)
    lh = A + np.logaddexp.accumulate(lb - A, axis=1)
    h = np.exp(lh)
    return h[:, 1:] if h0 is not None else h


def scan_backward_closed_form(hidden, gate, h0, dh, dh_last=None):
    """Closed-form adjoint of the recurrence (float64 numpy):

      lambda_t = dh_t + a_{t+1} lambda_{t+1}
      dgate_t = lambda_t z_t (1 - z_t) (g(hidden_t) - h_{t-1})
      dhidden_t = lambda_t z_t g'(hidden_t)
      dh0 = a_0 lambda_0
    Returns (dhidden, dgate, dh0 [B, Di])."""
    hidden = np.asarray(hidden, dtype=np.float64)
    gate = np.asarray(gate, dtype=np.float64)
    dh = np.asarray(dh, dtype=np.float64).copy()
    B, T, Di = hidden.shape
    if dh_last is not None:
        dh[:, -1] += np.asarray(dh_last, dtype=np.float64).reshape(B, Di)
    h = linear_recurrence(hidden, gate, h0)
    hp = np.concatenate([(np.zeros((B, 1, Di)) if h0 is None else np.asarray(h0, np.float64).reshape(B, 1, Di)),
                         h[:, :-1]], axis=1)
    z = _np_sigmoid(gate)
    a = _np_sigmoid(-gate)
    lam = np.zeros((B, T, Di))
    nxt = np.zeros((B, Di))
    for t in range(T - 1, -1, -1):
        lam[:, t] = dh[:, t] + nxt
        nxt = a[:, t] * lam[:, t]
    dgate = lam * z * a * (np_g(hidden) - hp)
    dhidden = lam * z * np_g_prime(hidden)
    return dhidden, dgate, nxt


# --------------------------------------------------------------------------- minLM pieces

def rms_norm(x, weight, eps=FP32_EPS):
    """torch.nn.RMSNorm(dim) as used at mingru/minLM.py:67,69,74: y = x * rsqrt(mean(x^2) + eps) * w.
    eps is float32's machine epsilon whatever the activation dtype."""
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * weight


def feed_forward(x, w1, b1, w2, b2):
    """mingru/minLM.py:17-23: Linear -> exact (erf) GELU -> Linear."""
    return F.linear(F.gelu(F.linear(x, w1, b1)), w2, b2)


def cross_entropy_mean(logits, labels):
    """mingru/minLM.py:146-149: mean over positions of logsumexp(logits) - logits[label]."""
    lse = torch.logsumexp(logits, dim=-1)
    picked = torch.gather(logits, -1, labels.unsqueeze(-1)).squeeze(-1)
    return (lse - picked).mean()


class _RoundBF16(torch.autograd.Function):
    """Identity that rounds its value (forward) and its gradient (backward)
    to bfloat16 and back: marks where a bf16-activation implementation stores
    a tensor in bf16."""

    @staticmethod
    def forward(ctx, x):
        return x.to(torch.bfloat16).to(x.dtype)

    @staticmethod
    def backward(ctx, g):
        return g.to(torch.bfloat16).to(g.dtype)


class _RoundGradBF16(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x):
        return x.clone()

    @staticmethod
    def backward(ctx, g):
        return g.to(torch.bfloat16).to(g.dtype)


def causal_dwconv(x, w_dw, b_dw, w_pw, b_pw):
    """CausalDepthWiseConv1d of mingru/minLM.py:27-39 on x [B, T, D]: a depthwise
    convolution over time with kernel k = w_dw.shape[-1], left-padded with k - 1
    zeros (so output t sees inputs t - k + 1 .. t), then a pointwise (1 x 1)
    convolution across channels:
        y[b, t, d] = b_dw[d] + sum_j w_dw[d, 0, j] x[b, t + j - (k - 1), d]
        z[b, t, :] = W_pw y[b, t, :] + b_pw        (W_pw = w_pw[:, :, 0])."""
    k = w_dw.shape[-1]
    T = x.shape[1]
    y = b_dw.expand_as(x).clone()
    for j in range(k):
        shift = k - 1 - j                      # input t - shift
        if shift >= T:
            continue
        y[:, shift:, :] += w_dw[:, 0, j] * x[:, :T - shift, :]
    return y @ w_pw[:, :, 0].t() + b_pw


def minlm_core(p, ids, depth, prev_hiddens=None, expansion=1.0, bf16_points=False):
    """Body of mingru/minLM.py:97-138 (embedding -> blocks -> final norm -> logits),
    dropout disabled; a layer whose state holds the conv's keys
    (`layers.i.0.net.{0,1}.{weight,bias}`, enable_conv=True) adds
    causal_dwconv(x) to x first (:109-112). p: state dict already in the working dtype.
    Returns (logits, next_prev_hiddens).

    bf16_points=True evaluates the same mathematics (in p's dtype) with every
    tensor rounded to bf16 where the build's bf16-activation path (fp32
    residual stream, fp32 scan state, fp32 logits) stores it: the GEMM
    weights and biases, the normalized block inputs, the GEMM and GELU
    outputs, and the gradients of all of those and of the logits. Two
    products are fp32-accurate there and stay unrounded here: the hidden half
    of to_hidden_and_gate (its input n and weight rows) and to_out; the scan
    output enters the residual stream (or to_out) in fp32. Its gradient is
    rounded to bf16 on the way back, as the build's backward stores it."""
    r = _RoundBF16.apply if bf16_points else (lambda t: t)
    rg = _RoundGradBF16.apply if bf16_points else (lambda t: t)
    x = F.embedding(ids, p["token_emb.weight"])                            # :97
    hiddens = iter(prev_hiddens or [])
    nxt = []
    for i in range(depth):                                                 # :107-135
        pre = f"layers.{i}."
        prev = next(hiddens, None)
        if prev is not None:
            prev = prev.to(x.dtype)
        if pre + "0.net.0.weight" in p:                                    # :109-112 (conv)
            x = causal_dwconv(x, p[pre + "0.net.0.weight"], p[pre + "0.net.0.bias"], p[pre + "0.net.1.weight"],
                              p[pre + "0.net.1.bias"]) + x
        n = rg(rms_norm(x, p[pre + "1.weight"]))                           # :121
        w_hg = p[pre + "2.to_hidden_and_gate.weight"]
        di = w_hg.shape[0] // 2
        hidden = F.linear(n, w_hg[:di])                                    # minGRU.py:45, hidden half (accurate)
        gate = F.linear(r(n), r(w_hg[di:]))                                #   gate half (bf16 operands)
        hg = r(torch.cat([hidden, gate], dim=-1))
        hidden, gate = hg.chunk(2, dim=-1)
        out, h_next = mingru_scan(hidden, gate, prev)
        out = rg(out)
        if expansion != 1.0:
            out = rg(F.linear(out, p[pre + "2.to_out.weight"]))            # minGRU.py:71 (accurate)
        x = out + x                                                        # :125
        nxt.append(h_next)
        n2 = r(rms_norm(x, p[pre + "3.weight"]))
        f1 = r(F.linear(n2, r(p[pre + "4.0.weight"]), r(p[pre + "4.0.bias"])))
        f3 = r(F.linear(r(F.gelu(f1)), r(p[pre + "4.2.weight"]), r(p[pre + "4.2.bias"])))
        x = f3 + x                                                         # :130 (FeedForward :17-23)
    embed = r(rms_norm(x, p["norm.weight"]))                               # :137
    return rg(F.linear(embed, r(p["to_logits.weight"]))), nxt              # :138


def minlm_forward(params, ids, depth, return_loss=True, prev_hiddens=None, expansion=1.0, dtype=torch.float64,
                  bf16_points=False):
    """mingru/minLM.py:86-155 with dropout disabled (dropout=0); the conv is applied
    where the state holds its keys (enable_conv=True).

    params: state dict with the reference's key names (floating tensors are
    cast to `dtype`). Returns (loss or logits, next_prev_hiddens).
    """
    p = {k: (v.to(dtype) if v.is_floating_point() else v) for k, v in params.items()}
    if return_loss:
        ids, labels = ids[:, :-1], ids[:, 1:]                              # :94-95
    if prev_hiddens is not None and not return_loss:
        ids = ids[:, -1:]                                                  # :101-102 (per-token, so slicing ids == slicing x)
    logits, nxt = minlm_core(p, ids, depth, prev_hiddens, expansion, bf16_points)
    if not return_loss:
        return logits, nxt
    return cross_entropy_mean(logits, labels), nxt                         # :146-149


def make_minlm_state(num_tokens, dim, depth, ff_mult=4, expansion=1.0, seed=0, dtype=torch.float32,
                     conv_kernel_size=None):
    """A state dict with the reference's keys, order and shapes
    (mingru/minLM.py:58-75, minGRU.py:40-41), initialised as
    mingru/minLM.py:157-206 describes (distributionally; the RNG draw order of
    the reference is not reproduced)."""
    gen = torch.Generator().manual_seed(seed)
    std = 0.02 / math.sqrt(dim)
    di = int(dim * expansion)
    f = int(dim * ff_mult)
    sd = {"token_emb.weight": torch.randn(num_tokens, dim, generator=gen) * std}
    for i in range(depth):
        pre = f"layers.{i}."
        if conv_kernel_size:  # enable_conv=True (random values: the reference keeps nn.Conv1d's init)
            k = conv_kernel_size
            sd[pre + "0.net.0.weight"] = torch.randn(dim, 1, k, generator=gen) / math.sqrt(k)
            sd[pre + "0.net.0.bias"] = torch.randn(dim, generator=gen) * 0.1
            sd[pre + "0.net.1.weight"] = torch.randn(dim, dim, 1, generator=gen) / math.sqrt(dim)
            sd[pre + "0.net.1.bias"] = torch.randn(dim, generator=gen) * 0.1
        sd[pre + "1.weight"] = torch.ones(dim)
        sd[pre + "2.to_hidden_and_gate.weight"] = torch.randn(2 * di, dim, generator=gen) * std
        if expansion != 1.0:
            sd[pre + "2.to_out.weight"] = torch.zeros(dim, di)
        sd[pre + "3.weight"] = torch.ones(dim)
        sd[pre + "4.0.weight"] = torch.randn(f, dim, generator=gen) * std
        bound = 1.0 / math.sqrt(dim)
        sd[pre + "4.0.bias"] = (torch.rand(f, generator=gen) * 2 - 1) * bound
        sd[pre + "4.2.weight"] = torch.zeros(dim, f)
        sd[pre + "4.2.bias"] = torch.zeros(dim)
    sd["norm.weight"] = torch.ones(dim)
    sd["to_logits.weight"] = torch.randn(num_tokens, dim, generator=gen) * std
    return {k: v.to(dtype) for k, v in sd.items()}
