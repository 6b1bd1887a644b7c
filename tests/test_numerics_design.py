"""CPU checks behind the bf16 path's choice of rounding points (fp64 oracle
pieces only; no GPU).

The hidden half of to_hidden_and_gate (reference mingru/minGRU.py:45, then g
of :24-25) is an fp32-accurate hi/lo product in the bf16 build. The check
below measures, for one minGRU layer at the cfg3 width, what each cheaper
form would cost the to_hidden_and_gate weight gradient against plain fp64
with every other point left exact: rounding either operand of the hidden
half to bf16 moves pre-activations across g's kink at 0 (slope 1/4 below, 1
above) and alone uses the whole 2e-2 gradient contract, while the hi/lo form
stays far inside it.
"""
import pytest
import torch
import torch.nn.functional as F

from oracle import mingru_oracle as O

_BF = torch.bfloat16


def _bf(t):
    return t.to(_BF).to(t.dtype)


def _hidden(n, wh, form):
    if form == "fp64":
        return F.linear(n, wh)
    if form == "hilo":  # the build's three products of bf16 parts: hi.hi + lo.hi + hi.lo
        nh, whh = _bf(n), _bf(wh)
        nl, wl = _bf(n - nh), _bf(wh - whh)
        return F.linear(nh, whh) + F.linear(nl, whh) + F.linear(nh, wl)
    if form == "x_bf16":
        return F.linear(_bf(n), wh)
    if form == "w_bf16":
        return F.linear(n, _bf(wh))
    return F.linear(_bf(n), _bf(wh))


def _hg_weight_grad(state, ids, form):
    p = {k: v.to(torch.float64).requires_grad_(True) for k, v in state.items() if v.is_floating_point()}
    inp, lab = ids[:, :-1], ids[:, 1:]
    x = F.embedding(inp, p["token_emb.weight"])
    n = O.rms_norm(x, p["layers.0.1.weight"])
    w = p["layers.0.2.to_hidden_and_gate.weight"]
    di = w.shape[0] // 2
    out, _ = O.mingru_scan(_hidden(n, w[:di], form), F.linear(n, w[di:]), None)
    x = out + x
    x = O.feed_forward(O.rms_norm(x, p["layers.0.3.weight"]), p["layers.0.4.0.weight"], p["layers.0.4.0.bias"],
                       p["layers.0.4.2.weight"], p["layers.0.4.2.bias"]) + x
    logits = F.linear(O.rms_norm(x, p["norm.weight"]), p["to_logits.weight"])
    O.cross_entropy_mean(logits, lab).backward()
    return w.grad


@pytest.mark.parametrize("seed", [0, 1])
def test_hidden_half_needs_an_fp32_accurate_product(seed):
    state = O.make_minlm_state(256, 1024, 1, seed=seed)
    ids = torch.randint(0, 256, (2, 1025), generator=torch.Generator().manual_seed(seed + 7))
    ref = _hg_weight_grad(state, ids, "fp64")
    err = {f: float((_hg_weight_grad(state, ids, f) - ref).norm() / ref.norm())
           for f in ("hilo", "x_bf16", "w_bf16", "bf16")}
    assert err["hilo"] < 1e-3, err
    for f in ("x_bf16", "w_bf16", "bf16"):
        assert err[f] > 1.5e-2, err  # (measured 2.0-2.8e-2, seeds 0-2)
