"""Pins the CPU oracle (oracle/mingru_oracle.py) to mathematics it must agree with.

Each check is chosen so that a plausible slip in the restatement (a dropped
term, a wrong sign, a shifted index, a transposed operand) fails it; the
last tests plant such slips in a copy of the oracle and confirm they are
caught.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import mingru_oracle as O


def _inputs(B, T, Di, seed=0, gate_std=1.0, hid_std=1.0):
    gen = torch.Generator().manual_seed(seed)
    hidden = torch.randn(B, T, Di, generator=gen, dtype=torch.float64) * hid_std
    gate = torch.randn(B, T, Di, generator=gen, dtype=torch.float64) * gate_std
    h0 = O.g(torch.randn(B, 1, Di, generator=gen, dtype=torch.float64))
    return hidden, gate, h0


# ----------------------------------------------------------------- gate math


def test_g_and_log_g_closed_forms():
    x = torch.tensor([-30.0, -20.5, -3.0, -1e-3, 0.0, 1e-3, 0.5, 3.0, 21.0, 40.0], dtype=torch.float64)
    expect = np.where(x.numpy() >= 0, x.numpy() + 0.5, 1.0 / (1.0 + np.exp(-x.numpy())))
    np.testing.assert_allclose(O.g(x).numpy(), expect, rtol=1e-15)
    # torch's softplus returns its input above 20 (threshold=20), so for
    # x < -20 log_g(x) = -softplus(-x) is exactly x
    log_expect = np.where(x.numpy() < -20, x.numpy(), np.log(expect))
    np.testing.assert_allclose(O.log_g(x).numpy(), log_expect, rtol=1e-13, atol=1e-15)
    # continuity of g at 0 from both branches
    assert float(O.g(torch.tensor(-1e-12, dtype=torch.float64))) == pytest.approx(0.5, abs=1e-12)


def test_log_g_gradient_at_zero_is_zero():
    # The reference's log_g uses relu(x)+0.5 on x >= 0, and relu'(0) = 0.
    x = torch.tensor([0.0, -0.0, 1.0, -1.0], dtype=torch.float64, requires_grad=True)
    O.log_g(x).sum().backward()
    s = torch.sigmoid(torch.tensor(-1.0, dtype=torch.float64))
    np.testing.assert_allclose(x.grad.numpy(), [0.0, 0.0, 1.0 / 1.5, 1.0 - float(s)], rtol=1e-12)


def test_gate_log_identities():
    gate = torch.linspace(-40, 40, 801, dtype=torch.float64)
    z = torch.sigmoid(gate)
    # log_coeffs = -softplus(gate) = log(1 - z); log_z = -softplus(-gate) = log z
    # (beyond |gate| = 20 torch's softplus threshold makes these exact only to
    # a relative exp(-20) ~ 2e-9)
    a = torch.sigmoid(-gate)  # 1 - z without cancellation
    np.testing.assert_allclose((-F.softplus(gate)).exp().numpy(), a.numpy(), rtol=3e-9, atol=0)
    np.testing.assert_allclose((-F.softplus(-gate)).exp().numpy(), z.numpy(), rtol=3e-9, atol=0)
    np.testing.assert_allclose((z + a).numpy(), 1.0, rtol=1e-15)


# ----------------------------------------------------------------- scan forward


@pytest.mark.parametrize("with_h0", [False, True])
@pytest.mark.parametrize("B,T,Di", [(2, 1, 8), (2, 2, 8), (3, 63, 16), (2, 257, 12)])
def test_scan_matches_linear_recurrence(B, T, Di, with_h0):
    hidden, gate, h0 = _inputs(B, T, Di, seed=T)
    out, nxt = O.mingru_scan(hidden, gate, h0 if with_h0 else None)
    ref = O.linear_recurrence(hidden.numpy(), gate.numpy(), h0.numpy() if with_h0 else None)
    np.testing.assert_allclose(out.numpy(), ref, rtol=1e-10)
    np.testing.assert_allclose(nxt.numpy(), ref[:, -1:], rtol=1e-10)


@pytest.mark.parametrize("with_h0", [False, True])
def test_scan_matches_logaddexp_accumulate(with_h0):
    hidden, gate, h0 = _inputs(2, 100, 8, seed=3, gate_std=3.0, hid_std=3.0)
    out, _ = O.mingru_scan(hidden, gate, h0 if with_h0 else None)
    ref = O.logaddexp_scan(hidden.numpy(), gate.numpy(), h0.numpy() if with_h0 else None)
    np.testing.assert_allclose(out.numpy(), ref, rtol=1e-10)


def test_linear_recurrence_known_values():
    # gate = 0 -> z = a = 1/2; hidden = 1 -> g = 1.5; h_t = 1.5 (1 - 2^-(t+1)) from h0 = 0
    T = 30
    hidden = np.ones((1, T, 1))
    gate = np.zeros((1, T, 1))
    h = O.linear_recurrence(hidden, gate)[0, :, 0]
    t = np.arange(T)
    np.testing.assert_allclose(h, 1.5 * (1 - 0.5 ** (t + 1)), rtol=1e-14)
    # with h0: h_t = 1.5 + (h0 - 1.5) 2^-(t+1)
    h = O.linear_recurrence(hidden, gate, np.full((1, 1), 4.0))[0, :, 0]
    np.testing.assert_allclose(h, 1.5 + 2.5 * 0.5 ** (t + 1), rtol=1e-14)


def test_scan_invariants():
    hidden, gate, h0 = _inputs(2, 200, 8, seed=5, gate_std=2.0, hid_std=2.0)
    out, _ = O.mingru_scan(hidden, gate, h0)
    gt = O.g(hidden)
    prev = torch.cat([h0, out[:, :-1]], dim=1)
    lo = torch.minimum(prev, gt) * (1 - 1e-12)
    hi = torch.maximum(prev, gt) * (1 + 1e-12)
    assert bool(((out >= lo) & (out <= hi)).all())
    assert bool((out > 0).all())
    # constant hidden c with h0 = g(c): the state never moves
    c = torch.full((1, 50, 4), -0.7, dtype=torch.float64)
    out_c, _ = O.mingru_scan(c, gate[:1, :50, :4], O.g(c[:, :1]))
    np.testing.assert_allclose(out_c.numpy(), O.g(c).numpy(), rtol=1e-12)


def test_scan_chunked_equals_full():
    hidden, gate, h0 = _inputs(2, 300, 8, seed=7)
    full, last = O.mingru_scan(hidden, gate, h0)
    a, la = O.mingru_scan(hidden[:, :123], gate[:, :123], h0)
    b, lb = O.mingru_scan(hidden[:, 123:], gate[:, 123:], la)
    np.testing.assert_allclose(torch.cat([a, b], 1).numpy(), full.numpy(), rtol=1e-11)
    np.testing.assert_allclose(lb.numpy(), last.numpy(), rtol=1e-11)


def test_scan_equals_repeated_single_steps():
    # T applications of the seq_len == 1 path (mingru/minGRU.py:47-52) == one scan
    hidden, gate, h0 = _inputs(2, 40, 8, seed=9)
    full, _ = O.mingru_scan(hidden, gate, h0)
    h = h0
    steps = []
    for t in range(40):
        h, _ = O.mingru_scan(hidden[:, t:t + 1], gate[:, t:t + 1], h)
        steps.append(h)
    np.testing.assert_allclose(torch.cat(steps, 1).numpy(), full.numpy(), rtol=1e-11)


# ----------------------------------------------------------------- scan backward


def test_scan_gradcheck():
    hidden, gate, h0 = _inputs(1, 9, 3, seed=11)
    hidden.requires_grad_(True)
    gate.requires_grad_(True)
    h0.requires_grad_(True)

    def f(hd, gt, hz):
        out, nxt = O.mingru_scan(hd, gt, hz)
        return out, nxt

    assert torch.autograd.gradcheck(f, (hidden, gate, h0), eps=1e-6, atol=1e-7, rtol=1e-5)


@pytest.mark.parametrize("with_h0", [False, True])
def test_closed_form_backward_matches_autograd(with_h0):
    hidden, gate, h0 = _inputs(2, 70, 6, seed=13, gate_std=2.0, hid_std=2.0)
    hidden[0, 3, 2] = 0.0  # exercise g'(0) = 0
    gen = torch.Generator().manual_seed(1)
    dh = torch.randn(2, 70, 6, generator=gen, dtype=torch.float64)
    dl = torch.randn(2, 1, 6, generator=gen, dtype=torch.float64)
    hd, gt, hz = (t.clone().requires_grad_(True) for t in (hidden, gate, h0))
    out, nxt = O.mingru_scan(hd, gt, hz if with_h0 else None)
    ((out * dh).sum() + (nxt * dl).sum()).backward()
    dhid, dgat, dh0 = O.scan_backward_closed_form(hidden.numpy(), gate.numpy(),
                                                   h0.numpy() if with_h0 else None, dh.numpy(), dl.numpy())
    np.testing.assert_allclose(hd.grad.numpy(), dhid, rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(gt.grad.numpy(), dgat, rtol=1e-9, atol=1e-12)
    if with_h0:
        np.testing.assert_allclose(hz.grad.numpy().reshape(2, 6), dh0, rtol=1e-9, atol=1e-12)


# ----------------------------------------------------------------- norm / loss / model


def test_rms_norm_matches_library():
    gen = torch.Generator().manual_seed(0)
    x = torch.randn(4, 7, 64, generator=gen) * 1e-3
    w = torch.randn(64, generator=gen)
    ref = F.rms_norm(x, (64,), w, eps=torch.finfo(torch.float32).eps)
    torch.testing.assert_close(O.rms_norm(x, w), ref, rtol=1e-5, atol=1e-6)
    # nn.RMSNorm(dim) with eps=None uses finfo(fp32).eps for fp32 input
    m = torch.nn.RMSNorm(64)
    with torch.no_grad():
        m.weight.copy_(w)
    torch.testing.assert_close(O.rms_norm(x, w), m(x), rtol=1e-5, atol=1e-6)


def test_cross_entropy_matches_library():
    gen = torch.Generator().manual_seed(0)
    logits = torch.randn(3, 11, 256, generator=gen, dtype=torch.float64) * 4
    labels = torch.randint(0, 256, (3, 11), generator=gen)
    ref = F.cross_entropy(logits.transpose(1, 2), labels)
    torch.testing.assert_close(O.cross_entropy_mean(logits, labels), ref, rtol=1e-12, atol=1e-12)


def test_minlm_state_layout():
    sd = O.make_minlm_state(256, 32, 2, ff_mult=4, expansion=1.0)
    keys = list(sd)
    assert keys[0] == "token_emb.weight" and keys[-2:] == ["norm.weight", "to_logits.weight"]
    assert keys[1:8] == ["layers.0.1.weight", "layers.0.2.to_hidden_and_gate.weight", "layers.0.3.weight",
                         "layers.0.4.0.weight", "layers.0.4.0.bias", "layers.0.4.2.weight", "layers.0.4.2.bias"]
    assert sd["layers.1.2.to_hidden_and_gate.weight"].shape == (64, 32)
    sd15 = O.make_minlm_state(256, 32, 1, expansion=1.5)
    assert sd15["layers.0.2.to_out.weight"].shape == (32, 48)


def test_minlm_forward_tbptt_continuity():
    # TBPTT (train.py:792-804): each chunk's forward sees chunk[:, :-1] with the
    # carried hiddens. That equals one forward over the concatenated pieces.
    sd = O.make_minlm_state(256, 16, 2, seed=1, dtype=torch.float64)
    gen = torch.Generator().manual_seed(2)
    for k in sd:
        if k.endswith("4.2.weight"):
            sd[k] = torch.randn(sd[k].shape, generator=gen, dtype=torch.float64) * 0.05
    ids = torch.randint(0, 256, (2, 3 * 9), generator=gen)
    chunks = ids.split(9, dim=1)
    h = None
    pieces = []
    for c in chunks:
        lg, h = O.minlm_core(sd, c[:, :-1], 2, prev_hiddens=h)
        pieces.append(lg)
    full, hf = O.minlm_core(sd, torch.cat([c[:, :-1] for c in chunks], 1), 2)
    torch.testing.assert_close(torch.cat(pieces, 1), full, rtol=1e-9, atol=1e-12)
    for a, b in zip(h, hf):
        torch.testing.assert_close(a, b, rtol=1e-9, atol=1e-12)
    # and the loss path is the mean CE of those logits against the shifted ids
    loss, _ = O.minlm_forward(sd, chunks[0], 2, return_loss=True)
    ref = F.cross_entropy(pieces[0].transpose(1, 2), chunks[0][:, 1:])
    torch.testing.assert_close(loss, ref, rtol=1e-12, atol=1e-12)


# ----------------------------------------------------------------- planted mistakes are caught


def test_planted_sign_error_is_caught():
    hidden, gate, h0 = _inputs(2, 50, 4, seed=17)
    ref = O.linear_recurrence(hidden.numpy(), gate.numpy(), h0.numpy())
    # the reference formula with one sign flipped: log_coeffs = -softplus(-gate)
    lc = F.pad(-F.softplus(-gate), (0, 0, 1, 0))
    lv = torch.cat((h0.log(), -F.softplus(-gate) + O.log_g(hidden)), 1)
    bad = O.heinsen_associative_scan_log(lc, lv)[:, -50:]
    assert not np.allclose(bad.numpy(), ref, rtol=1e-3)
    # a dropped term (log_z omitted from log_values)
    lv2 = torch.cat((h0.log(), O.log_g(hidden)), 1)
    bad2 = O.heinsen_associative_scan_log(F.pad(-F.softplus(gate), (0, 0, 1, 0)), lv2)[:, -50:]
    assert not np.allclose(bad2.numpy(), ref, rtol=1e-3)


def test_planted_index_shift_is_caught():
    hidden, gate, h0 = _inputs(2, 50, 4, seed=19)
    ref = O.linear_recurrence(hidden.numpy(), gate.numpy(), h0.numpy())
    # dropping the seed position from the wrong end (out[:, :T] instead of out[:, -T:])
    log_coeffs = -F.softplus(gate)
    log_values = -F.softplus(-gate) + O.log_g(hidden)
    lv = torch.cat((h0.log(), log_values), 1)
    lc = F.pad(log_coeffs, (0, 0, 1, 0))
    shifted = O.heinsen_associative_scan_log(lc, lv)[:, :50]
    assert not np.allclose(shifted.numpy(), ref, rtol=1e-3)
    # and a closed-form backward with h_t in place of h_{t-1} differs from autograd
    dh = torch.ones(2, 50, 4, dtype=torch.float64)
    _, dg, _ = O.scan_backward_closed_form(hidden.numpy(), gate.numpy(), h0.numpy(), dh.numpy())
    z = 1 / (1 + np.exp(-gate.numpy()))
    h = ref
    lam_guess = dg / (z * (1 - z) * (O.np_g(hidden.numpy()) - np.concatenate([h0.numpy(), h[:, :-1]], 1)))
    wrong = lam_guess * z * (1 - z) * (O.np_g(hidden.numpy()) - h)
    assert not np.allclose(wrong, dg, rtol=1e-3)


@pytest.mark.parametrize("T,k", [(9, 3), (9, 4), (2, 4), (1, 3)])
def test_causal_dwconv_matches_torch_conv1d(T, k):
    """The oracle's explicit-sum restatement of CausalDepthWiseConv1d
    (mingru/minLM.py:27-39) against the same module built from torch's
    nn.Conv1d (left zero padding, depthwise then pointwise), including
    sequences shorter than the kernel."""
    torch.manual_seed(T * 10 + k)
    B, D = 2, 6
    x = torch.randn(B, T, D, dtype=torch.float64)
    net = torch.nn.Sequential(torch.nn.Conv1d(D, D, kernel_size=k, groups=D),
                              torch.nn.Conv1d(D, D, kernel_size=1)).double()
    want = net(F.pad(x.transpose(1, 2), (k - 1, 0), value=0.0)).transpose(1, 2)
    got = O.causal_dwconv(x, net[0].weight, net[0].bias, net[1].weight, net[1].bias)
    torch.testing.assert_close(got, want, rtol=1e-12, atol=1e-12)
    # causal: output t does not depend on inputs after t
    x2 = x.clone()
    x2[:, T - 1, :] += 1.0
    got2 = O.causal_dwconv(x2, net[0].weight, net[0].bias, net[1].weight, net[1].bias)
    torch.testing.assert_close(got2[:, :T - 1], got[:, :T - 1], rtol=0, atol=0)
