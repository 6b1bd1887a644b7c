"""GPU parity of the loss head (mg_cross_entropy_fwd_bwd, reference
mingru/minLM.py:146-149), the fused Schedule-Free AdamW step
(mg_sf_adamw_step, checked against oracle/sf_adamw.py) and the bf16 linear
layers with cached weight copies.

Tolerances: fp32 1e-5 relative (loss, logits gradient); bf16 activations
2e-2; optimizer state fp32 1e-6 relative after several steps.
"""
import pytest
import torch
import torch.nn.functional as F

from oracle import sf_adamw as S

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-300))


@pytest.mark.parametrize("V", [256, 260, 64, 1000])
@pytest.mark.parametrize("scale", [1.0, 30.0])
def test_cross_entropy_fp32(V, scale):
    from gruboros_amd.loss import CrossEntropyFromLogits

    gen = torch.Generator().manual_seed(V)
    N = 777
    logits = torch.randn(N, V, generator=gen, dtype=torch.float64) * scale
    labels = torch.randint(0, V, (N,), generator=gen)
    labels[:3] = torch.tensor([0, V - 1, 0])
    lg = logits.float().to(DEV).requires_grad_(True)
    loss = CrossEntropyFromLogits.apply(lg, labels.to(DEV))
    (loss * 0.25).backward()
    lr = logits.clone().requires_grad_(True)
    ref = F.cross_entropy(lr, labels)
    (ref * 0.25).backward()
    assert abs(float(loss) - float(ref)) / float(ref) < 1e-5
    assert _rel(lg.grad, lr.grad) < 1e-5


def test_logits_cross_entropy_bf16_matches_reference_head():
    """embed bf16 [B, T, D] through to_logits + CE vs the fp64 reference head."""
    from gruboros_amd.loss import logits_cross_entropy

    torch.manual_seed(0)
    B, T, D, V = 4, 127, 256, 256
    head = torch.nn.Linear(D, V, bias=False).to(DEV)
    embed = torch.randn(B, T, D, device=DEV).to(torch.bfloat16).requires_grad_(True)
    labels = torch.randint(0, V, (B, T), device=DEV)
    loss = logits_cross_entropy(embed, head, labels)
    loss.backward()
    e64 = embed.detach().double().cpu().requires_grad_(True)
    w64 = head.weight.detach().double().cpu().requires_grad_(True)
    ref = F.cross_entropy(F.linear(e64, w64).transpose(1, 2), labels.cpu())
    ref.backward()
    assert abs(float(loss) - float(ref)) / float(ref) < 2e-2
    assert _rel(embed.grad, e64.grad) < 2e-2
    assert _rel(head.weight.grad, w64.grad) < 2e-2
    assert head.weight.grad.dtype == torch.float32


def test_cross_entropy_flags_bad_labels():
    from gruboros_amd import _lib

    L = _lib.lib()
    N, V = 16, 256
    logits = torch.randn(N, V, device=DEV)
    labels = torch.zeros(N, dtype=torch.int64, device=DEV)
    labels[5] = V + 3
    dl = torch.empty(N, V, device=DEV)
    part = torch.empty(L.mg_cross_entropy_partials(N), device=DEV)
    bad = torch.zeros(1, dtype=torch.int32, device=DEV)
    rc = L.mg_cross_entropy_fwd_bwd(0, _lib.ptr(logits), _lib.ptr(labels), 0, _lib.ptr(dl), _lib.ptr(part),
                                    _lib.ptr(bad), N, V, 1.0 / N, _lib.stream_of(logits))
    assert rc == 0
    torch.cuda.synchronize()
    assert int(bad) == 1


def test_sf_step_keeps_the_hi_lo_pair_current():
    """For a weight with a hi/lo pair (the fp32-accurate products' operand),
    the fused step writes the pair of the updated weight itself: bit for bit
    what mg_split_hilo makes from the new fp32 master, its hi half is the bf16
    copy the other products read, and a dense bf16 copy (the decoder's) is
    re-made from the new master. Weights without a pair keep their dense copy
    updated in place."""
    from gruboros_amd.gemm import split_hilo
    from gruboros_amd.linear import bf16_copy, bf16_pair
    from gruboros_amd.optim import AdamWScheduleFree

    g = torch.Generator(device=DEV).manual_seed(11)
    w = torch.nn.Parameter(torch.randn(256, 128, device=DEV, generator=g) * 0.05)
    v = torch.nn.Parameter(torch.randn(64, 96, device=DEV, generator=g) * 0.05)
    opt = AdamWScheduleFree([w, v], lr=1e-2, weight_decay=0.01)
    opt.train()
    pair0 = bf16_pair(w)
    dense0 = bf16_copy(w, dense=True)
    vb0 = bf16_copy(v)
    for _ in range(3):
        w.grad = torch.randn(w.shape, device=DEV, generator=g)
        v.grad = torch.randn(v.shape, device=DEV, generator=g)
        opt.step()
    torch.cuda.synchronize()
    pair = bf16_pair(w)
    assert pair is pair0  # the cached pair, rewritten in place by the step
    assert torch.equal(pair.view(torch.int16), split_hilo(w.detach()).view(torch.int16))
    assert torch.equal(bf16_copy(w).float(), w.detach().bfloat16().float())
    dense = bf16_copy(w, dense=True)
    assert dense is not dense0 and dense.is_contiguous()
    assert torch.equal(dense, w.detach().bfloat16())
    assert bf16_copy(v) is vb0 and torch.equal(vb0, v.detach().bfloat16())


@pytest.mark.parametrize("form", ["denominator", "lr"])
@pytest.mark.parametrize("wd", [0.0, 0.01])
def test_sf_adamw_fused_matches_restatement(wd, form):
    """Both scalar schedules: the package's ("denominator") and Algorithm 1 of
    the paper ("lr"; the restatement of that form is pinned to Algorithm 1 by
    tests/test_oracle_sf.py)."""
    from gruboros_amd.optim import AdamWScheduleFree

    torch.manual_seed(1)
    shapes = [(1000, 33), (257,), (4, 4), (8192, 3), (7,)]
    ps = [torch.nn.Parameter(torch.randn(s, device=DEV)) for s in shapes]
    ref_ps = [p.detach().double().cpu().clone() for p in ps]
    opt = AdamWScheduleFree(ps, lr=1e-2, betas=(0.9, 0.999), weight_decay=wd, warmup_steps=2, bias_correction=form)
    opt.train()
    ref = S.RefAdamWScheduleFree(ref_ps, lr=1e-2, betas=(0.9, 0.999), weight_decay=wd, warmup_steps=2, form=form)
    for step in range(5):
        grads = [torch.randn(s, device=DEV) for s in shapes]
        for p, g in zip(ps, grads):
            p.grad = g
        opt.step()
        ref.step([g.double().cpu() for g in grads])
    for i, p in enumerate(ps):
        st = opt.state[p]
        assert _rel(p, ref.params[i]) < 1e-6
        assert _rel(st["z"], ref.z[i]) < 1e-6
        assert _rel(st["exp_avg_sq"], ref.v[i]) < 1e-6
    # eval()/train() mode switches of the package: x = (y - (1 - b1) z) / b1 and back
    y = ps[0].detach().clone()
    opt.eval()
    torch.testing.assert_close(ps[0], (y - 0.1 * opt.state[ps[0]]["z"]) / 0.9, rtol=1e-5, atol=1e-6)
    opt.train()
    torch.testing.assert_close(ps[0], y, rtol=1e-5, atol=1e-6)


def test_sf_adamw_table_is_resent_only_when_it_changes():
    """The tensor table goes to the device only when its rows change: gradients
    written in place keep it, gradients at new addresses send a new one; every
    step matches the restatement either way."""
    from gruboros_amd.optim import AdamWScheduleFree

    torch.manual_seed(3)
    shapes = [(300, 17), (65,)]
    ps = [torch.nn.Parameter(torch.randn(s, device=DEV)) for s in shapes]
    ref = S.RefAdamWScheduleFree([p.detach().double().cpu().clone() for p in ps], lr=1e-2, betas=(0.9, 0.999),
                                 weight_decay=0.01, warmup_steps=0)
    opt = AdamWScheduleFree(ps, lr=1e-2, betas=(0.9, 0.999), weight_decay=0.01)
    opt.train()
    grads = [torch.empty(s, device=DEV) for s in shapes]
    held = []
    sent = []
    for step in range(5):
        if step == 3:  # new gradient tensors while the old ones stay alive: new addresses
            held.append(grads)
            grads = [torch.empty(s, device=DEV) for s in shapes]
        for g in grads:
            g.normal_()
        for p, g in zip(ps, grads):
            p.grad = g
        opt.step()
        ref.step([g.double().cpu() for g in grads])
        sent.append(next(iter(opt._tables.values())).sent)
        for i, p in enumerate(ps):
            assert _rel(p, ref.params[i]) < 1e-6, (step, i)
            assert _rel(opt.state[p]["z"], ref.z[i]) < 1e-6, (step, i)
    assert sent[1] is sent[0] and sent[2] is sent[0]  # same rows: not sent again
    assert sent[3] is not sent[2] and sent[3] != sent[2]  # new gradient addresses: sent
    assert sent[4] is sent[3]


def test_bf16_weight_copy_follows_the_master():
    from gruboros_amd.linear import bf16_copy, linear
    from gruboros_amd.optim import AdamWScheduleFree

    torch.manual_seed(2)
    layer = torch.nn.Linear(64, 32).to(DEV)
    x = torch.randn(5, 64, device=DEV).to(torch.bfloat16)
    wb = bf16_copy(layer.weight)
    torch.testing.assert_close(wb, layer.weight.detach().to(torch.bfloat16))
    # in-place change by the caller (e.g. gossip blend) -> copy re-made
    with torch.no_grad():
        layer.weight.mul_(0.5).add_(1.0)
    torch.testing.assert_close(bf16_copy(layer.weight), layer.weight.detach().to(torch.bfloat16))
    # optimizer step writes master and copy together
    opt = AdamWScheduleFree(layer.parameters(), lr=1e-2)
    opt.train()
    y = linear(x, layer)
    y.float().square().sum().backward()
    assert layer.weight.grad.dtype == torch.float32 and layer.bias.grad.dtype == torch.float32
    opt.step()
    torch.testing.assert_close(bf16_copy(layer.weight), layer.weight.detach().to(torch.bfloat16))
    # gradients of the bf16 linear vs fp64
    x64 = x.double().cpu().requires_grad_(True)
    w64 = layer.weight.detach().double().cpu().requires_grad_(True)
    b64 = layer.bias.detach().double().cpu().requires_grad_(True)
    layer.zero_grad()
    xg = x.clone().requires_grad_(True)
    out = linear(xg, layer)
    dy = torch.randn(out.shape, device=DEV)
    (out.float() * dy).sum().backward()
    (F.linear(x64, w64, b64) * dy.double().cpu()).sum().backward()
    assert _rel(xg.grad, x64.grad) < 2e-2
    assert _rel(layer.weight.grad, w64.grad) < 2e-2
    assert _rel(layer.bias.grad, b64.grad) < 2e-2


@pytest.mark.parametrize("N,D,V", [(777, 256, 256), (64, 128, 64), (1000, 1024, 256), (130, 64, 200)])
def test_streaming_loss_head_matches_fp64(N, D, V):
    """mg_logits_cross_entropy (logits product + CE + gradient, no logits in memory)
    vs the fp64 reference head F.cross_entropy(F.linear(e, W)), incl. partial row blocks."""
    from gruboros_amd import _lib

    gen = torch.Generator().manual_seed(N + V)
    e = (torch.randn(N, D, generator=gen, dtype=torch.float64)).to(torch.bfloat16)
    w = (torch.randn(V, D, generator=gen, dtype=torch.float64) * 0.1).to(torch.bfloat16)
    lab = torch.randint(0, V, (N,), generator=gen)
    lab[:2] = torch.tensor([0, V - 1])
    L = _lib.lib()
    dl = torch.full((N, V + 8), 3.0, device=DEV, dtype=torch.bfloat16)
    part = torch.empty(L.mg_logits_cross_entropy_partials(N), device=DEV)
    bad = torch.zeros(1, dtype=torch.int32, device=DEV)
    ed, wd, ld = e.to(DEV), w.to(DEV), lab.to(DEV)
    rc = L.mg_logits_cross_entropy(_lib.ptr(ed), D, _lib.ptr(wd), D, _lib.ptr(ld), _lib.ptr(dl), V + 8, _lib.ptr(part),
                                   _lib.ptr(bad), N, D, V, 1.0 / N, _lib.stream_of(ed))
    assert rc == 0
    torch.cuda.synchronize()
    logits = (e.double() @ w.double().t()).requires_grad_(True)
    ref = F.cross_entropy(logits, lab)
    ref.backward()
    assert abs(float(part.sum()) / N - float(ref)) / float(ref) < 1e-5
    assert _rel(dl[:, :V].float(), logits.grad) < 4e-3
    assert bool((dl[:, V:] == 3.0).all())  # padding columns untouched
    assert int(bad) == 0


@pytest.mark.parametrize("N,C", [(1, 8), (777, 1024), (16376, 4096), (300, 264)])
def test_column_sum_and_gelu_backward(N, C):
    """mg_column_sum and mg_gelu_bwd vs fp64 torch (column sums; GELU's exact backward)."""
    from gruboros_amd.linear import column_sum, gelu_backward

    g = torch.Generator(device=DEV).manual_seed(N + C)
    x = torch.randn(N, C, device=DEV, generator=g).to(torch.bfloat16)
    pre = (torch.randn(N, C, device=DEV, generator=g) * 2).to(torch.bfloat16)
    s = column_sum(x)
    ref = x.double().sum(0)
    assert (s.double() - ref).abs().max() <= 1e-5 * (x.double().abs().sum(0).max() + 1)
    xf = x.float()
    assert _rel(column_sum(xf), ref) < 1e-6
    dpre, db = gelu_backward(x, pre)
    p64 = pre.double().cpu().requires_grad_(True)
    F.gelu(p64).backward(x.double().cpu())
    assert _rel(dpre, p64.grad) < 4e-3
    # the bias gradient sums the rounded dpre values
    assert (db.double() - dpre.double().sum(0)).abs().max() <= 1e-5 * (dpre.double().abs().sum(0).max() + 1)


@pytest.mark.parametrize("N,C1,C2", [(16376, 4096, 1024), (37, 264, 16), (777, 1536, 1024), (5, 8, 2056)])
@pytest.mark.parametrize("dh_dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
def test_feed_forward_bias_grads_in_one_launch(N, C1, C2, dh_dtype):
    """mg_ff_bias_bwd (the FeedForward backward's GELU backward and both bias gradients,
    reference mingru/minLM.py:17-23) equals mg_gelu_bwd + mg_column_sum bit for bit: the same
    per-element stochastic rounding, partial rows and reduction order. (16376, 4096, 1024) is
    the cfg3 layer."""
    from gruboros_amd.linear import column_sum, gelu_backward, gelu_backward_bias_grads

    g = torch.Generator(device=DEV).manual_seed(N + C1 + C2)
    dh = torch.randn(N, C1, device=DEV, generator=g).to(dh_dtype)
    pre = (torch.randn(N, C1, device=DEV, generator=g) * 2).to(torch.bfloat16)
    dy = torch.randn(N, C2, device=DEV, generator=g).to(torch.bfloat16)
    dpre, db1, db2 = gelu_backward_bias_grads(dh, pre, dy)
    dpre_r, db1_r = gelu_backward(dh, pre)
    db2_r = column_sum(dy)
    assert torch.equal(dpre, dpre_r) and torch.equal(db1, db1_r) and torch.equal(db2, db2_r)


def test_gradient_rounding_is_stochastic_and_deterministic():
    """bf16 gradient stores round stochastically (as mg_gelu_bwd's dpre does):
    4 M equal fp32 values 0.3 ulp above a bf16 value round up in 30% of the
    elements (round-to-nearest would round all of them down), so the mean
    keeps the fp32 value; the result is a function of the inputs (a second
    call gives the same bits); values that are bf16 already stay exact."""
    from gruboros_amd.linear import gelu_backward

    N, C = 4096, 1024
    v = 1.0 + 0.3 * 2.0 ** -7  # bf16 spacing at 1.0 is 2^-7
    dh = torch.full((N, C), v, device=DEV)
    pre = torch.full((N, C), 8.0, device=DEV, dtype=torch.bfloat16)  # gelu'(8) = 1 in fp32
    dpre, _ = gelu_backward(dh, pre, want_bias_grad=False)
    vals = dpre.float()
    assert set(vals.unique().tolist()) == {1.0, 1.0 + 2.0 ** -7}
    frac_up = float((vals > 1.0).float().mean())
    assert abs(frac_up - 0.3) < 0.005, frac_up
    assert abs(float(vals.double().mean()) - v) < 1e-5
    again, _ = gelu_backward(dh, pre, want_bias_grad=False)
    assert torch.equal(again, dpre)
    exact, _ = gelu_backward(torch.full((N, C), 1.0 + 2.0 ** -7, device=DEV), pre, want_bias_grad=False)
    assert bool((exact.float() == 1.0 + 2.0 ** -7).all())
