"""GPU parity of the fused gate-math + scan kernels (mg_scan_fwd / mg_scan_bwd)
against the CPU oracle's float64 restatement of the reference
(mingru/minGRU.py:16-20, :24-28, :43-69) and its autograd gradients.

Tolerances (written here, from the build's parity contract): fp32 inputs ->
1e-4 relative (elementwise for h, which is > 0; norm-relative for gradients,
which cross zero); bf16 inputs/outputs with fp32 state -> 2e-2 relative.
"""
import numpy as np
import pytest
import torch

from oracle import mingru_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"
TOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2}


def _make(B, T, Di, dtype, with_h0, seed, scale=1.0, specials=False):
    gen = torch.Generator().manual_seed(seed)
    hidden = torch.randn(B, T, Di, generator=gen) * scale
    gate = torch.randn(B, T, Di, generator=gen) * scale
    if specials:
        flat_h, flat_g = hidden.view(-1), gate.view(-1)
        n = flat_h.numel()
        idx = torch.randperm(n, generator=gen)[: max(1, n // 8)]
        flat_h[idx[0::4]] = 0.0                       # g'(0) = 0 branch
        flat_g[idx[1::4]] = 100.0                     # a underflows to ~0
        flat_g[idx[2::4]] = -100.0                    # z underflows to ~0
        flat_h[idx[3::4]] = -60.0                     # g ~ 1e-26
    h0 = O.g(torch.randn(B, 1, Di, generator=gen)) if with_h0 else None
    dh = torch.randn(B, T, Di, generator=gen)
    dlast = torch.randn(B, 1, Di, generator=gen)
    hidden, gate, dh = hidden.to(dtype), gate.to(dtype), dh.to(dtype)
    return hidden, gate, h0, dh, dlast


def _oracle(hidden, gate, h0, dh, dlast):
    hd = hidden.double().requires_grad_(True)
    gt = gate.double().requires_grad_(True)
    hz = h0.double().requires_grad_(True) if h0 is not None else None
    out, nxt = O.mingru_scan(hd, gt, hz)
    ((out * dh.double()).sum() + (nxt * dlast.double()).sum()).backward()
    return out.detach(), nxt.detach(), hd.grad, gt.grad, (hz.grad if hz is not None else None)


def _rel_elem(x, ref):
    return float(((x.double() - ref).abs() / ref.abs().clamp_min(1e-30)).max())


def _rel_norm(x, ref):
    ref = ref.double()
    return float((x.double() - ref).norm() / ref.norm().clamp_min(1e-300))


def _run(hidden, gate, h0, dh, dlast, packed):
    from gruboros_amd.scan import gate_scan, gate_scan_packed

    hd = hidden.to(DEV).requires_grad_(True)
    gt = gate.to(DEV).requires_grad_(True)
    hz = h0.to(DEV).requires_grad_(True) if h0 is not None else None
    if packed:
        hg = torch.cat([hd, gt], -1).detach().requires_grad_(True)
        out, nxt = gate_scan_packed(hg, hz)
    else:
        out, nxt = gate_scan(hd, gt, hz)
    assert out.dtype == hidden.dtype and nxt.dtype == torch.float32
    assert out.shape == hidden.shape and nxt.shape == (hidden.shape[0], 1, hidden.shape[2])
    ((out.float() * dh.to(DEV).float()).sum() + (nxt * dlast.to(DEV)).sum()).backward()
    torch.cuda.synchronize()
    if packed:
        Di = hidden.shape[-1]
        dhid, dgat = hg.grad[..., :Di], hg.grad[..., Di:]
    else:
        dhid, dgat = hd.grad, gt.grad
    return (out.detach().float().cpu(), nxt.detach().cpu(), dhid.float().cpu(), dgat.float().cpu(),
            (hz.grad.cpu() if hz is not None else None))


def _check(res, ref, dtype, label):
    out, nxt, dhid, dgat, dh0 = res
    r_out, r_nxt, r_dhid, r_dgat, r_dh0 = ref
    tol = TOL[dtype]
    errs = {
        "h": _rel_elem(out, r_out),
        "h_last": _rel_elem(nxt, r_nxt),
        "dhidden": _rel_norm(dhid, r_dhid),
        "dgate": _rel_norm(dgat, r_dgat),
    }
    if r_dh0 is not None:
        errs["dh0"] = _rel_norm(dh0, r_dh0)
    print(label, {k: f"{v:.2e}" for k, v in errs.items()}, flush=True)
    for k, v in errs.items():
        assert v <= tol, f"{label}: {k} relative error {v:.3e} > {tol}"


SHAPES = [
    (1, 1, 4, True), (2, 1, 64, False), (2, 2, 8, True), (3, 63, 68, True), (2, 127, 64, False),
    (2, 128, 64, True), (2, 129, 64, False), (2, 257, 200, True), (1, 1000, 4, False), (2, 515, 132, True),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("B,T,Di,with_h0", SHAPES)
def test_scan_parity_shapes(B, T, Di, with_h0, dtype):
    args = _make(B, T, Di, dtype, with_h0, seed=B * 1000 + T + Di)
    ref = _oracle(*args)
    _check(_run(*args, packed=False), ref, dtype, f"{B}x{T}x{Di} h0={with_h0} {dtype}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_scan_parity_packed_projection_layout(dtype):
    args = _make(2, 300, 96, dtype, True, seed=5)
    ref = _oracle(*args)
    _check(_run(*args, packed=True), ref, dtype, f"packed {dtype}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_scan_parity_extremes(dtype):
    # large pre-activations, exact zeros, saturated gates: exercises the
    # softplus threshold region and underflow of a, z and g
    args = _make(2, 400, 64, dtype, True, seed=11, scale=12.0, specials=True)
    ref = _oracle(*args)
    _check(_run(*args, packed=False), ref, dtype, f"extremes {dtype}")


def test_scan_cfg1_fp32_three_way():
    """cfg1 shape (B4 T1024 Di512, fp32, no prev_hidden): kernel vs fp64 oracle,
    reference-formulation fp32 vs fp64, kernel vs reference fp32."""
    args = _make(4, 1024, 512, torch.float32, False, seed=0)
    ref64 = _oracle(*args)
    res = _run(*args, packed=False)
    hidden, gate = args[0], args[1]
    out32, _ = O.mingru_scan(hidden, gate, None)
    e_k64 = _rel_elem(res[0], ref64[0])
    e_r64 = _rel_elem(out32, ref64[0])
    e_kr = _rel_elem(res[0], out32.double())
    print(f"cfg1 h: kernel-vs-fp64 {e_k64:.2e}  ref32-vs-fp64 {e_r64:.2e}  kernel-vs-ref32 {e_kr:.2e}", flush=True)
    _check(res, ref64, torch.float32, "cfg1")
    assert e_k64 <= e_r64 + 1e-6  # the linear-space kernel is at least as accurate as the reference formula


def test_scan_cfg2_full_size_bf16():
    """cfg2 (B16 T8192 Di2048, bf16 in/out, fp32 state, prev_hidden = g(N(0,1))).

    Every channel of the full-size run is checked through size-independent
    properties; a strided sample of 64 channels is checked against the
    float64 brute-force recurrence and closed-form adjoint."""
    from gruboros_amd.scan import gate_scan

    B, T, Di = 16, 8192, 2048
    gen = torch.Generator(device=DEV).manual_seed(0)
    hidden = torch.randn(B, T, Di, device=DEV, generator=gen).to(torch.bfloat16)
    gate = torch.randn(B, T, Di, device=DEV, generator=gen).to(torch.bfloat16)
    h0 = O.g(torch.randn(B, 1, Di, device=DEV, generator=gen))
    dh = torch.randn(B, T, Di, device=DEV, generator=gen).to(torch.bfloat16)
    hd, gt = hidden.clone().requires_grad_(True), gate.clone().requires_grad_(True)
    out, last = gate_scan(hd, gt, h0)
    out.backward(dh)
    out, last = out.detach(), last.detach()
    torch.cuda.synchronize()

    # properties over every channel: positivity, and chunked == full
    assert bool((out > 0).all()) and bool(torch.isfinite(hd.grad.float()).all())
    a, la = gate_scan(hidden[:, :3000], gate[:, :3000], h0)
    b, lb = gate_scan(hidden[:, 3000:], gate[:, 3000:], la)
    torch.testing.assert_close(lb, last, rtol=1e-5, atol=0)
    assert float((torch.cat([a, b], 1).float() - out.float()).abs().max() / out.float().abs().max()) < 1e-2

    # sampled channels vs float64 brute force
    sel = torch.arange(0, Di, Di // 64, device=DEV)
    hs, gs, ds = hidden[..., sel].double().cpu().numpy(), gate[..., sel].double().cpu().numpy(), \
        dh[..., sel].double().cpu().numpy()
    h0s = h0[..., sel].double().cpu().numpy()
    ref = O.linear_recurrence(hs, gs, h0s)
    e_h = float(np.max(np.abs(out[..., sel].double().cpu().numpy() - ref) / ref))
    dhid, dgat, _ = O.scan_backward_closed_form(hs, gs, h0s, ds)
    e_dh = float(np.linalg.norm(hd.grad[..., sel].double().cpu().numpy() - dhid) / np.linalg.norm(dhid))
    e_dg = float(np.linalg.norm(gt.grad[..., sel].double().cpu().numpy() - dgat) / np.linalg.norm(dgat))
    e_last = float(np.max(np.abs(last[..., sel].double().cpu().numpy() - ref[:, -1:]) / ref[:, -1:]))
    print(f"cfg2 sample: h {e_h:.2e} h_last {e_last:.2e} dhidden {e_dh:.2e} dgate {e_dg:.2e}", flush=True)
    assert e_h <= 2e-2 and e_dh <= 2e-2 and e_dg <= 2e-2 and e_last <= 1e-4


def test_workspace_reuse_across_calls():
    """The look-back workspace is cleared once and then reused call after
    call (the kernels alternate a parity bit instead of clearing it): a run of
    forward/backward calls on one cached workspace, with other shapes and
    length-1 steps in between, gives bit for bit the results of calls on a
    freshly initialised workspace, and stays within tolerance of fp64."""
    from gruboros_amd import scan as S

    S.release_workspaces()
    cases = [(3, 700, 132, torch.bfloat16, True, s) for s in range(5)]
    cases += [(2, 1, 64, torch.float32, True, 9), (3, 700, 132, torch.float32, False, 10), (1, 129, 8, torch.bfloat16,
                                                                                               True, 11)]
    cases += [(3, 700, 132, torch.bfloat16, False, s) for s in range(20, 23)]
    reused = [_run(*_make(B, T, Di, dt, h0, seed=s), packed=False) for B, T, Di, dt, h0, s in cases]
    for (B, T, Di, dt, h0, s), got in zip(cases, reused):
        S.release_workspaces()
        args = _make(B, T, Di, dt, h0, seed=s)
        fresh = _run(*args, packed=False)
        for x, y in zip(got, fresh):
            assert (x is None and y is None) or torch.equal(x, y), (B, T, Di, dt, s)
        _check(got, _oracle(*args), dt, f"reuse {B}x{T}x{Di} seed {s}")


def _capi_fwd(L, hd, gt, h, ws, B, T, Di, ckpt=None):
    from gruboros_amd import _lib

    P = _lib.ptr
    return L.mg_scan_fwd(1, P(hd), P(gt), T * Di, Di, None, 1, P(h), T * Di, Di, None, P(ckpt), B, T, Di, P(ws),
                         ws.numel(), _lib.stream_of(hd))


def _capi_bwd(L, hd, gt, h, dh, dhid, dgat, ws, B, T, Di):
    from gruboros_amd import _lib

    P = _lib.ptr
    return L.mg_scan_bwd(1, P(hd), P(gt), T * Di, Di, None, 1, P(h), T * Di, Di, None, P(dh), T * Di, Di, None,
                         P(dhid), P(dgat), T * Di, Di, None, B, T, Di, P(ws), ws.numel(), _lib.stream_of(hd))


def test_workspace_errors_end_the_kernel():
    """Misused look-back workspaces end the kernels with an error word, not a
    wait without end, and mg_scan_workspace_check reports them:
      * a workspace that was never initialised (its header is not there): every
        workgroup returns at once;
      * one initialised for another shape: the same;
      * one whose ticket counters were corrupted (set to 1, as overlapping calls
        on one workspace could leave them), so every chain waits on a word that
        is never published: run with a poll limit of 64 (set from the host) so
        every wait ends after 64 polls, in both directions.
    After mg_scan_workspace_init the same memory gives bit for bit the results
    of a fresh workspace."""
    from gruboros_amd import _lib

    L, P = _lib.lib(), _lib.ptr
    B, T, Di = 2, 1024, 128  # 8 forward / 16 backward tiles per chain, 4 chains
    hidden, gate, _, dh, _ = _make(B, T, Di, torch.bfloat16, False, seed=3)
    hd, gt, dhd = hidden.to(DEV), gate.to(DEV), dh.to(DEV)
    h = torch.empty_like(hd)
    dhid, dgat = torch.empty_like(hd), torch.empty_like(hd)
    need = L.mg_scan_workspace_bytes(B, T, Di)
    ws = torch.zeros(need + 65536, dtype=torch.uint8, device=DEV)
    st = _lib.stream_of(hd)
    ncb = B * Di // 64

    print("case: never initialised", flush=True)
    assert _capi_fwd(L, hd, gt, h, ws, B, T, Di) == 0
    assert L.mg_scan_workspace_check(P(ws), st) == 3 and b"never initialised" in L.mg_last_error()

    print("case: initialised for another shape", flush=True)
    assert L.mg_scan_workspace_init(P(ws), ws.numel(), B, T // 2, Di, st) == 0
    assert _capi_fwd(L, hd, gt, h, ws, B, T, Di) == 0
    assert _capi_bwd(L, hd, gt, h, dhd, dhid, dgat, ws, B, T, Di) == 0
    assert L.mg_scan_workspace_check(P(ws), st) == 3 and b"another shape" in L.mg_last_error()

    for direction in ("forward", "backward"):
        print(f"case: corrupted {direction} ticket counters, 64 polls", flush=True)
        assert L.mg_scan_workspace_init(P(ws), ws.numel(), B, T, Di, st) == 0
        assert L.mg_scan_workspace_set_max_polls(P(ws), 64, st) == 0
        if direction == "forward":
            ws[256:256 + 4 * ncb].view(torch.int32).fill_(1)
            assert _capi_fwd(L, hd, gt, h, ws, B, T, Di) == 0
        else:
            assert _capi_fwd(L, hd, gt, h, ws, B, T, Di) == 0
            ws[256 + 4 * ncb:256 + 8 * ncb].view(torch.int32).fill_(1)
            assert _capi_bwd(L, hd, gt, h, dhd, dhid, dgat, ws, B, T, Di) == 0
        assert L.mg_scan_workspace_check(P(ws), st) == _lib.MG_ERR_STALL
        assert b"gave up after 64 polls" in L.mg_last_error()

    print("case: re-initialised", flush=True)
    fresh = torch.zeros(need, dtype=torch.uint8, device=DEV)
    outs = []
    for w in (ws, fresh):
        assert L.mg_scan_workspace_init(P(w), w.numel(), B, T, Di, st) == 0
        ho, gh, gg = torch.empty_like(hd), torch.empty_like(hd), torch.empty_like(hd)
        assert _capi_fwd(L, hd, gt, ho, w, B, T, Di) == 0
        assert _capi_bwd(L, hd, gt, ho, dhd, gh, gg, w, B, T, Di) == 0
        assert L.mg_scan_workspace_check(P(w), st) == 0
        outs.append((ho, gh, gg))
    for a, b in zip(*outs):
        assert torch.equal(a, b)


def test_backward_output_strides():
    """mg_scan_bwd writes dhidden/dgate with their own strides: reading the
    packed projection output [B, T, 2 Di] and writing two dense [B, T, Di]
    gradients gives the values of the packed gradient buffer."""
    from gruboros_amd import scan as S

    B, T, Di = 3, 700, 132
    hidden, gate, h0, dh, dlast = _make(B, T, Di, torch.bfloat16, True, seed=21)
    hg = torch.cat([hidden, gate], -1).to(DEV)
    h0d, dhd, dl = h0.to(DEV), dh.to(DEV), dlast.to(DEV)
    hv, gv = hg[..., :Di], hg[..., Di:]
    h, _, ckpt = S._launch_fwd(hv, gv, h0d, torch.bfloat16, need_ckpt=True)
    packed = torch.empty_like(hg)
    S._launch_bwd(hv, gv, h0d, h, ckpt, dhd, dl, packed[..., :Di], packed[..., Di:], False)
    dhid, dgat = torch.empty(B, T, Di, dtype=torch.bfloat16, device=DEV), torch.empty(B, T, Di, dtype=torch.bfloat16,
                                                                                       device=DEV)
    S._launch_bwd(hv, gv, h0d, h, ckpt, dhd, dl, dhid, dgat, False)
    assert torch.equal(dhid, packed[..., :Di]) and torch.equal(dgat, packed[..., Di:])
    S.check_workspaces()


def test_fp32_output_from_bf16_inputs():
    """The minLM block scans bf16 projections into an fp32 hidden sequence
    (out_dtype=float32): fp32-accurate states, and gradients through the fp32
    output path (dh fp32), against the fp64 oracle on the same bf16 inputs."""
    from gruboros_amd.scan import gate_scan_packed

    B, T, Di = 2, 515, 132
    hidden, gate, h0, dh, dlast = _make(B, T, Di, torch.bfloat16, True, seed=33)
    hg = torch.cat([hidden, gate], -1).to(DEV).requires_grad_(True)
    out, nxt = gate_scan_packed(hg, h0.to(DEV), out_dtype=torch.float32)
    assert out.dtype == torch.float32
    ((out * dh.to(DEV).float()).sum() + (nxt * dlast.to(DEV)).sum()).backward()
    ref = _oracle(hidden, gate, h0, dh.float(), dlast)
    assert _rel_elem(out.detach().cpu(), ref[0]) <= 1e-5
    assert _rel_elem(nxt.detach().cpu(), ref[1]) <= 1e-5
    assert _rel_norm(hg.grad[..., :Di].float().cpu(), ref[2]) <= 1e-2
    assert _rel_norm(hg.grad[..., Di:].float().cpu(), ref[3]) <= 1e-2


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("B,T,Di,with_h0", [(2, 515, 132, True), (8, 2047, 1024, False), (1, 7, 64, False)])
def test_residual_scan_matches_scan_plus_add(B, T, Di, with_h0, dtype):
    """mg_scan_fwd_residual (the minLM block at expansion 1: x_out = res + h, h kept as fp32
    checkpoints) against mg_scan_fwd followed by the add: x_out bit for bit, h_last and the
    checkpoints equal; and the backward with h = NULL (states rebuilt from the checkpoints)
    against the backward reading h: dhidden, dgate and dh0 equal, then both against the fp64
    oracle (reference mingru/minGRU.py:16-20, :47-69). (8, 2047, 1024) is the cfg3 layer."""
    from gruboros_amd import scan as S

    hidden, gate, h0, dh, dlast = _make(B, T, Di, dtype, with_h0, seed=B * 31 + T)
    hg = torch.cat([hidden, gate], -1).to(DEV)
    hv, gv = hg[..., :Di], hg[..., Di:]
    h0d = h0.to(DEV) if h0 is not None else None
    res = torch.randn(B, T, Di, generator=torch.Generator().manual_seed(7)).to(DEV)
    x_out, h_last_r, ckpt_r = S._launch_fwd_residual(hv, gv, h0d, res)
    h, h_last, ckpt = S._launch_fwd(hv, gv, h0d, torch.float32, need_ckpt=False)
    assert torch.equal(x_out, res + h)
    assert torch.equal(h_last_r, h_last)
    if dtype == torch.bfloat16:  # the checkpoints the bf16-output path writes (slots T // 8 on are never written)
        _, _, ckpt_b = S._launch_fwd(hv, gv, h0d, torch.bfloat16, need_ckpt=True)
        n = (T // 8) * B * Di
        assert torch.equal(ckpt_r[:n], ckpt_b[:n])
    dhd = dh.to(DEV).float()
    dl = dlast.to(DEV)
    g_ck, g_h = torch.empty_like(hg), torch.empty_like(hg)
    dh0_ck = S._launch_bwd(hv, gv, h0d, None, ckpt_r, dhd, dl, g_ck[..., :Di], g_ck[..., Di:], with_h0)
    dh0_h = S._launch_bwd(hv, gv, h0d, h, None, dhd, dl, g_h[..., :Di], g_h[..., Di:], with_h0)
    S.check_workspaces()
    # A checkpoint is the state at the end of a forward run, while the forward's next run
    # starts from the composed run maps, so rebuilt and stored states differ by fp32
    # rounding; the bf16 gradients' stochastic rounding then lands on the other side now
    # and then (its hash reads the values). So: near-equal, and both against the oracle.
    close = 1e-5 if dtype == torch.float32 else 4e-3
    assert _rel_norm(g_ck.float().cpu(), g_h.float().cpu()) <= close
    if with_h0:
        assert _rel_norm(dh0_ck.cpu(), dh0_h.cpu()) <= close
    if B * T * Di <= 1 << 20:
        ref = _oracle(hidden, gate, h0, dh.float(), dlast)
        tol = TOL[dtype]
        assert _rel_norm(g_ck[..., :Di].float().cpu(), ref[2]) <= tol
        assert _rel_norm(g_ck[..., Di:].float().cpu(), ref[3]) <= tol
