"""GPU parity of the bf16 MFMA products (mg_gemm) against float64 products
of the same bf16 inputs (plain torch on the CPU) and, at full model sizes,
against torch's float32 product on the GPU.

Tolerances: fp32 outputs 1e-5 relative (Frobenius), per-element within
1e-5 of the row scale; bf16 outputs are one bf16 rounding of the fp32 value
(relative 2^-8 per element, plus the fp32 accumulation error).
"""
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _operand(rows, k, layout, gen, scale=1.0, pad=0):
    """bf16 operand with logical shape [rows, k] stored K- or MN-contiguous (pad = extra leading-dim room)."""
    from gruboros_amd.gemm import KCONTIG

    logical = (torch.randn(rows, k, generator=gen, dtype=torch.float64) * scale).to(torch.bfloat16)
    if layout == KCONTIG:
        store = torch.zeros(rows, k + pad, dtype=torch.bfloat16)
        store[:, :k] = logical
        dev = store.to(DEV)[:, :k]
    else:
        store = torch.zeros(k, rows + pad, dtype=torch.bfloat16)
        store[:, :rows] = logical.t()
        dev = store.to(DEV)[:, :rows]
    return logical.double(), dev


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-300))


@pytest.mark.parametrize("a_layout,b_layout", [(0, 0), (0, 1), (1, 1), (1, 0)])
@pytest.mark.parametrize("M,N,K", [(1, 8, 8), (37, 64, 200), (128, 256, 64), (300, 520, 1024), (1000, 136, 72),
                                   (513, 264, 8)])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_gemm_layouts(a_layout, b_layout, M, N, K, out_dtype):
    from gruboros_amd.gemm import gemm

    if a_layout == 1 and M % 8:
        M = (M + 7) // 8 * 8
    gen = torch.Generator().manual_seed(M * 7 + N * 3 + K)
    a64, a = _operand(M, K, a_layout, gen, pad=8)
    b64, b = _operand(N, K, b_layout, gen, pad=8)
    ref = a64 @ b64.t()
    out = torch.full((M, N + 8), 7.0, device=DEV, dtype=out_dtype)[:, :N]
    gemm(a, a_layout, b, b_layout, M, N, K, out)
    torch.cuda.synchronize()
    got = out.double().cpu()
    if out_dtype == torch.float32:
        assert _rel(got, ref) < 1e-5
    else:
        # one rounding to bf16 of a value accurate to ~1e-6
        err = (got - ref).abs()
        assert bool((err <= ref.abs() * 2.0 ** -8 + 1e-5 * ref.abs().max()).all())
    # the padding columns of C are untouched
    assert bool((torch.full((M, 8), 7.0, device=DEV, dtype=out_dtype) ==
                 out.as_strided((M, 8), (N + 8, 1), out.storage_offset() + N)).all())


def test_gemm_epilogues():
    from gruboros_amd.gemm import EPI_BIAS, EPI_BIAS_GELU, EPI_GELU_GRAD, KCONTIG, MNCONTIG, gemm

    gen = torch.Generator().manual_seed(5)
    M, N, K = 777, 264, 136
    a64, a = _operand(M, K, KCONTIG, gen)
    b64, b = _operand(N, K, KCONTIG, gen, scale=0.2)
    bias = torch.randn(N, generator=gen, dtype=torch.float64).float()
    acc = a64 @ b64.t()
    # bias, fp32 and bf16 outputs
    for dt in (torch.float32, torch.bfloat16):
        out = torch.empty(M, N, device=DEV, dtype=dt)
        gemm(a, KCONTIG, b, KCONTIG, M, N, K, out, epilogue=EPI_BIAS, bias=bias.to(DEV))
        assert _rel(out, acc + bias.double()) < (1e-5 if dt == torch.float32 else 4e-3)
    # bias + GELU: aux = bf16(acc + bias), out = gelu(aux)
    aux = torch.empty(M, N, device=DEV, dtype=torch.bfloat16)
    out = torch.empty(M, N, device=DEV, dtype=torch.bfloat16)
    gemm(a, KCONTIG, b, KCONTIG, M, N, K, out, epilogue=EPI_BIAS_GELU, bias=bias.to(DEV), aux=aux)
    pre = acc + bias.double()
    assert _rel(aux, pre) < 4e-3
    gelu_of_aux = torch.nn.functional.gelu(aux.double().cpu())
    assert _rel(out, gelu_of_aux) < 4e-3
    # GELU gradient: out = (dy w) * gelu'(aux)
    dy64, dy = _operand(M, N, KCONTIG, gen)
    w64 = b64  # [N, K]; dX = dY W: A = dy (K-contig over N), B(k=n, j) = w[n][j] -> MN-contig
    dx = torch.empty(M, K, device=DEV, dtype=torch.bfloat16)
    aux2 = aux[:, :K].contiguous() if K <= N else None
    gemm(dy, KCONTIG, b, MNCONTIG, M, K, N, dx, epilogue=EPI_GELU_GRAD, aux=aux2)
    x = aux2.double().cpu().requires_grad_(True)
    torch.nn.functional.gelu(x).backward(torch.ones_like(x))
    ref = (dy64 @ w64) * x.grad
    assert _rel(dx, ref) < 4e-3


def test_gemm_epilogues_256_tiles():
    """The bias, bias+GELU and GELU-gradient epilogues of the 256 x 256 kernels
    (chosen once a product has at least one 256 x 256 tile per CU): ragged M,
    against torch's fp32 product of the same bf16 inputs on the GPU."""
    from gruboros_amd.gemm import EPI_BIAS, EPI_BIAS_GELU, EPI_GELU_GRAD, KCONTIG, MNCONTIG, gemm

    g = torch.Generator(device=DEV).manual_seed(21)
    M, N, K = 4133, 4096, 192  # 17 x 16 = 272 tiles of 256 x 256
    x = torch.randn(M, K, device=DEV, generator=g).to(torch.bfloat16)
    w = (torch.randn(N, K, device=DEV, generator=g) * 0.1).to(torch.bfloat16)
    bias = torch.randn(N, device=DEV, generator=g)
    pre_ref = x.float() @ w.float().t() + bias
    y = torch.empty(M, N, device=DEV, dtype=torch.bfloat16)
    gemm(x, KCONTIG, w, KCONTIG, M, N, K, y, epilogue=EPI_BIAS, bias=bias)
    assert _rel(y, pre_ref) < 4e-3
    pre = torch.empty(M, N, device=DEV, dtype=torch.bfloat16)
    gemm(x, KCONTIG, w, KCONTIG, M, N, K, y, epilogue=EPI_BIAS_GELU, bias=bias, aux=pre)
    assert _rel(pre, pre_ref) < 4e-3
    assert _rel(y, torch.nn.functional.gelu(pre.float())) < 4e-3
    # GELU gradient: dX = (dY W) * gelu'(pre), dY [M, N], W [N, K] read MN-contiguous
    dy = torch.randn(M, K, device=DEV, generator=g).to(torch.bfloat16)
    w2 = (torch.randn(K, N, device=DEV, generator=g) * 0.1).to(torch.bfloat16)
    dx = torch.empty(M, N, device=DEV, dtype=torch.bfloat16)
    gemm(dy, KCONTIG, w2, MNCONTIG, M, N, K, dx, epilogue=EPI_GELU_GRAD, aux=pre)
    p = pre.float().requires_grad_(True)
    torch.nn.functional.gelu(p).backward(torch.ones_like(p))
    assert _rel(dx, (dy.float() @ w2.float()) * p.grad) < 4e-3


def test_bias_gelu_epilogue_every_bf16_value():
    """The bias + GELU epilogue over all 65536 bf16 values: x = 0 and bias =
    every bf16 bit pattern (as fp32), so aux = bias and C = bf16(gelu(aux)).
    The persistent kernel (512 x 65536: 512 tiles) looks GELU up in a table;
    the per-tile kernel (16 rows) computes it: the two agree bit for bit.
    Against torch's CPU GELU (the same fp32 formula x (1 + erf(x / sqrt 2)) / 2
    with another erf): equal on >= 99.5% of the finite values, and within
    |x| 2^-22 (the rounding of 1 + erf, which cancels for x < -3) plus one bf16
    spacing everywhere. Checked by the formula's value instead: NaN -> NaN,
    +inf -> +inf, -inf -> NaN, and x > 2^127 -> x (torch's CPU kernel forms
    x (1 + erf) first and overflows there)."""
    from gruboros_amd.gemm import EPI_BIAS_GELU, KCONTIG, gemm

    bits = torch.arange(-32768, 32768, dtype=torch.int32).to(torch.int16)
    vals = bits.view(torch.bfloat16)
    N, K = vals.numel(), 128
    bias = vals.float().to(DEV)
    w = torch.randn(N, K, device=DEV).to(torch.bfloat16)
    pre = vals.clone()
    pre[bits == -32768] = 0.0  # aux = 0 + bias: +0 for -0
    outs = []
    for M in (512, 16):
        x = torch.zeros(M, K, device=DEV, dtype=torch.bfloat16)
        aux = torch.empty(M, N, device=DEV, dtype=torch.bfloat16)
        out = torch.empty(M, N, device=DEV, dtype=torch.bfloat16)
        gemm(x, KCONTIG, w, KCONTIG, M, N, K, out, epilogue=EPI_BIAS_GELU, bias=bias, aux=aux)
        torch.cuda.synchronize()
        a = aux.cpu()
        assert bool(((a.view(torch.int16) == pre.view(torch.int16)) | (a.isnan() & pre.isnan())).all())
        outs.append(out.cpu())
    big, small = outs
    assert bool((big.view(torch.int16) == small[:1].view(torch.int16)).all())  # table == computed, every row
    got = small[0]
    assert bool(got[pre.isnan()].isnan().all())
    inf = pre.isinf()
    assert got[inf & (pre > 0)].item() == float("inf") and bool(got[inf & (pre < 0)].isnan().all())
    huge = pre.float() > 2.0 ** 127
    assert bool((got[huge].view(torch.int16) == pre[huge].view(torch.int16)).all())
    fin = pre.isfinite() & ~huge
    ref = torch.nn.functional.gelu(pre[fin].float()).bfloat16()
    g = got[fin]
    assert not bool(g.isnan().any())
    same = g.view(torch.int16) == ref.view(torch.int16)
    assert float(same.float().mean()) >= 0.995, int((~same).sum())
    xd, gd, rd = pre[fin].double(), g.double(), ref.double()
    assert bool(((gd - rd).abs() <= xd.abs() * 2.0 ** -22 + rd.abs() * 2.0 ** -7 + 2.0 ** -133).all())


def test_gemm_accumulate_and_split():
    """fp32 dW-shaped product (long K, 79 k-tiles): split along K into slices
    of an odd k-tile count, summed by the reduction pass; accumulate adds to C."""
    from gruboros_amd.gemm import linear_dw

    gen = torch.Generator().manual_seed(9)
    T, O, I = 5000, 264, 136
    dy = (torch.randn(T, O, generator=gen, dtype=torch.float64)).to(torch.bfloat16)
    x = (torch.randn(T, I, generator=gen, dtype=torch.float64)).to(torch.bfloat16)
    ref = dy.double().t() @ x.double()
    out = linear_dw(dy.to(DEV), x.to(DEV))
    assert _rel(out, ref) < 1e-5
    base = torch.randn(O, I, generator=gen).float()
    acc = base.to(DEV)
    linear_dw(dy.to(DEV), x.to(DEV), out=acc, accumulate=True)
    assert _rel(acc, ref + base.double()) < 1e-5


def test_gemm_deterministic_flag():
    """Weight-gradient product with and without the split along K (partials
    summed in split order by a separate reduction pass): both forms repeat bit
    for bit, also with other shapes run on the same workspace in between, and
    they agree with each other."""
    from gruboros_amd.gemm import linear_dw

    g = torch.Generator(device=DEV).manual_seed(11)
    dy = torch.randn(16376, 1024, device=DEV, generator=g).to(torch.bfloat16)
    x = torch.randn(16376, 1024, device=DEV, generator=g).to(torch.bfloat16)
    dy4 = torch.randn(16376, 4096, device=DEV, generator=g).to(torch.bfloat16)
    d1 = linear_dw(dy, x, deterministic=True)
    d2 = linear_dw(dy, x, deterministic=True)
    split = linear_dw(dy, x, deterministic=False)
    w4 = linear_dw(dy4, x, deterministic=False)   # another split plan on the same workspace
    split2 = linear_dw(dy, x, deterministic=False)
    w4b = linear_dw(dy4, x, deterministic=False)
    assert torch.equal(d1, d2)
    assert torch.equal(split, split2) and torch.equal(w4, w4b)
    assert _rel(split, d1) < 1e-6
    assert _rel(w4, dy4.float().t() @ x.float()) < 1e-5
    acc = d1.clone()
    linear_dw(dy, x, out=acc, accumulate=True, deterministic=True)
    assert _rel(acc, 2 * d1) < 1e-6


@pytest.mark.parametrize("which", ["hg_fwd", "hg_dx", "hg_dw", "ff1_fwd", "ff2_dw", "logits_fwd"])
def test_gemm_model_sizes(which):
    """cfg3 shapes (16376 tokens, d1024, ff 4096, vocab 256) vs torch's fp32 product on the GPU."""
    from gruboros_amd.gemm import linear_dw, linear_dx, linear_fwd

    g = torch.Generator(device=DEV).manual_seed(3)
    T = 16376
    shapes = {"hg_fwd": (1024, 2048), "hg_dx": (1024, 2048), "hg_dw": (1024, 2048), "ff1_fwd": (1024, 4096),
              "ff2_dw": (4096, 1024), "logits_fwd": (1024, 256)}
    fin, fout = shapes[which]
    x = torch.randn(T, fin, device=DEV, generator=g).to(torch.bfloat16)
    w = (torch.randn(fout, fin, device=DEV, generator=g) * 0.02).to(torch.bfloat16)
    dy = torch.randn(T, fout, device=DEV, generator=g).to(torch.bfloat16)
    if which.endswith("fwd"):
        got = linear_fwd(x, w, out_dtype=torch.float32)
        ref = x.float() @ w.float().t()
    elif which.endswith("dx"):
        got = linear_dx(dy, w).float()
        ref = dy.float() @ w.float()
    else:
        got = linear_dw(dy, x)
        ref = dy.float().t() @ x.float()
    tol = 1e-5 if got.dtype == torch.float32 and not which.endswith("dx") else 4e-3
    assert _rel(got, ref) < tol


@pytest.mark.parametrize("fused_fwd", [True, False])
@pytest.mark.parametrize("fused_bwd", [True, False])
def test_feed_forward_bf16_matches_fp64(fused_fwd, fused_bwd, monkeypatch):
    """bf16 FeedForward with the GELU in the MFMA epilogues or in separate
    passes (forward and backward independently) vs the fp64 reference
    Linear -> GELU -> Linear (reference mingru/minLM.py:17-23)."""
    from gruboros_amd import linear as lin
    from gruboros_amd.linear import feed_forward

    monkeypatch.setattr(lin, "FUSED_GELU_FORWARD", fused_fwd)
    monkeypatch.setattr(lin, "FUSED_GELU_BACKWARD", fused_bwd)
    torch.manual_seed(4)
    D, F_ = 256, 1024
    ff = torch.nn.Sequential(torch.nn.Linear(D, F_), torch.nn.GELU(), torch.nn.Linear(F_, D)).to(DEV)
    with torch.no_grad():
        ff[2].weight.normal_(0, 0.05)
        ff[2].bias.normal_(0, 0.1)
    x = torch.randn(3, 333, D, device=DEV).to(torch.bfloat16).requires_grad_(True)
    y = feed_forward(x, ff)
    assert y.dtype == torch.bfloat16 and y.shape == (3, 333, D)
    dy = torch.randn(y.shape, device=DEV)
    (y.float() * dy).sum().backward()
    ref = [t.detach().double().cpu().requires_grad_(True) for t in (x, ff[0].weight, ff[0].bias, ff[2].weight, ff[2].bias)]
    x64, w1, b1, w2, b2 = ref
    y64 = torch.nn.functional.linear(torch.nn.functional.gelu(torch.nn.functional.linear(x64, w1, b1)), w2, b2)
    (y64 * dy.double().cpu()).sum().backward()
    assert _rel(y, y64) < 2e-2
    for got, want in ((x.grad, x64.grad), (ff[0].weight.grad, w1.grad), (ff[0].bias.grad, b1.grad),
                      (ff[2].weight.grad, w2.grad), (ff[2].bias.grad, b2.grad)):
        assert got.dtype == (torch.bfloat16 if got is x.grad else torch.float32)
        assert _rel(got, want) < 2e-2


def test_split_hilo_matches_torch_rounding():
    from gruboros_amd.gemm import split_hilo

    gen = torch.Generator(device=DEV).manual_seed(4)
    x = torch.randn(77, 136, device=DEV, generator=gen) * torch.logspace(-6, 6, 136, device=DEV)
    pair = split_hilo(x)
    hi = x.to(torch.bfloat16)
    lo = (x - hi.float()).to(torch.bfloat16)
    assert torch.equal(pair[:, :136], hi) and torch.equal(pair[:, 136:], lo)
    err = (pair[:, :136].double() + pair[:, 136:].double() - x.double()).abs()
    assert bool((err <= x.double().abs() * 2.0 ** -16).all())


@pytest.mark.parametrize("M,N,K,out_dtype", [(300, 200, 136, torch.float32), (16376, 1024, 1024, torch.bfloat16),
                                              (16376, 1024, 1536, torch.float32), (1000, 96, 72, torch.float32)])
def test_hilo_product_is_fp32_accurate(M, N, K, out_dtype):
    """MG_GEMM_HILO from fp32 operands split into hi/lo pairs: the fp32 result
    is within 2e-5 (norm-relative; expected ~7e-6 from the pair's 2^-16
    representation error and the dropped lo*lo term) of the fp64 product of
    the fp32 operands, where a plain bf16 product of the same operands is
    ~3e-3 off; bf16
    outputs are one rounding of that value. Shapes: ragged, the cfg3 hidden
    half (written into the packed [N, 2 Di] projection buffer), the cfg3
    expansion-1.5 to_out (fp32 out), and a small K."""
    from gruboros_amd.gemm import KCONTIG, gemm, linear_fwd_hilo, split_hilo

    gen = torch.Generator(device=DEV).manual_seed(M + N + K)
    a = torch.randn(M, K, device=DEV, generator=gen)
    b = torch.randn(N, K, device=DEV, generator=gen) * 0.02
    ref = (a.double() @ b.double().t()).cpu()
    buf = torch.full((M, 2 * N), 3.0, device=DEV, dtype=out_dtype)
    out = buf[:, :N]
    linear_fwd_hilo(split_hilo(a), split_hilo(b), out, K)
    plain = torch.empty(M, N, device=DEV)
    gemm(a.to(torch.bfloat16), KCONTIG, b.to(torch.bfloat16), KCONTIG, M, N, K, plain)
    torch.cuda.synchronize()
    e_plain = _rel(plain, ref)
    if out_dtype == torch.float32:
        e = _rel(out, ref)
        print(f"hilo {M}x{N}x{K}: {e:.2e} (plain bf16 {e_plain:.2e})", flush=True)
        assert e <= 2e-5 and e_plain > 1e-3
    else:
        got = out.double().cpu()
        assert bool(((got - ref).abs() <= ref.abs() * 2.0 ** -8 + 1e-5 * ref.abs().max()).all())
    assert bool((buf[:, N:] == 3.0).all())  # the other half of the packed buffer is untouched


def _dev_operand(rows, k, layout, g, scale=1.0):
    """bf16 operand [rows, k] (logical) stored K-contiguous ([rows, k]) or MN-contiguous ([k, rows])."""
    logical = (torch.randn(rows, k, device=DEV, generator=g) * scale).to(torch.bfloat16)
    return logical, (logical if layout == 0 else logical.t().contiguous())


@pytest.mark.parametrize("al,bl,M,N,K", [
    (0, 0, 16376, 1024, 1024),   # forward products: ragged M (rows past M read zero)
    (0, 1, 16376, 1024, 2048),   # input gradients (B read through the transposed LDS read)
    (1, 0, 4096, 4096, 1024),    # MN-contiguous A
    (1, 1, 2048, 1024, 16376),   # weight gradients: ragged K tail, split along K
    (1, 1, 4096, 1024, 4104),    # the shortest K on 256 x 256 weight-gradient tiles, ragged
    (1, 1, 4096, 1024, 1000),    # short ragged K: 128 x 128 tiles
])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_gemm_four_wave_tiles(al, bl, M, N, K, out_dtype):
    """The four-wave 256 x 256 loop (mainloop_w4: every operand layout, no masked
    loads; weight gradients below K 4096 take 128 x 128 tiles) against fp64 products
    of the same bf16 operands."""
    from gruboros_amd.gemm import gemm

    g = torch.Generator(device=DEV).manual_seed(M + N + K + al + 2 * bl)
    a, ad = _dev_operand(M, K, al, g)
    b, bd = _dev_operand(N, K, bl, g)
    ref = a.double() @ b.double().t()
    out = torch.full((M, N + 8), 5.0, device=DEV, dtype=out_dtype)[:, :N]
    gemm(ad, al, bd, bl, M, N, K, out)
    torch.cuda.synchronize()
    if out_dtype == torch.float32:
        assert _rel(out, ref) < 1e-5
    else:
        err = (out.double() - ref).abs()
        assert bool((err <= ref.abs() * 2.0 ** -8 + 1e-5 * ref.abs().max()).all())
    if out_dtype == torch.float32 and al == 1 and bl == 1:
        # deterministic (unsplit) and accumulating forms of the weight gradient
        det = torch.empty(M, N, device=DEV)
        gemm(ad, al, bd, bl, M, N, K, det, deterministic=True)
        assert _rel(det, ref) < 1e-5
        acc = torch.ones(M, N, device=DEV)
        gemm(ad, al, bd, bl, M, N, K, acc, accumulate=True)
        assert _rel(acc - 1.0, ref) < 1e-5


def test_gemm_four_wave_epilogues():
    """Epilogues on the four-wave tiles: bias, bias + GELU (pre-activation kept),
    the GELU gradient on an input-gradient product, and the stochastic rounding
    of a bf16 gradient (unbiased: the mean error of 16 M elements is ~0)."""
    import torch.nn.functional as F

    from gruboros_amd.gemm import EPI_BIAS, EPI_BIAS_GELU, EPI_GELU_GRAD, KCONTIG, MNCONTIG, gemm

    g = torch.Generator(device=DEV).manual_seed(9)
    M, N, K = 16376, 1024, 1024
    a, _ = _dev_operand(M, K, 0, g)
    b, _ = _dev_operand(N, K, 0, g, scale=0.05)
    bias = torch.randn(N, device=DEV, generator=g)
    acc64 = a.double() @ b.double().t()
    y = torch.empty(M, N, device=DEV, dtype=torch.bfloat16)
    gemm(a, KCONTIG, b, KCONTIG, M, N, K, y, epilogue=EPI_BIAS, bias=bias)
    ref = acc64 + bias.double()
    assert bool(((y.double() - ref).abs() <= ref.abs() * 2.0 ** -8 + 1e-5 * ref.abs().max()).all())
    pre = torch.empty_like(y)
    gemm(a, KCONTIG, b, KCONTIG, M, N, K, y, epilogue=EPI_BIAS_GELU, bias=bias, aux=pre)
    assert bool(((pre.double() - ref).abs() <= ref.abs() * 2.0 ** -8 + 1e-5 * ref.abs().max()).all())
    assert _rel(y, F.gelu(pre.double())) < 4e-3
    # input-gradient layout with the GELU gradient: C = (dY W) * gelu'(pre)
    wt, wt_mn = _dev_operand(N, K, 1, g, scale=0.05)  # B(k, n) stored [K, N]
    dx = torch.empty(M, N, device=DEV, dtype=torch.bfloat16)
    gemm(a, KCONTIG, wt_mn, MNCONTIG, M, N, K, dx, epilogue=EPI_GELU_GRAD, aux=pre)
    p64 = pre.double().requires_grad_(True)
    F.gelu(p64).backward(a.double() @ wt.double().t())
    assert _rel(dx, p64.grad) < 4e-3
    # stochastic rounding of a plain bf16 result: unbiased against the fp32 value
    c32 = torch.empty(M, N, device=DEV)
    gemm(a, KCONTIG, wt_mn, MNCONTIG, M, N, K, c32)
    sr = torch.empty(M, N, device=DEV, dtype=torch.bfloat16)
    gemm(a, KCONTIG, wt_mn, MNCONTIG, M, N, K, sr, stochastic=True)
    rel_err = (sr.double() - c32.double()) / c32.double().abs().clamp_min(1e-3)
    assert float(rel_err.abs().max()) <= 2.0 ** -7 * 1.01   # within one bf16 spacing
    assert abs(float(rel_err.mean())) < 2e-5                # unbiased (round-to-nearest: also ~0, but
    ne = (sr != c32.to(torch.bfloat16)).float().mean()       # it differs from round-to-nearest often)
    assert float(ne) > 0.2


def test_products_over_2gib_run_in_row_blocks():
    """Operands spanning more than mg_gemm's 2 GiB buffer range (the cfg4
    full-length FeedForward: 262,144 rows x 4096) run as row blocks: the
    forward and input-gradient products block by row, the weight gradient by
    K, each block added to the last. Checked around the block boundary and at
    the end against fp32 products of the same bf16 operands."""
    from gruboros_amd.gemm import _row_step, linear_dw, linear_fwd

    N, K, O = 1_100_000, 1024, 256
    step = _row_step(N, 2 * K, 2 * O)
    assert step < N  # the product is split
    g = torch.Generator(device=DEV).manual_seed(7)
    x = torch.randn(N, K, device=DEV, generator=g).to(torch.bfloat16)
    w = (torch.randn(O, K, device=DEV, generator=g) * 0.05).to(torch.bfloat16)
    y = linear_fwd(x, w)
    for r0, r1 in ((0, 256), (step - 512, step + 512), (N - 300, N)):
        ref = x[r0:r1].float() @ w.float().t()
        err = (y[r0:r1].float() - ref).abs().max() / ref.abs().max()
        assert float(err) < 8e-3, (r0, float(err))
    dy = torch.randn(N, O, device=DEV, generator=g).to(torch.bfloat16)
    dw = linear_dw(dy, x)
    ref = torch.zeros(O, K, device=DEV, dtype=torch.float64)
    for r0 in range(0, N, 1 << 18):
        ref += (dy[r0:r0 + (1 << 18)].float().t() @ x[r0:r0 + (1 << 18)].float()).double()
    err = (dw.double() - ref).abs().max() / ref.abs().max()
    assert float(err) < 1e-4, float(err)


@pytest.mark.parametrize("al,bl,M,N,K,hilo", [
    (0, 0, 4133, 4104, 256, False),    # ragged M and N, 17 x 17 tiles: some workgroups take two
    (0, 1, 16376, 4096, 1024, False),  # the input gradient into the FeedForward (4 tiles per workgroup)
    (1, 0, 4352, 4096, 512, False),    # MN-contiguous A
    (1, 1, 4352, 4096, 128, False),    # both MN-contiguous
    (0, 0, 4133, 2048, 1024, True),    # hi/lo operands (three K segments)
])
def test_gemm_persistent_matches_per_tile_kernel(al, bl, M, N, K, hilo, monkeypatch):
    """Products with more 256 x 256 tiles than CUs and a bf16 output run the
    persistent kernel (one workgroup per CU walking its tiles, the next tile's
    first k-tile prefetched under the last k-tile, the epilogue in registers).
    Every epilogue must equal the per-tile kernel's result bit for bit (same
    sums in the same order, same rounding), and the plain product must match
    the fp64 product of the same operands."""
    from gruboros_amd.gemm import EPI_BIAS, EPI_BIAS_GELU, EPI_NONE, gemm

    g = torch.Generator(device=DEV).manual_seed(M + N + K + 3 * al + 5 * bl)
    kk = 2 * K if hilo else K
    a, ad = _dev_operand(M, kk, al, g)
    b, bd = _dev_operand(N, kk, bl, g, scale=0.05)
    bias = torch.randn(N, device=DEV, generator=g)
    cases = [dict(epilogue=EPI_NONE), dict(stochastic=True)]
    if not hilo:
        cases += [dict(epilogue=EPI_BIAS), dict(epilogue=EPI_BIAS_GELU)]
    for kw in cases:
        outs = []
        for mode in ("1", "0"):
            monkeypatch.setenv("MG_GEMM_PERSIST", mode)
            y_full = torch.full((M, N + 8), 3.0, device=DEV, dtype=torch.bfloat16)
            pre_full = torch.full((M, N + 8), 3.0, device=DEV, dtype=torch.bfloat16)
            y, pre = y_full[:, :N], pre_full[:, :N]
            extra = {}
            if kw.get("epilogue") in (EPI_BIAS, EPI_BIAS_GELU):
                extra["bias"] = bias
            if kw.get("epilogue") == EPI_BIAS_GELU:
                extra["aux"] = pre
            gemm(ad, al, bd, bl, M, N, K, y, hilo=hilo, **kw, **extra)
            torch.cuda.synchronize()
            outs.append((y_full, pre_full))
        print(f"persistent {al}{bl} {M}x{N}x{K} hilo={hilo} {kw}", flush=True)
        assert torch.equal(outs[0][0], outs[1][0]), f"output differs from the per-tile kernel ({kw})"
        assert torch.equal(outs[0][1], outs[1][1]), f"aux differs from the per-tile kernel ({kw})"
        if kw == dict(epilogue=EPI_NONE):
            if hilo:  # A_hi B_hi + A_lo B_hi + A_hi B_lo (the lo x lo term is left out by design)
                ah, al_, bh, bl_ = a[:, :K].double(), a[:, K:].double(), b[:, :K].double(), b[:, K:].double()
                ref = ah @ bh.t() + al_ @ bh.t() + ah @ bl_.t()
            else:
                ref = a.double() @ b.double().t()
            got = outs[0][0][:, :N].double()
            assert bool(((got - ref).abs() <= ref.abs() * 2.0 ** -8 + 1e-5 * ref.abs().max()).all())
            assert bool((outs[0][0][:, N:] == 3.0).all()), "padding columns written"


@pytest.mark.parametrize("al,bl,M,N,K", [
    (1, 1, 2048, 1024, 16376),   # to_hidden_and_gate weight gradient: 32 tiles x 8 splits
    (1, 1, 4096, 1024, 16376),   # FeedForward weight gradients: 64 tiles x 4 splits
    (1, 1, 256, 1024, 16376),    # logits weight gradient: 4 tiles, many splits
    (0, 0, 512, 520, 4000),      # K-contiguous split product (ragged N)
])
def test_gemm_split_layout_matches(al, bl, M, N, K, monkeypatch):
    """K-split fp32 products run as a 1-D grid whose workgroups on one XCD
    share a split (split_tile_of). The partials and their in-order reduction
    are the same as with the 2-D (tile, split) grid, so the results must be
    equal bit for bit; and within 1e-5 of the fp64 product."""
    from gruboros_amd.gemm import gemm

    g = torch.Generator(device=DEV).manual_seed(M + N + K + al)
    a, ad = _dev_operand(M, K, al, g)
    b, bd = _dev_operand(N, K, bl, g)
    outs = []
    for mode in ("1", "0"):
        monkeypatch.setenv("MG_GEMM_XCD_SPLIT", mode)
        out = torch.empty(M, N, device=DEV)
        gemm(ad, al, bd, bl, M, N, K, out)
        torch.cuda.synchronize()
        outs.append(out)
    assert torch.equal(outs[0], outs[1])
    assert _rel(outs[0], a.double() @ b.double().t()) < 1e-5


@pytest.mark.parametrize("al,bl,M,N,K", [
    (0, 1, 2048, 1024, 6144),    # to_hidden_and_gate input gradient at one [1, 2048] chunk: 128 tiles x 2 splits
    (0, 0, 512, 520, 4000),      # ragged N, 20 tiles x 12 splits
    (1, 1, 256, 264, 3000),      # both MN-contiguous (weight-gradient layout), ragged K
    (0, 1, 37, 64, 2000),        # one ragged tile, 8 splits
])
def test_gemm_bf16_split_rounds_the_fp32_split_sum(al, bl, M, N, K):
    """bf16 products with no epilogue whose tiles leave CUs idle split along K as the fp32
    products do (fp32 partials, summed in split order by the reduction pass), and the pass rounds
    the sum once: to nearest, or stochastically with the unsplit epilogue's hash of the element
    index. So they equal the fp32 split product rounded by torch (to nearest) or by
    mg_round_bf16_sr with the gradient salt 0x9e5b, bit for bit; with a bias epilogue, the bias
    is added to that fp32 sum before the rounding to nearest; and the unsplit product
    (deterministic flag) and the split one are both within one bf16 rounding of the fp64 product."""
    from gruboros_amd import _lib
    from gruboros_amd.gemm import EPI_BIAS, EPI_NONE, gemm, round_bf16_sr

    L = _lib.lib()
    for epi in (EPI_NONE, EPI_BIAS):
        assert L.mg_gemm_workspace_bytes(al, bl, M, N, K, epi, _lib.dtype_code(torch.bfloat16), 0) > 0, "not split"
    g = torch.Generator(device=DEV).manual_seed(M + N + K + 7 * al + 11 * bl)
    a, ad = _dev_operand(M, K, al, g)
    b, bd = _dev_operand(N, K, bl, g, scale=0.05)
    f32 = torch.empty(M, N, device=DEV)
    gemm(ad, al, bd, bl, M, N, K, f32)
    rn = torch.full((M, N), 3.0, device=DEV, dtype=torch.bfloat16)
    gemm(ad, al, bd, bl, M, N, K, rn)
    sr = torch.full_like(rn, 3.0)
    gemm(ad, al, bd, bl, M, N, K, sr, stochastic=True)
    sr2 = torch.full_like(rn, 3.0)
    gemm(ad, al, bd, bl, M, N, K, sr2, stochastic=True)
    whole = torch.full_like(rn, 3.0)
    gemm(ad, al, bd, bl, M, N, K, whole, deterministic=True)
    bias = torch.randn(N, device=DEV, generator=g)
    rb = torch.full_like(rn, 3.0)
    gemm(ad, al, bd, bl, M, N, K, rb, epilogue=EPI_BIAS, bias=bias)
    torch.cuda.synchronize()
    print(f"bf16 split {al}{bl} {M}x{N}x{K}", flush=True)
    assert torch.equal(rn, f32.to(torch.bfloat16))
    assert torch.equal(rb, (f32 + bias).to(torch.bfloat16))
    assert torch.equal(sr, round_bf16_sr(f32, salt=0x9e5b)) and torch.equal(sr, sr2)
    ref = a.double() @ b.double().t()
    floor = 1e-5 * float(ref.abs().max())
    for got, ulps in ((rn, 2.0 ** -8), (whole, 2.0 ** -8), (sr, 2.0 ** -7)):
        assert bool(((got.double() - ref).abs() <= ref.abs() * ulps + floor).all())
    if M * N >= 1 << 16:  # stochastic rounding is unbiased: the signed errors average out
        err = sr.double() - f32.double()
        assert abs(float(err.mean())) <= 0.05 * float(err.abs().mean())


@pytest.mark.parametrize("shapes,K,paired,strided", [
    (((1024, 4096), (4096, 1024)), 16376, True, False),    # cfg3 FeedForward weight gradients: 128 tiles x 2 splits
    (((1024, 1024), (1024, 2048)), 3000, True, False),     # 48 tiles x 5 splits, ragged K
    (((1024, 1536), (3072, 1024)), 8192, True, True),      # to_out + to_hidden_and_gate at x1.5, hi halves of pairs
    (((264, 512), (512, 264)), 5000, False, False),        # not whole 256 x 256 tiles: each product alone
    (((2048, 8192), (8192, 2048)), 1024, False, False),    # cfg5 widths: 512 tiles, no split
])
def test_wgrad_pair_matches_fp64_and_single_products(shapes, K, paired, strided):
    """mg_gemm_wgrad_pair (the FeedForward's dW2 = dp^T act and dW1 = dpre^T n2
    in one K-split launch) against float64 products of the same bf16 inputs
    (1e-5 relative), against one mg_gemm per product (1e-6 when the pair runs
    paired, which splits K in half as many parts; bit for bit when it runs
    each product alone), repeat calls bit for bit, and accumulation."""
    from gruboros_amd import _lib
    from gruboros_amd.gemm import linear_dw, linear_dw_pair

    L = _lib.lib()
    (m0, n0), (m1, n1) = shapes
    t0, t1 = (m0 // 256) * (n0 // 256), (m1 // 256) * (n1 // 256)
    whole = m0 % 256 == 0 and n0 % 256 == 0 and m1 % 256 == 0 and n1 % 256 == 0
    assert paired == (whole and min(t0, t1) >= 16 and t0 + t1 < 256)
    g = torch.Generator(device=DEV).manual_seed(K + m0)
    dy0, x0 = [torch.randn(K, c, device=DEV, generator=g).to(torch.bfloat16) for c in (m0, n0)]
    dy1, x1 = [torch.randn(K, c, device=DEV, generator=g).to(torch.bfloat16) for c in (m1, n1)]
    if strided:  # the x operands as the first halves of [K, 2 n] rows, as the hi/lo pairs are read
        x0 = torch.cat([x0, torch.randn_like(x0, dtype=torch.float32).to(torch.bfloat16)], 1)[:, :n0]
        x1 = torch.cat([x1, torch.randn_like(x1, dtype=torch.float32).to(torch.bfloat16)], 1)[:, :n1]
    a, b = linear_dw_pair(dy0, x0, dy1, x1)
    a2, b2 = linear_dw_pair(dy0, x0, dy1, x1)
    assert torch.equal(a, a2) and torch.equal(b, b2)
    for got, dy, x in ((a, dy0, x0), (b, dy1, x1)):
        ref = dy.double().t() @ x.double()
        assert _rel(got, ref) < 1e-5
        single = linear_dw(dy, x)
        if paired:
            assert _rel(got, single) < 1e-6
        else:
            assert torch.equal(got, single)
    # accumulation: dw += product, through the C ABI
    base0 = torch.randn(m0, n0, device=DEV, generator=g)
    base1 = torch.randn(m1, n1, device=DEV, generator=g)
    c0, c1 = base0.clone(), base1.clone()
    wsb = L.mg_gemm_wgrad_pair_workspace_bytes(m0, n0, m1, n1, K, 1)
    ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=DEV)
    P = _lib.ptr
    _lib.check(L.mg_gemm_wgrad_pair(P(dy0), m0, P(x0), x0.stride(0), m0, n0, P(c0), n0, P(dy1), m1, P(x1),
                                    x1.stride(0), m1, n1, P(c1), n1, K, 1, P(ws), ws.numel(), _lib.stream_of(c0)),
               "mg_gemm_wgrad_pair")
    assert _rel(c0, base0.double() + a.double()) < 1e-6
    assert _rel(c1, base1.double() + b.double()) < 1e-6
    # deterministic: each product alone and unsplit, as mg_gemm's deterministic form
    d0, d1 = linear_dw_pair(dy0, x0, dy1, x1, deterministic=True)
    assert torch.equal(d0, linear_dw(dy0, x0, deterministic=True))
    assert torch.equal(d1, linear_dw(dy1, x1, deterministic=True))


def test_split_limbs_reconstructs_fp32_exactly():
    """mg_split_limbs: h + m + l == x for fp32 values over a wide range of magnitudes (the
    differences x - h and x - h - m are exact in fp32), each limb a bf16 value, in both
    segment layouts and for both patterns."""
    from gruboros_amd import gemm

    g = torch.Generator().manual_seed(5)
    x = torch.randn(64, 96, generator=g) * torch.exp2(torch.randint(-60, 60, (64, 96), generator=g).float())
    xd = x.to(DEV)
    for pattern, order in ((gemm.LIMBS_A, (0, 1, 0, 1, 2, 0)), (gemm.LIMBS_B, (0, 0, 1, 1, 0, 2))):
        side = gemm.split_limbs(xd, pattern, False).float().cpu().view(64, 6, 96)
        stack = gemm.split_limbs(xd, pattern, True).float().cpu().view(6, 64, 96)
        assert torch.equal(side.transpose(0, 1), stack)
        limbs = {}
        for s, which in enumerate(order):
            if which in limbs:
                assert torch.equal(limbs[which], stack[s])
            limbs[which] = stack[s]
        h, m, l = limbs[0], limbs[1], limbs[2]
        assert torch.equal(h, x.to(torch.bfloat16).float())
        assert torch.equal(h.double() + m.double() + l.double(), x.double())
    # four values per thread (cols % 8 != 0)
    y = torch.randn(5, 20, generator=g)
    side = gemm.split_limbs(y.to(DEV), gemm.LIMBS_B, False).float().cpu().view(5, 6, 20)
    assert torch.equal(side[:, 0] + side[:, 2] + side[:, 5], y)


@pytest.mark.parametrize("N,K,O,bias", [(4096, 512, 1024, False), (4092, 1024, 256, False), (37, 64, 200, True),
                                        (1000, 1536, 1024, True)])
def test_f32_linear_matches_fp64(N, K, O, bias):
    """F32Linear (the fp32 path's nn.Linear, reference mingru/minGRU.py:45,71 and minLM.py:17-23,
    :138 in fp32) against float64 for the output and the x, W and bias gradients: all three
    products on mg_gemm over three-limb bf16 splits, fp32-accurate (within 2e-6,
    norm-relative: an fp32 product's accumulation error at these K). N = 4092 and 37 put the
    weight gradient's reduction off a multiple of 8; (4096, 512, 1024) is cfg1's
    to_hidden_and_gate."""
    from gruboros_amd.linear import f32_linear

    g = torch.Generator().manual_seed(N + K + O)
    x = torch.randn(N, K, generator=g, dtype=torch.float64)
    w = torch.randn(O, K, generator=g, dtype=torch.float64) / K ** 0.5
    b = torch.randn(O, generator=g, dtype=torch.float64) if bias else None
    dy = torch.randn(N, O, generator=g, dtype=torch.float64)
    xd = x.float().to(DEV).requires_grad_(True)
    wd = w.float().to(DEV).requires_grad_(True)
    bd = b.float().to(DEV).requires_grad_(True) if bias else None
    y = f32_linear(xd, wd, bd)
    y.backward(dy.float().to(DEV))
    xr, wr = x.float().double().requires_grad_(True), w.float().double().requires_grad_(True)
    br = b.float().double().requires_grad_(True) if bias else None
    yr = torch.nn.functional.linear(xr, wr, br)
    yr.backward(dy.float().double())
    errs = {"y": _rel(y, yr), "dx": _rel(xd.grad, xr.grad), "dW": _rel(wd.grad, wr.grad)}
    if bias:
        errs["db"] = _rel(bd.grad, br.grad)
    print(f"f32_linear N={N} K={K} O={O}", {k: f"{v:.1e}" for k, v in errs.items()}, flush=True)
    assert all(v <= 2e-6 for v in errs.values()), errs


@pytest.mark.parametrize("M,N,K,hc", [(16376, 2048, 1024, 1024), (300, 520, 128, 256), (1000, 1536, 256, 512),
                                      (4, 264, 128, 256)])
def test_hilo_prefix_matches_the_two_products(M, N, K, hc):
    """mg_gemm_hilo_prefix (to_hidden_and_gate's forward in one launch, reference
    mingru/minGRU.py:45) equals the hi/lo product of its first hc columns and the plain
    product of the hi halves for the rest, bit for bit; and the hi/lo columns are
    fp32-accurate against float64. (16376, 2048, 1024, 1024) is the cfg3 layer."""
    from gruboros_amd import gemm

    g = torch.Generator(device=DEV).manual_seed(M + N + K)
    x = torch.randn(M, K, device=DEV, generator=g)
    w = torch.randn(N, K, device=DEV, generator=g) / K ** 0.5
    xp, wp = gemm.split_hilo(x), gemm.split_hilo(w)
    assert gemm.hilo_prefix_fits(xp, wp, K, hc)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    gemm.linear_fwd_hilo_prefix(xp, wp, out, K, hc)
    ref = torch.empty_like(out)
    gemm.linear_fwd_hilo(xp, wp[:hc], ref[:, :hc], K)
    gemm.gemm(xp[:, :K], gemm.KCONTIG, wp[hc:, :K], gemm.KCONTIG, M, N - hc, K, ref[:, hc:])
    assert torch.equal(out, ref)
    exact = (x.double() @ w.double().t())[:, :hc]
    assert _rel(out[:, :hc], exact) <= 2 ** -8
