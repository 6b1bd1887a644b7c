"""Host-side behaviour that needs no GPU: the seeded initialisation of the
drop-in minLM (reference mingru/minLM.py:157-206) and the `mingru` alias with
its default compute dtype."""
import math

import torch
from torch import nn


def _replay_reference_init(seed, num_tokens, dim, depth, ff_mult, expansion):
    """The draws reference minLM(...) makes from torch's global RNG after
    torch.manual_seed(seed), in its order, read from its source:
      construction (mingru/minLM.py:57-75; minGRU.py:38-41; FeedForward
      :17-23): nn.Embedding's N(0, 1); per layer the kaiming-uniform weights
      of to_hidden_and_gate and, for expansion != 1, to_out, then the
      FeedForward's Linear(dim, F) weight and bias and Linear(F, dim) weight
      and bias (nn.Linear.reset_parameters: kaiming_uniform_(a=sqrt 5), bias
      U(+-1/sqrt(fan_in))); to_logits' kaiming-uniform weight;
      then _initialize_weights (:157-206): N(0, std) for the embedding, the
      logits head, and per layer to_hidden_and_gate and FeedForward[0].weight
      (std = 0.02 / sqrt(dim)); zeros for to_out and FeedForward[2].
    Returns the expected state dict."""
    torch.manual_seed(seed)
    di, f = int(dim * expansion), int(dim * ff_mult)

    def lin(o, i, bias):
        w = torch.empty(o, i)
        nn.init.kaiming_uniform_(w, a=math.sqrt(5))
        b = None
        if bias:
            b = torch.empty(o).uniform_(-1 / math.sqrt(i), 1 / math.sqrt(i))
        return w, b

    sd = {"token_emb.weight": torch.empty(num_tokens, dim).normal_()}
    layers = []
    for _ in range(depth):
        hg, _ = lin(2 * di, dim, False)
        to = lin(dim, di, False)[0] if expansion != 1.0 else None
        w1, b1 = lin(f, dim, True)
        w2, b2 = lin(dim, f, True)
        layers.append((hg, to, w1, b1, w2, b2))
    logits, _ = lin(num_tokens, dim, False)
    std = 0.02 / math.sqrt(dim)
    sd["token_emb.weight"].normal_(0.0, std)
    logits.normal_(0.0, std)
    for i, (hg, to, w1, b1, w2, b2) in enumerate(layers):
        hg.normal_(0.0, std)
        w1.normal_(0.0, std)
        pre = f"layers.{i}."
        sd[pre + "1.weight"] = torch.ones(dim)
        sd[pre + "2.to_hidden_and_gate.weight"] = hg
        if to is not None:
            sd[pre + "2.to_out.weight"] = torch.zeros_like(to)
        sd[pre + "3.weight"] = torch.ones(dim)
        sd[pre + "4.0.weight"], sd[pre + "4.0.bias"] = w1, b1
        sd[pre + "4.2.weight"], sd[pre + "4.2.bias"] = torch.zeros_like(w2), torch.zeros_like(b2)
    sd["norm.weight"] = torch.ones(dim)
    sd["to_logits.weight"] = logits
    return sd


def test_seeded_init_replays_the_reference_draws():
    """minLM built after torch.manual_seed(s) holds, bit for bit, the values
    of the reference's draw sequence (for both expansion values, since
    to_out adds a draw), and two same-seed builds are identical."""
    from gruboros_amd.mingru.minLM import minLM

    for expansion in (1.0, 1.5):
        kw = dict(num_tokens=256, dim=96, depth=3, ff_mult=4, expansion=expansion)
        want = _replay_reference_init(7, **kw)
        torch.manual_seed(7)
        got = minLM(**kw).state_dict()
        assert list(got) == list(want)
        for k in want:
            assert torch.equal(got[k], want[k]), k
        torch.manual_seed(7)
        again = minLM(**kw).state_dict()
        assert all(torch.equal(again[k], got[k]) for k in got)


def test_seeded_init_moments():
    """The distributions of mingru/minLM.py:157-206 at a cfg3-like width:
    zeros for the second FeedForward linear and to_out, ones for the norms,
    N(0, 0.02/sqrt(D)) for the embedding, logits head, to_hidden_and_gate and
    the first FeedForward weight (mean and std within sampling error), the
    first FeedForward bias uniform in +-1/sqrt(D)."""
    from gruboros_amd.mingru.minLM import minLM

    D = 512
    torch.manual_seed(0)
    m = minLM(num_tokens=256, dim=D, depth=2, ff_mult=4, expansion=1.5)
    std = 0.02 / math.sqrt(D)
    for name, p in m.named_parameters():
        p = p.detach().double()
        if name.endswith(("4.2.weight", "4.2.bias", "to_out.weight")):
            assert bool((p == 0).all()), name
        elif name.endswith(("1.weight", "3.weight")) or name == "norm.weight":
            assert bool((p == 1).all()), name
        elif name.endswith("4.0.bias"):
            bound = 1 / math.sqrt(D)
            assert float(p.abs().max()) <= bound
            assert abs(float(p.std()) - bound / math.sqrt(3)) < 0.1 * bound / math.sqrt(3)
        else:
            n = p.numel()
            assert abs(float(p.mean())) < 5 * std / math.sqrt(n), name
            assert abs(float(p.std()) / std - 1) < 5 / math.sqrt(2 * n), name


def test_alias_and_default_compute_dtype():
    """install_alias makes `import mingru.minLM` resolve to the drop-in (the
    two import lines of reference train.py:26 / generate.py:19 then work
    unchanged) and compute_dtype sets the activation dtype of every minLM
    built without one."""
    import importlib
    import sys

    from gruboros_amd import mingru as pkg
    from gruboros_amd.mingru import _defaults

    saved = {k: sys.modules.get(k) for k in ("mingru", "mingru.minGRU", "mingru.minLM")}
    try:
        for k in saved:
            sys.modules.pop(k, None)
        pkg.install_alias(compute_dtype=torch.bfloat16)
        mod = importlib.import_module("mingru.minLM")
        from gruboros_amd.mingru import minLM as ours

        assert mod is ours and _defaults.COMPUTE_DTYPE == torch.bfloat16
    finally:
        pkg.set_default_compute_dtype(None)
        for k, v in saved.items():
            if v is None:
                sys.modules.pop(k, None)
            else:
                sys.modules[k] = v


def test_block_path_width_conditions():
    """The bf16 block path takes only widths every product and kernel of it
    takes (D, Di = D * expansion, F = D * ff_mult multiples of 8); other
    models go to the op-by-op path (checked on the GPU in
    test_widths_outside_the_block_path_train_on_the_op_path)."""
    from gruboros_amd import blocks
    from gruboros_amd.mingru.minLM import minLM

    def ok(dim, expansion, ff_mult=4):
        return blocks.supported(minLM(num_tokens=256, dim=dim, depth=1, ff_mult=ff_mult, expansion=expansion,
                                      compute_dtype=torch.bfloat16))

    assert ok(1024, 1.0) and ok(1024, 1.5) and ok(1000, 1.0)
    assert not ok(1000, 1.5)            # Di = 1500
    assert not ok(1024, 1.0, 4.001)     # F = 4097
    assert not ok(1004, 1.0)            # D = 1004


def test_build_refuses_spills_in_inline_assembly_kernels():
    """gruboros_amd.build reads hipcc's resource-usage remarks for gemm.hip and refuses a build
    in which a kernel with inline-assembly MFMAs spills registers (such a spill once gave
    wrong products); other kernels may spill."""
    from gruboros_amd.build import _spilled_kernels

    remarks = "\n".join([
        "gemm.hip:1:1: remark: Function Name: _ZN2mg4gemm23gemm_persist_w4m_kernelILb1ELb1ELi0ELb1EEEvNS0_6ParamsE",
        "gemm.hip:1:1: remark:     VGPRs Spill: 41",
        "gemm.hip:1:1: remark: Function Name: _ZN2mg4gemm11gemm_kernelILi256ELi256ELi2ELi4ELb1ELb0ELi0EfLi2EEEvNS0_6ParamsE",
        "gemm.hip:1:1: remark:     VGPRs Spill: 1",
        "gemm.hip:1:1: remark: Function Name: _ZN2mg4gemm16gemm_pair_kernelILi256ELi256ELi2ELi2ELb0ELb0EEEvNS0_6ParamsES2_",
        "gemm.hip:1:1: remark:     VGPRs Spill: 0",
    ])
    bad = _spilled_kernels(remarks)
    assert [n for _, n in bad] == [41] and "persist_w4m" in bad[0][0]


def test_decoder_applies_to_fp32_models_within_their_staged_limit():
    """gruboros_amd.decode.unsupported_reason (host logic only): an fp32 model (generate.py
    --use-f32) is served by the fp32 decode steps, whose staged rows are at most 4096 long at
    batch 5-8 (twice the LDS of bf16 rows); a float16 model (--use-fp16) by the fp16 steps; a
    float64 model stays on the parallel path."""
    import torch

    from gruboros_amd.decode import unsupported_reason
    from gruboros_amd.mingru.minLM import minLM

    m = minLM(num_tokens=256, dim=64, depth=1, ff_mult=64)  # FeedForward width 4096
    assert unsupported_reason(m, 8) is None
    m2 = minLM(num_tokens=256, dim=64, depth=1, ff_mult=128)  # 8192
    assert unsupported_reason(m2, 4) is None
    assert "4096" in unsupported_reason(m2, 8)
    assert unsupported_reason(m2.half(), 8) is None  # 16-bit rows: the full 8192
    assert "fp32 model" in unsupported_reason(m.double(), 1)
