"""GPU parity of the one-token decode path (gruboros_amd.decode.Decoder on
mg_decode_mingru / mg_decode_ff / mg_decode_head) for the generation loop of
reference generate.py:184-212.

Checks:
  * against the drop-in model's own one-token call on its parallel path
    (model(token, prev_hiddens=...) with the decode routing off, reference
    mingru/minLM.py:101-102 with minGRU's one-step path
    mingru/minGRU.py:47-52) step by step: logits and states;
  * against one parallel forward over prompt + generated tokens (T single
    steps equal one T-long scan);
  * the captured HIP graph replays exactly what the launches compute, also
    after the weights change.
Tolerances: bf16 activations, so relative (Frobenius) 1e-2 on logits and
states: the two paths sum the projections in different orders, and a bf16
rounding of a projection output can land on the other side.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-300))


def _model(dim=256, depth=2, seed=0, expansion=1.0, ff_mult=4):
    from gruboros_amd.mingru.minLM import minLM

    torch.manual_seed(seed)
    m = minLM(num_tokens=256, dim=dim, depth=depth, ff_mult=ff_mult, expansion=expansion,
              compute_dtype=torch.bfloat16)
    with torch.no_grad():
        for layer in m.layers:  # non-zero second FF (and to_out) weights so every block contributes
            layer[4][2].weight.normal_(0, 0.02)
            if expansion != 1.0:
                layer[2].to_out.weight.normal_(0, 1.0 / (layer[2].to_out.weight.shape[1] ** 0.5))
    return m.to(DEV).eval()


@pytest.mark.parametrize("B,dim", [(1, 256), (3, 256), (8, 256), (5, 1024), (8, 1024)])
def test_decoder_matches_one_token_model_calls(B, dim):
    """dim 1024 gives the FeedForward width 4096 of the cfg3 model (the
    second product stages its [B, 4096] input in more than one batch of loads)."""
    from gruboros_amd.decode import Decoder

    m = _model(dim=dim)
    m.decode_kernels = False  # the reference calls below run the parallel path
    gen = torch.Generator(device=DEV).manual_seed(B)
    prompt = torch.randint(0, 256, (B, 17), device=DEV, generator=gen)
    dec = Decoder(m, B)
    with torch.no_grad():
        logits, hid = m(prompt, return_prev_hiddens=True)
        last = dec.prefill(prompt)
        assert torch.equal(last, logits[:, -1])
        for step in range(6):
            tok = torch.randint(0, 256, (B,), device=DEV, generator=gen)
            logits, hid = m(tok[:, None], return_prev_hiddens=True, prev_hiddens=hid)
            got = dec.step(tok)
            e_l = _rel(got, logits[:, -1])
            e_h = max(_rel(a, b) for a, b in zip(dec.hiddens(), hid))
            print(f"B={B} dim={dim} step {step}: logits {e_l:.2e} states {e_h:.2e}", flush=True)
            assert e_l < 1e-2 and e_h < 1e-2


def test_decoder_equals_parallel_forward():
    from gruboros_amd.decode import Decoder

    B, P, N = 2, 9, 12
    m = _model(dim=512, depth=3, seed=1)
    gen = torch.Generator(device=DEV).manual_seed(5)
    seq = torch.randint(0, 256, (B, P + N), device=DEV, generator=gen)
    dec = Decoder(m, B)
    with torch.no_grad():
        full, hid = m(seq, return_prev_hiddens=True)
        dec.prefill(seq[:, :P])
        for t in range(P, P + N):
            got = dec.step(seq[:, t])
            assert _rel(got, full[:, t]) < 1e-2, t
        for a, b in zip(dec.hiddens(), hid):
            assert _rel(a, b) < 1e-2


def test_decoder_graph_replays_the_launches():
    from gruboros_amd.decode import Decoder

    B = 4
    m = _model(seed=2)
    gen = torch.Generator(device=DEV).manual_seed(3)
    prompt = torch.randint(0, 256, (B, 5), device=DEV, generator=gen)
    toks = [torch.randint(0, 256, (B,), device=DEV, generator=gen) for _ in range(5)]
    eager, graph = Decoder(m, B, graph=False), Decoder(m, B, graph=True)
    for d in (eager, graph):
        d.prefill(prompt)
    for i, t in enumerate(toks):
        if i == 3:  # weights changed in place (as a gossip merge or a checkpoint load does)
            with torch.no_grad():
                m.layers[0][2].to_hidden_and_gate.weight.mul_(0.5)
                m.to_logits.weight.add_(0.01)
        a = eager.step(t).clone()
        b = graph.step(t).clone()
        assert torch.equal(a, b), i
        for x, y in zip(eager.hiddens(), graph.hiddens()):
            assert torch.equal(x, y), i


@pytest.mark.parametrize("B", [1, 4])
def test_decoder_matches_fp64_oracle_cfg3_shape(B):
    """Decoder.prefill + Decoder.step at the cfg3 model shape (d1024 L8 ff4,
    expansion 1.0) against the fp64 restatement of the reference's generation
    calls (oracle.minlm_forward with return_loss=False: the prompt's parallel
    forward, then one token per call with prev_hiddens, reference
    generate.py:184-207, mingru/minLM.py:101-102, minGRU.py:47-52) on the same
    parameters: logits and per-layer states within 2e-2 (bf16 weights and
    activations against unrounded fp64) over 8 generated tokens."""
    from gruboros_amd.decode import Decoder
    from oracle import mingru_oracle as O

    m = _model(dim=1024, depth=8, seed=5)
    with torch.no_grad():
        for layer in m.layers:  # FF2 at a scale that keeps the blocks' outputs comparable
            layer[4][2].weight.normal_(0, 0.02 / 32)
    sd = {k: v.detach().cpu() for k, v in m.state_dict().items()}
    gen = torch.Generator(device=DEV).manual_seed(11 + B)
    prompt = torch.randint(0, 256, (B, 17), device=DEV, generator=gen)
    dec = Decoder(m, B)
    with torch.no_grad():
        last = dec.prefill(prompt)
        ref_logits, ref_hid = O.minlm_forward(sd, prompt.cpu(), 8, return_loss=False)
        assert _rel(last, ref_logits[:, -1]) < 2e-2
        for step in range(8):
            tok = torch.randint(0, 256, (B,), device=DEV, generator=gen)
            got = dec.step(tok)
            ref_logits, ref_hid = O.minlm_forward(sd, tok[:, None].cpu(), 8, return_loss=False, prev_hiddens=ref_hid)
            e_l = _rel(got, ref_logits[:, -1])
            e_h = max(_rel(a, b) for a, b in zip(dec.hiddens(), ref_hid))
            print(f"decode vs fp64 B={B} step {step}: logits {e_l:.2e} states {e_h:.2e}", flush=True)
            assert e_l < 2e-2 and e_h < 2e-2


def _against_oracle(m, B, steps, tag, tol=2e-2):
    """Decoder.prefill + Decoder.step against the fp64 restatement of the reference's
    generation calls on m's parameters (as m computes with them): logits and per-layer
    states within tol."""
    from gruboros_amd.decode import Decoder
    from oracle import mingru_oracle as O

    depth = len(m.layers)
    expansion = m.layers[0][2].to_hidden_and_gate.weight.shape[0] / (2 * m.dim)
    sd = {k: v.detach().double().cpu() for k, v in m.state_dict().items()}
    gen = torch.Generator(device=DEV).manual_seed(17 + B)
    prompt = torch.randint(0, 256, (B, 13), device=DEV, generator=gen)
    dec = Decoder(m, B)
    with torch.no_grad():
        last = dec.prefill(prompt)
        ref_logits, ref_hid = O.minlm_forward(sd, prompt.cpu(), depth, return_loss=False, expansion=expansion)
        assert _rel(last, ref_logits[:, -1]) < tol
        for step in range(steps):
            tok = torch.randint(0, 256, (B,), device=DEV, generator=gen)
            got = dec.step(tok)
            ref_logits, ref_hid = O.minlm_forward(sd, tok[:, None].cpu(), depth, return_loss=False,
                                                  prev_hiddens=ref_hid, expansion=expansion)
            e_l = _rel(got, ref_logits[:, -1])
            e_h = max(_rel(a, b) for a, b in zip(dec.hiddens(), ref_hid))
            print(f"{tag} B={B} step {step}: logits {e_l:.2e} states {e_h:.2e}", flush=True)
            assert e_l < tol and e_h < tol


@pytest.mark.parametrize("B", [1, 4])
@pytest.mark.parametrize("cast", [False, True], ids=["fp32_masters", "cast_bf16"])
def test_decoder_production_ratios_match_fp64_oracle(B, cast):
    """The reference's production widths (dim 1024, expansion 3.0, ff_mult 1.5:
    train.cuda.sh:60-62): Di 3072 through mg_decode_mingru_expanded and
    mg_decode_to_out, FeedForward 1536; a model with fp32 masters and
    compute_dtype bf16, and one cast with .to(torch.bfloat16) as
    generate.py:140-141 does (bf16 norm weights and embedding). Against the
    fp64 restatement (mingru/minGRU.py:45-52,69-71, minLM.py:97-138)."""
    m = _model(dim=1024, depth=3, seed=7, expansion=3.0, ff_mult=1.5)
    if cast:
        m = m.to(torch.bfloat16)
    _against_oracle(m, B, 6, f"exp3 ff1.5 cast={cast}")


def test_decoder_widest_feed_forward_at_batch_8():
    """FeedForward width 8192 at batch 8: the second product stages 8 x 8192 bf16
    (128 KiB) of input in LDS."""
    m = _model(dim=1024, depth=2, seed=8, ff_mult=8)
    with torch.no_grad():
        for layer in m.layers:
            layer[4][2].weight.normal_(0, 0.02 / 32)
    _against_oracle(m, 8, 4, "ff8192")


def test_model_calls_run_on_the_decoder():
    """minLM.forward's one-token calls under no_grad (generate.py:199-203) return what
    Decoder.step computes, bit for bit, with fresh hiddens per call; hiddens from
    elsewhere (another branch of the same prompt) are copied in."""
    from gruboros_amd import decode
    from gruboros_amd.decode import Decoder

    B = 2
    m = _model(dim=512, depth=3, seed=9, expansion=1.5, ff_mult=1.5)
    gen = torch.Generator(device=DEV).manual_seed(21)
    prompt = torch.randint(0, 256, (B, 7), device=DEV, generator=gen)
    toks = [torch.randint(0, 256, (B,), device=DEV, generator=gen) for _ in range(4)]
    dec = Decoder(m, B)
    with torch.no_grad():
        _, hid0 = m(prompt, return_prev_hiddens=True)
        dec.prefill(prompt)
        hid = hid0
        for t in toks:
            logits, hid = m(t[:, None], return_prev_hiddens=True, prev_hiddens=hid)
            ref = dec.step(t)
            assert logits.shape == (B, 1, 256) and torch.equal(logits[:, 0], ref)
            assert all(torch.equal(a.view(B, -1), b.view(B, -1)) for a, b in zip(hid, dec.hiddens()))
        # a branch from the prompt's hiddens again: copied in, same first-step result
        logits_b, _ = m(toks[0][:, None], return_prev_hiddens=True, prev_hiddens=hid0)
        dec.set_hiddens(hid0)
        assert torch.equal(logits_b[:, 0], dec.step(toks[0]))
    assert any(isinstance(d, Decoder) for d in decode._CACHE[m].values())
    with torch.enable_grad():  # a call that records gradients stays on the parallel path
        m(toks[0][:, None], prev_hiddens=hid0)
    assert sum(isinstance(d, Decoder) for d in decode._CACHE[m].values()) == 1


def test_decoder_follows_optimizer_steps():
    """A model's cached decoder (minLM.forward's one-token calls) sees the weights a fused
    SF-AdamW step changed through raw pointers (no version bump; the step keeps the bf16
    copies and hi/lo pairs current or drops them): after a training step, its logits equal a
    fresh Decoder's bit for bit, as does a parameter replaced by a new Parameter object."""
    from gruboros_amd.decode import Decoder
    from gruboros_amd.optim import AdamWScheduleFree

    B = 2
    m = _model(dim=256, depth=2, seed=12, expansion=1.5, ff_mult=1.5)
    opt = AdamWScheduleFree(m.parameters(), lr=1e-2)
    gen = torch.Generator(device=DEV).manual_seed(13)
    ids = torch.randint(0, 256, (B, 33), device=DEV, generator=gen)
    tok = torch.randint(0, 256, (B, 1), device=DEV, generator=gen)

    def one_token():
        with torch.no_grad():
            _, hid = m(ids[:, :8], return_prev_hiddens=True)
            logits, _ = m(tok, return_prev_hiddens=True, prev_hiddens=hid)
            fresh = Decoder(m, B)
            fresh.set_hiddens(hid)
            return logits[:, 0], fresh.step(tok[:, 0]).clone()

    for case in ("before", "after a step", "after another step"):
        if case != "before":
            m.train()
            opt.train()
            loss = m(ids, return_loss=True)
            loss.backward()
            opt.step()
            opt.zero_grad(set_to_none=True)
            m.eval()
            opt.eval()
        routed, fresh = one_token()
        print(f"case: {case}", flush=True)
        assert torch.equal(routed, fresh), case
    with torch.no_grad():
        w = m.layers[1][4][0].weight
        m.layers[1][4][0].weight = torch.nn.Parameter(w.detach() * 0.5)
    routed, fresh = one_token()
    assert torch.equal(routed, fresh), "replaced parameter"


def _model_f32(dim, depth, seed, expansion=1.0, ff_mult=4):
    """An fp32 minLM as generate.py --use-f32 leaves it (no cast, no compute_dtype)."""
    from gruboros_amd.mingru.minLM import minLM

    torch.manual_seed(seed)
    m = minLM(num_tokens=256, dim=dim, depth=depth, ff_mult=ff_mult, expansion=expansion)
    with torch.no_grad():
        for layer in m.layers:
            layer[4][2].weight.normal_(0, 0.02)
            if expansion != 1.0:
                layer[2].to_out.weight.normal_(0, 1.0 / (layer[2].to_out.weight.shape[1] ** 0.5))
    return m.to(DEV).eval()


@pytest.mark.parametrize("B,dim,expansion,ff_mult", [
    (1, 1024, 3.0, 1.5),   # generate.py --use-f32 at the production widths (Di 3072, F 1536)
    (4, 512, 1.0, 4),
    (8, 1024, 1.0, 4),     # F 4096: the longest fp32 staged row at batch 5-8
])
def test_decoder_fp32_model_matches_fp64_oracle(B, dim, expansion, ff_mult):
    """An fp32 model (reference generate.py:277 --use-f32) decodes on the *_f32 steps: fp32
    weights and activations, no rounding point. Against the fp64 restatement of the generation
    calls (generate.py:184-207, mingru/minLM.py:101-102, minGRU.py:47-52,69-71): logits and
    states within 1e-4 over 6 tokens (fp32 sums in another order)."""
    m = _model_f32(dim, 3, seed=40 + B, expansion=expansion, ff_mult=ff_mult)
    _against_oracle(m, B, 6, f"fp32 d{dim} exp{expansion} ff{ff_mult}", tol=1e-4)


def test_fp32_model_calls_run_on_the_decoder():
    """An fp32 model's one-token calls under no_grad route to the fp32 decode steps (their
    logits are fp32 and equal Decoder.step's bit for bit) and agree with the parallel path
    (minLM.decode_kernels off: the fp32-accurate three-limb products) within 1e-5."""
    from gruboros_amd.decode import Decoder

    B = 2
    m = _model_f32(512, 2, seed=51, expansion=1.5, ff_mult=1.5)
    gen = torch.Generator(device=DEV).manual_seed(52)
    prompt = torch.randint(0, 256, (B, 7), device=DEV, generator=gen)
    toks = [torch.randint(0, 256, (B,), device=DEV, generator=gen) for _ in range(3)]
    dec = Decoder(m, B)
    assert dec.f32
    with torch.no_grad():
        _, hid = m(prompt, return_prev_hiddens=True)
        dec.prefill(prompt)
        ref_hid = hid
        for t in toks:
            logits, hid = m(t[:, None], return_prev_hiddens=True, prev_hiddens=hid)
            assert logits.dtype == torch.float32
            assert torch.equal(logits[:, 0], dec.step(t))
            m.decode_kernels = False
            ref, ref_hid = m(t[:, None], return_prev_hiddens=True, prev_hiddens=ref_hid)
            m.decode_kernels = True
            e = _rel(logits, ref)
            print(f"fp32 routed vs parallel path: {e:.2e}", flush=True)
            assert e < 1e-5


@pytest.mark.parametrize("B,dim,expansion,ff_mult", [(1, 1024, 3.0, 1.5), (8, 512, 1.0, 4)])
def test_decoder_fp16_model_matches_fp64_oracle(B, dim, expansion, ff_mult):
    """A model cast with .to(torch.float16) (reference generate.py:143-144, --use-f32
    --use-fp16) decodes on the *_f16 steps (fp16 weights, the bf16 steps' rounding points at
    fp16). Against the fp64 restatement on the same (fp16-valued) parameters: logits and
    states within 1e-2 over 6 tokens."""
    m = _model_f32(dim, 3, seed=60 + B, expansion=expansion, ff_mult=ff_mult).half()
    _against_oracle(m, B, 6, f"fp16 d{dim} exp{expansion} ff{ff_mult}", tol=1e-2)


def test_fp16_model_calls_run_on_the_decoder():
    """A float16 model's one-token calls route to the fp16 steps: fp16 logits equal to
    Decoder.step's, and within 1e-2 of the model's own parallel path (its products in fp16,
    its kernels in fp32)."""
    from gruboros_amd.decode import Decoder

    B = 2
    m = _model_f32(512, 2, seed=61, expansion=1.5, ff_mult=1.5).half()
    gen = torch.Generator(device=DEV).manual_seed(62)
    prompt = torch.randint(0, 256, (B, 7), device=DEV, generator=gen)
    toks = [torch.randint(0, 256, (B,), device=DEV, generator=gen) for _ in range(3)]
    dec = Decoder(m, B)
    assert dec.kind == "f16"
    with torch.no_grad():
        _, hid = m(prompt, return_prev_hiddens=True)
        dec.prefill(prompt)
        ref_hid = hid
        for t in toks:
            logits, hid = m(t[:, None], return_prev_hiddens=True, prev_hiddens=hid)
            assert logits.dtype == torch.float16
            assert torch.equal(logits[:, 0], dec.step(t))
            m.decode_kernels = False
            ref, ref_hid = m(t[:, None], return_prev_hiddens=True, prev_hiddens=ref_hid)
            m.decode_kernels = True
            e = _rel(logits, ref)
            print(f"fp16 routed vs parallel path: {e:.2e}", flush=True)
            assert e < 1e-2
