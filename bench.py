"""Benchmark of the minGRU / minLM training hot path on one MI355X.

`python bench.py [--gpus 1] [--steps K] [--warmup W]` prints ONE JSON line:
  value      = minLM training tokens/sec (cfg3: vocab 256, dim 1024, depth 8,
               ff_mult 4, expansion 1.0, batch 8, seq 2048, bf16 activations,
               fp32 master weights, Schedule-Free AdamW step), counted as
               train.py:745 does (batch * chunk tokens per step).
  reference_loop = the same step in train.py:795-809's form (return_prev_hiddens,
               loss.detach().item() after the forward, loss / grad_accum).
  roofline   = the scan forward + backward on cfg2 (B16 T8192 H2048 bf16, the
               scan microbenchmark BASELINE.json names), HBM-bound; achieved =
               (6 + 12) B/element (algorithmic bytes) * 2^28 / the summed average
               launch times of the two kernels; forward and backward beside it.
  scan       = cfg2 forward, backward and forward+backward figures.
  cpu_baseline = the oracle's fp32 restatement of the reference step on the
               host's cores at the cfg3 shape (forward, backward, SF-AdamW step);
               cpu_baseline_scan = the oracle's cfg2 scan at batch 1, scaled x16.
Inputs are synthetic and already resident in HBM when the timed region starts.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
METRIC = "train tokens/sec (minLM d1024 L8 seq2048 bf16, 1 GPU); scan HBM GB/s vs peak"


def measured_traffic(kernel, path=os.path.join(ROOT, "profiles", "scan_cfg2_traffic.md")):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE
    summary (calibrated against a plain copy), or None."""
    try:
        for line in open(path):
            if line.startswith(f"traffic_bytes_per_launch {kernel}:"):
                return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def cfg3_matmul_params(dim=1024, depth=8, ff_mult=4, vocab=256, expansion=1.0):
    di = int(dim * expansion)
    f = int(dim * ff_mult)
    per_layer = 2 * di * dim + (dim * di if expansion != 1.0 else 0) + 2 * f * dim
    return depth * per_layer + vocab * dim


def bench_train(steps, warmup, B=8, S=2048, dim=1024, depth=8, accum=1, ref_loop=False):
    """One optimizer step = `accum` forward+backward micro-steps on [B, S] ids (the loss
    scaled by 1/accum as in train.py:798-800), then the Schedule-Free AdamW step.
    ref_loop: each micro-step as train.py:795-801 writes it: the model called with
    return_prev_hiddens=True, the loss read to the host (loss.detach().item(), one
    device sync per micro-step) before loss / grad_accum is backpropagated."""
    import torch

    from gruboros_amd.mingru.minLM import minLM
    from gruboros_amd.optim import AdamWScheduleFree

    torch.manual_seed(0)
    model = minLM(num_tokens=256, dim=dim, depth=depth, ff_mult=4, expansion=1.0,
                  compute_dtype=torch.bfloat16).cuda()
    opt = AdamWScheduleFree(model.parameters(), lr=1e-3, betas=(0.9, 0.999), weight_decay=0.01)
    opt.train()
    gen = torch.Generator(device="cuda").manual_seed(0)
    ids = [torch.randint(0, 256, (B, S), device="cuda", generator=gen) for _ in range(accum)]

    def step():
        for i in range(accum):
            loss = model(ids[i], return_loss=True)
            (loss / accum if accum > 1 else loss).backward()
        opt.step()
        opt.zero_grad(set_to_none=True)
        return loss

    if ref_loop:
        def step():  # noqa: F811
            for i in range(accum):
                loss, _hiddens = model(ids[i], return_loss=True, return_prev_hiddens=True, prev_hiddens=None)
                step.chunk_loss = loss.detach().item()
                (loss / accum).backward()
            opt.step()
            opt.zero_grad()
            return loss

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(steps):
        loss = step()
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = ev0.elapsed_time(ev1) / steps
    flops = 6.0 * cfg3_matmul_params(dim, depth) * B * (S - 1) * accum
    return {"ms_per_step": ms, "wall_s": wall, "tokens_per_step": B * S * accum, "loss": float(loss.detach()),
            "tflops": flops / (ms * 1e-3) / 1e12, "flops_per_step": flops,
            "params": sum(p.numel() for p in model.parameters())}


def bench_production_train(steps=3, warmup=2, chunks=8, S=2048):
    """The reference's production training run (train.cuda.sh:60-62: dim 1024, expansion 3.0,
    ff_mult 1.5, --params 1g -> depth 79; train.cuda.sh:71-73: grad_accum 8, chunk_size 2048,
    context_chunks 8; batch 1), as train.py:782-809 runs it: each optimizer step backpropagates
    8 consecutive [1, 2048] chunks of one sequence, the hiddens carried from chunk to chunk
    (detached), the loss scaled by 1 / grad_accum. Tokens counted as train.py:745 does
    (batch x chunk_size per chunk)."""
    import torch

    from gruboros_amd.mingru.minLM import minLM
    from gruboros_amd.optim import AdamWScheduleFree

    torch.manual_seed(0)
    dim, depth, expansion, ff_mult = 1024, 79, 3.0, 1.5
    model = minLM(num_tokens=256, dim=dim, depth=depth, ff_mult=ff_mult, expansion=expansion,
                  compute_dtype=torch.bfloat16).cuda()
    opt = AdamWScheduleFree(model.parameters(), lr=1e-3, betas=(0.9, 0.995), weight_decay=1e-4)
    opt.train()
    gen = torch.Generator(device="cuda").manual_seed(0)
    ids = [torch.randint(0, 256, (1, S), device="cuda", generator=gen) for _ in range(chunks)]

    def step():
        hid = None
        for i in range(chunks):
            loss, hid = model(ids[i], return_loss=True, return_prev_hiddens=True, prev_hiddens=hid)
            hid = [h.detach() for h in hid]
            (loss / chunks).backward()
        opt.step()
        opt.zero_grad(set_to_none=True)
        return loss

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        loss = step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / steps * 1e3
    tokens = chunks * S
    flops = 6.0 * cfg3_matmul_params(dim, depth, ff_mult=ff_mult, expansion=expansion) * tokens
    params = sum(p.numel() for p in model.parameters())
    del model, opt
    return {"workload": f"production run shape: minLM d{dim} L{depth} exp{expansion} ff{ff_mult} "
                        f"({params / 1e9:.2f} B params, bf16 compute), {chunks} chunks of [1, {S}] per optimizer "
                        "step, hiddens carried, SF-AdamW",
            "steps": steps, "warmup": warmup, "ms_per_step": ms, "tokens_per_s": tokens / (ms * 1e-3),
            "TFLOPs": flops / (ms * 1e-3) / 1e12, "frac_bf16_peak": flops / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS,
            "loss": float(loss.detach())}


def bench_scan(reps=20, B=16, T=8192, Di=2048):
    import torch

    from gruboros_amd.scan import _launch_bwd, _launch_fwd

    gen = torch.Generator(device="cuda").manual_seed(0)
    hidden = torch.randn(B, T, Di, device="cuda", generator=gen).to(torch.bfloat16)
    gate = torch.randn(B, T, Di, device="cuda", generator=gen).to(torch.bfloat16)
    x = torch.randn(B, 1, Di, device="cuda", generator=gen)
    h0 = torch.where(x >= 0, x + 0.5, x.sigmoid()).reshape(B, Di).contiguous()
    dh = torch.randn(B, T, Di, device="cuda", generator=gen).to(torch.bfloat16)
    dhid = torch.empty_like(hidden)
    dgat = torch.empty_like(gate)
    n = B * T * Di

    def fwd():
        return _launch_fwd(hidden, gate, h0, torch.bfloat16, need_ckpt=True)

    h, _, ckpt = fwd()

    def bwd():
        _launch_bwd(hidden, gate, h0, h, ckpt, dh, None, dhid, dgat, True)

    # ~30 ms of the same work first: the GPU clocks ramp up under sustained load
    for _ in range(30):
        fwd()
        bwd()
    torch.cuda.synchronize()
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(3 * reps)]
    for r in range(reps):
        evs[3 * r].record()
        fwd()
        evs[3 * r + 1].record()
        bwd()
        evs[3 * r + 2].record()
    torch.cuda.synchronize()
    tf = sum(evs[3 * r].elapsed_time(evs[3 * r + 1]) for r in range(reps)) / reps
    tb = sum(evs[3 * r + 1].elapsed_time(evs[3 * r + 2]) for r in range(reps)) / reps
    gbs = lambda nbytes, ms: nbytes / (ms * 1e-3) / 1e9  # noqa: E731
    return {
        "elements": n,
        "fwd_ms": tf, "bwd_ms": tb, "fwd_bwd_ms": tf + tb,
        "fwd_GBs": gbs(6 * n, tf), "bwd_GBs": gbs(12 * n, tb), "fwd_bwd_GBs": gbs(18 * n, tf + tb),
        "fwd_bwd_frac": gbs(18 * n, tf + tb) / HBM_PEAK_GBS,
        "note": "event times cover the scan kernels only (the look-back workspace is initialised once)",
    }


def _event_time(fn, reps):
    import torch

    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps  # ms


def bench_ceilings(n=1 << 28, reps=10):
    """Achievable HBM bandwidth of plain streaming kernels on the same box, as a
    yardstick for the scan's fraction of the datasheet peak: torch's copy
    (1 read, 1 write), add (2 reads, 1 write) and addcmul (3 reads, 1 write)
    over n bf16 elements per tensor (512 MiB each at the default n)."""
    import torch

    t = [torch.empty(n, dtype=torch.bfloat16, device="cuda").normal_() for _ in range(4)]
    a, b, c, o = t
    ops = {"copy_1r1w": (lambda: o.copy_(a), 2), "add_2r1w": (lambda: torch.add(a, b, out=o), 3),
           "addcmul_3r1w": (lambda: torch.addcmul(a, b, c, out=o), 4)}
    for _ in range(100):  # ~20 ms of copies first: the GPU clocks ramp up under sustained load
        o.copy_(a)
    res = {}
    for name, (fn, tensors) in ops.items():
        ms = _event_time(fn, reps)
        res[name + "_GBs"] = tensors * 2 * n / (ms * 1e-3) / 1e9
    res["peak_GBs"] = HBM_PEAK_GBS
    del t, a, b, c, o
    torch.cuda.empty_cache()
    return res


def bench_decode(steps=200, batches=(1, 8), dim=1024, depth=8, prompt=64, expansion=1.0, ff_mult=4, cast=False,
                 f32=False, f16=False):
    """Generation (reference generate.py:184-212): tokens/s of the per-token step,
    greedy sampling on the device, no host sync per token.
    `model_call`: the drop-in model called once per token as generate.py does (its
    one-token calls run on the decode kernels); `model_call_parallel_path`: the same
    with minLM.decode_kernels off (the parallel forward on one position);
    `decoder_graph`: gruboros_amd.decode.Decoder (decode kernels, one HIP graph
    replay per token). `weight_GBs`: bf16 weight bytes read per step / step time.
    cast: the model's parameters cast with .to(torch.bfloat16) as generate.py:140-141
    does; f32: the model kept in fp32 (generate.py --use-f32); f16: cast with
    .to(torch.float16) (--use-f32 --use-fp16); else fp32 masters with compute_dtype bf16. `weight_GBs` counts the weights at their stored width."""
    import torch

    from gruboros_amd.decode import Decoder
    from gruboros_amd.mingru.minLM import minLM

    torch.manual_seed(0)
    with torch.device("cuda"):
        model = minLM(num_tokens=256, dim=dim, depth=depth, ff_mult=ff_mult, expansion=expansion,
                      compute_dtype=None if (cast or f32 or f16) else torch.bfloat16).eval()
    if cast:
        model = model.to(torch.bfloat16)
    if f16:
        model = model.to(torch.float16)
    wbytes = (4 if f32 else 2) * sum(p.numel() for n, p in model.named_parameters()
                                     if p.dim() == 2 and "token_emb" not in n)
    res = {"model": f"minLM d{dim} L{depth} expansion {expansion} ff_mult {ff_mult} "
                    f"{'cast to bf16' if cast else 'fp32' if f32 else 'cast to fp16' if f16 else 'bf16 activations'}",
           "steps": steps, "weight_bytes_per_step": wbytes}
    gen = torch.Generator(device="cuda").manual_seed(0)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def timed(fn, tok, n):
        for _ in range(5):
            tok = fn(tok)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(n):
            tok = fn(tok)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n

    for B in batches:
        ids = torch.randint(0, 256, (B, prompt), device="cuda", generator=gen)
        row = {}
        with torch.no_grad():
            for key, on in (("model_call", True), ("model_call_parallel_path", False)):
                # the model called once per token, as reference generate.py does
                model.decode_kernels = on
                logits, hid = model(ids, return_prev_hiddens=True)
                state = {"hid": hid}

                def call(tok):
                    logits, state["hid"] = model(tok[:, None], return_prev_hiddens=True, prev_hiddens=state["hid"])
                    return logits[:, -1].argmax(-1)

                ms = timed(call, logits[:, -1].argmax(-1), steps if on else max(steps // 4, 10))
                row[key] = {"ms_per_token_step": ms, "tokens_per_s": B / (ms * 1e-3)}
            model.decode_kernels = True
            dec = Decoder(model, B)
            ms = timed(lambda tok: dec.step(tok).argmax(-1), dec.prefill(ids).argmax(-1), steps)
            row["decoder_graph"] = {"ms_per_token_step": ms, "tokens_per_s": B / (ms * 1e-3),
                                    "weight_GBs": wbytes / (ms * 1e-3) / 1e9}
        res[f"batch{B}"] = row
    del model
    torch.cuda.empty_cache()
    return res


def bench_cfg1(steps=50, warmup=5):
    """cfg1: one minGRU layer, dim 512, expansion 1.0, batch 4 x seq 1024,
    fp32 (the reference's precision: to_hidden_and_gate on mg_gemm over three-limb bf16 splits, the fp32 scan),
    x ~ N(0, 1), prev_hidden None; forward + backward of sum(out * dout) per step."""
    import torch

    from gruboros_amd.mingru.minGRU import minGRU

    torch.manual_seed(0)
    m = minGRU(512, 1.0).cuda()
    g = torch.Generator(device="cuda").manual_seed(0)
    x = torch.randn(4, 1024, 512, device="cuda", generator=g).requires_grad_(True)
    dout = torch.randn(4, 1024, 512, device="cuda", generator=g)

    def step():
        out = m(x)
        out.backward(dout)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    return {"workload": "cfg1 minGRU layer fp32 (dim 512, expansion 1.0, B4 T1024) forward + backward",
            "steps": steps, "ms_per_step": ms, "tokens_per_s": 4 * 1024 / (ms * 1e-3)}


def bench_kernels(reps=20, N=8 * 2047, D=1024, F=4096, V=256):
    """Per-kernel figures at the cfg3 shapes (16,376 token rows): HBM GB/s of
    the fused norm (algorithmic bytes: fwd 12, bwd 16 per element) and the
    streaming loss head, TFLOP/s of the hand-written MFMA products."""
    import torch

    from gruboros_amd import _lib, gemm
    from gruboros_amd.norm import FP32_EPS

    L = _lib.lib()
    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(0)
    out = {}
    x = torch.randn(N, D, device=dev, generator=g)
    delta = torch.randn(N, D, device=dev, generator=g).to(torch.bfloat16)
    w = torch.rand(D, device=dev, generator=g) + 0.5
    x_out = torch.empty_like(x)
    y = torch.empty(N, D, device=dev, dtype=torch.bfloat16)
    rstd = torch.empty(N, device=dev)
    st = _lib.stream_of(x)
    P = _lib.ptr

    def nf():
        _lib.check(L.mg_add_rmsnorm_fwd(P(x), 1, P(delta), P(w), P(x_out), 1, P(y), None, D, P(rstd), N, D,
                                        FP32_EPS, st))
    ms = _event_time(nf, reps)
    out["add_rmsnorm_fwd"] = {"us": ms * 1e3, "GBs": 12 * N * D / (ms * 1e-3) / 1e9}
    dy = torch.randn(N, D, device=dev, generator=g).to(torch.bfloat16)
    dres = torch.randn(N, D, device=dev, generator=g)
    dx = torch.empty_like(x)
    dd = torch.empty_like(delta)
    dw = torch.empty(D, device=dev)
    ws = torch.empty(L.mg_add_rmsnorm_bwd_workspace_bytes(N, D), dtype=torch.uint8, device=dev)

    def nb():
        _lib.check(L.mg_add_rmsnorm_bwd(P(x_out), P(w), P(rstd), 1, P(dy), P(dres), P(dx), 1, P(dd), P(dw), N, D,
                                        P(ws), ws.numel(), st))
    ms = _event_time(nb, reps)
    out["add_rmsnorm_bwd"] = {"us": ms * 1e3, "GBs": 16 * N * D / (ms * 1e-3) / 1e9}

    e = torch.randn(N, D, device=dev, generator=g).to(torch.bfloat16)
    wl = (torch.randn(V, D, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    lab = torch.randint(0, V, (N,), device=dev, generator=g)
    dl = torch.empty(N, V, device=dev, dtype=torch.bfloat16)
    part = torch.empty(L.mg_logits_cross_entropy_partials(N), device=dev)

    def ce():
        _lib.check(L.mg_logits_cross_entropy(P(e), D, P(wl), D, P(lab), P(dl), V, P(part), None, N, D, V, 1.0 / N, st))
    ms = _event_time(ce, reps)
    out["logits_cross_entropy"] = {"us": ms * 1e3, "GBs": (2 * N * D + 2 * V * D + 8 * N + 2 * N * V) / (ms * 1e-3) / 1e9,
                                   "TFLOPs": 2.0 * N * D * V / (ms * 1e-3) / 1e12}
    gemms = {}
    for name, fin, fout in (("to_hidden_and_gate", D, 2 * D), ("ff_in", D, F), ("ff_out", F, D)):
        xa = torch.randn(N, fin, device=dev, generator=g).to(torch.bfloat16)
        wa = (torch.randn(fout, fin, device=dev, generator=g) * 0.02).to(torch.bfloat16)
        da = torch.randn(N, fout, device=dev, generator=g).to(torch.bfloat16)
        fl = 2.0 * N * fin * fout
        for kind, fn in (("fwd", lambda: gemm.linear_fwd(xa, wa)), ("dx", lambda: gemm.linear_dx(da, wa)),
                         ("dw", lambda: gemm.linear_dw(da, xa))):
            ms = _event_time(fn, reps)
            gemms[f"{name}_{kind}"] = {"us": ms * 1e3, "TFLOPs": fl / (ms * 1e-3) / 1e12,
                                       "frac_bf16_peak": fl / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS}
        if name == "ff_in":  # the FeedForward's first product as the step runs it: bias + GELU epilogue
            ba = torch.randn(fout, device=dev, generator=g)
            pre = torch.empty(N, fout, device=dev, dtype=torch.bfloat16)
            ms = _event_time(lambda: gemm.linear_fwd(xa, wa, ba, gelu_pre=pre), reps)
            gemms["ff_in_fwd_bias_gelu"] = {"us": ms * 1e3, "TFLOPs": fl / (ms * 1e-3) / 1e12,
                                            "frac_bf16_peak": fl / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS}
    out["mfma_gemm"] = gemms
    return out


def _cpu_name():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown CPU"


def cpu_baseline(B=8, S=2048, dim=1024, depth=8, max_steps=2, seconds_budget=30.0):
    """The oracle's fp32 restatement of the reference step at the cfg3 shape on the
    host's cores: forward and autograd backward of mingru/minLM.py:86-155 (conv and
    dropout off), then the Schedule-Free AdamW step (oracle.sf_adamw, the package's
    update; train.py:808). One untimed warm-up step on a [1, 256] batch, then [B, S]
    steps (at least one, at most `max_steps`, and a second only when the first leaves
    room under `seconds_budget`); the median step time gives tokens/s. On the GPU
    box's 16 host cores a cfg3 step takes ~7.5 s (on an 8-core host ~2 min: pass a
    smaller B there; every op but the optimizer step is linear in the batch)."""
    import torch

    from oracle import mingru_oracle as O
    from oracle.sf_adamw import RefAdamWScheduleFree

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    sd = O.make_minlm_state(256, dim, depth, ff_mult=4, expansion=1.0, seed=0)
    params = {k: v.clone().requires_grad_(True) for k, v in sd.items()}
    opt = RefAdamWScheduleFree(list(params.values()), lr=1e-3, betas=(0.9, 0.999), weight_decay=0.01)
    gen = torch.Generator().manual_seed(0)

    def one(ids):
        loss, _ = O.minlm_forward(params, ids, depth, return_loss=True, dtype=torch.float32)
        loss.backward()
        opt.step([p.grad for p in params.values()])
        for p in params.values():
            p.grad = None

    one(torch.randint(0, 256, (1, 256), generator=gen))  # warm-up
    ids = torch.randint(0, 256, (B, S), generator=gen)
    times = []
    t_start = time.perf_counter()
    while not times or (len(times) < max_steps and time.perf_counter() - t_start + times[-1] < seconds_budget):
        t0 = time.perf_counter()
        one(ids)
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    return {"value": B * (S - 1) / med, "unit": "tokens/s", "cores": cores, "kind": "port",
            "s_per_step": med,
            "sample": f"cfg3 step (d{dim} L{depth} ff4 vocab 256), batch {B} x seq {S}: fp32 forward + backward + "
                      f"SF-AdamW step of the oracle restatement, median of {len(times)} full steps after a "
                      f"[1, 256] warm-up; torch CPU with {cores} threads on {_cpu_name()}"}


def cpu_baseline_scan(T=8192, Di=2048, B_full=16):
    """The oracle's restatement of the reference scan (mingru/minGRU.py:53-69, log-space
    Heinsen scan) forward + autograd backward in fp32 on the host's cores, at cfg2's
    shape with batch 1; the cfg2 figure (batch 16) is 16x its time."""
    import torch

    from oracle import mingru_oracle as O

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    gen = torch.Generator().manual_seed(0)
    hidden = torch.randn(1, T, Di, generator=gen).requires_grad_(True)
    gate = torch.randn(1, T, Di, generator=gen).requires_grad_(True)
    h0 = O.g(torch.randn(1, 1, Di, generator=gen))
    dh = torch.randn(1, T, Di, generator=gen)

    def one():
        out, _ = O.mingru_scan(hidden, gate, h0)
        out.backward(dh)
        hidden.grad = gate.grad = None

    one()  # warm-up
    t0 = time.perf_counter()
    one()
    dt = time.perf_counter() - t0
    n_full = B_full * T * Di
    t_full = dt * B_full
    return {"value": 18.0 * n_full / t_full / 1e9, "unit": "GB/s (cfg2 algorithmic bytes, 18 B/element)",
            "cores": cores, "kind": "port", "s_cfg2_fwd_bwd": t_full,
            "sample": f"oracle log-space scan fp32 forward + autograd backward at batch 1 x T {T} x H {Di} "
                      f"({dt:.2f} s), scaled x{B_full} to cfg2's batch; torch CPU with {cores} threads "
                      f"on {_cpu_name()}"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--scan-reps", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only", choices=["train", "scan", "kernels", "decode", "ceilings", "cfg1", "production"],
                    default=None)
    ap.add_argument("--workload", choices=["cfg3", "cfg5"], default="cfg3",
                    help="training workload for `value`: cfg3 (the BASELINE metric, default) or cfg5 "
                         "(~1B params: d2048 L24, batch 4 x seq 4096, gradient accumulation 4)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run a plain 1 GiB device copy (torch copy kernel): the known-size "
                         "reference for FETCH_SIZE/WRITE_SIZE counter scaling")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the minGRU hot path is built and "
              "measured on a single MI355X in this build.", file=sys.stderr)
        sys.exit(2)

    import torch

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    from gruboros_amd import _lib

    _lib.lib()
    print(f"[bench] device {torch.cuda.get_device_name(0)}", file=sys.stderr, flush=True)

    if args.copy_calibration:
        src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda").random_(0, 255)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
        print("[bench] copy calibration: 3 x 1 GiB device copies (1073741824 B read + written each)",
              file=sys.stderr, flush=True)

    train = ref = scan = kern = dec = ceil = None
    # The training step (`value`) runs first: after the decode phase's ~0.6 s
    # of light, latency-bound work the first training steps run ~25% slower
    # (measured: 14.9 vs 11.9 ms/step, back to 11.9 on a second run).
    if args.only in (None, "train"):
        if args.workload == "cfg5":
            train = bench_train(args.steps, args.warmup, B=4, S=4096, dim=2048, depth=24, accum=4)
        else:
            train = bench_train(args.steps, args.warmup)
        print(f"[bench] train {json.dumps(train)}", file=sys.stderr, flush=True)
        if args.workload == "cfg3":
            r = bench_train(args.steps, args.warmup, ref_loop=True)
            ref = {"ms_per_step": r["ms_per_step"], "value": r["tokens_per_step"] / (r["ms_per_step"] * 1e-3),
                   "unit": "tokens/s",
                   "form": "train.py:795-809: model(chunk, return_loss=True, return_prev_hiddens=True, "
                           "prev_hiddens=None); loss.detach().item(); (loss / grad_accum).backward(); "
                           "optimizer.step(); optimizer.zero_grad() (grad_accum 1)"}
            print(f"[bench] reference loop {json.dumps(ref)}", file=sys.stderr, flush=True)
    prod = None
    if args.only == "production" or (args.only is None and args.workload == "cfg3"):
        # before the decode phase, for the reason given above: this step is host-heavy (~22 k
        # launches) and measured 343-346 ms alone against 359-370 ms after the decode phase
        torch.cuda.empty_cache()
        prod = bench_production_train()
        print(f"[bench] production train {json.dumps(prod)}", file=sys.stderr, flush=True)
        torch.cuda.empty_cache()
    if args.only in (None, "ceilings"):
        ceil = bench_ceilings()
        print(f"[bench] ceilings {json.dumps(ceil)}", file=sys.stderr, flush=True)
    if args.only in (None, "scan"):
        scan = bench_scan(args.scan_reps)
        print(f"[bench] scan {json.dumps(scan)}", file=sys.stderr, flush=True)
    if args.only in (None, "kernels"):
        kern = bench_kernels()
        print(f"[bench] kernels {json.dumps(kern)}", file=sys.stderr, flush=True)
    if args.only in (None, "decode"):
        dec = bench_decode()
        print(f"[bench] decode {json.dumps(dec)}", file=sys.stderr, flush=True)
        # generate.py's own model at the reference's production run (train.cuda.sh:60-62:
        # dim 1024, expansion 3.0, ff_mult 1.5, --params 1g -> depth 79), cast to bf16
        dec_prod = bench_decode(steps=100, batches=(1, 8), dim=1024, depth=79, expansion=3.0, ff_mult=1.5,
                                cast=True)
        print(f"[bench] decode production {json.dumps(dec_prod)}", file=sys.stderr, flush=True)
        # the same model as generate.py --use-f32 leaves it (fp32, no cast), batch 1
        dec_prod32 = bench_decode(steps=50, batches=(1,), dim=1024, depth=79, expansion=3.0, ff_mult=1.5, f32=True)
        print(f"[bench] decode production fp32 {json.dumps(dec_prod32)}", file=sys.stderr, flush=True)
        dec_prod16 = bench_decode(steps=50, batches=(1,), dim=1024, depth=79, expansion=3.0, ff_mult=1.5, f16=True)
        print(f"[bench] decode production fp16 {json.dumps(dec_prod16)}", file=sys.stderr, flush=True)
    cfg1 = None
    if args.only in (None, "cfg1"):
        cfg1 = bench_cfg1()
        print(f"[bench] cfg1 {json.dumps(cfg1)}", file=sys.stderr, flush=True)
    cfg5 = None
    if args.only is None and args.workload == "cfg3":
        # the ~1B-parameter configuration beside the headline: a few optimizer
        # steps of 4 accumulated [4, 4096] micro-batches (d2048, L24)
        torch.cuda.empty_cache()
        t5 = bench_train(3, 1, B=4, S=4096, dim=2048, depth=24, accum=4)
        cfg5 = {"workload": "cfg5 minLM train step (vocab 256, d2048, L24, ff4, exp1.0, 4 x [4, 4096] micro-batches "
                            "accumulated, SF-AdamW)", "steps": 3, "warmup": 1,
                "ms_per_step": t5["ms_per_step"], "tokens_per_s": t5["tokens_per_step"] / (t5["ms_per_step"] * 1e-3),
                "TFLOPs": t5["tflops"], "frac_bf16_peak": t5["tflops"] / BF16_PEAK_TFLOPS}
        print(f"[bench] cfg5 {json.dumps(cfg5)}", file=sys.stderr, flush=True)
        torch.cuda.empty_cache()
    cpu = cpu_scan = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline()
        print(f"[bench] cpu {json.dumps(cpu)}", file=sys.stderr, flush=True)
        cpu_scan = cpu_baseline_scan()
        print(f"[bench] cpu scan {json.dumps(cpu_scan)}", file=sys.stderr, flush=True)

    out = {
        "metric": METRIC,
        "value": (train["tokens_per_step"] / (train["ms_per_step"] * 1e-3)) if train else None,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": train["ms_per_step"] if train else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (uniform random byte ids; random-init weights; scan inputs N(0,1))",
        "config": ({"workload": "cfg3 minLM train step (vocab 256, d1024, L8, ff4, exp1.0, B8, seq2048, "
                                "SF-AdamW) for value; cfg2 scan B16 T8192 H2048 bf16 forward+backward for roofline",
                    "global_batch": 8, "seq_len": 2048, "parallelism": "single GPU"}
                   if args.workload == "cfg3" else
                   {"workload": "cfg5 minLM train step (vocab 256, d2048, L24, ff4, exp1.0, B4, seq4096, "
                                "grad accum 4, SF-AdamW) for value; cfg2 scan for roofline",
                    "global_batch": 16, "seq_len": 4096, "parallelism": "single GPU"}),
    }
    if scan:
        fb_gbs = scan["fwd_bwd_GBs"]
        tf, tb = measured_traffic("scan_fwd_kernel"), measured_traffic("scan_bwd_kernel")
        out["roofline"] = {"kernel": "scan_fwd_kernel + scan_bwd_kernel <bf16,bf16> (cfg2)", "bound": "hbm",
                           "achieved": fb_gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": fb_gbs / HBM_PEAK_GBS,
                           "traffic": (tf + tb) if tf is not None and tb is not None else None,
                           "algorithmic_bytes": 18 * scan["elements"],
                           "forward": {"achieved": scan["fwd_GBs"], "frac": scan["fwd_GBs"] / HBM_PEAK_GBS,
                                       "us": scan["fwd_ms"] * 1e3, "algorithmic_bytes": 6 * scan["elements"],
                                       "traffic": tf},
                           "backward": {"achieved": scan["bwd_GBs"], "frac": scan["bwd_GBs"] / HBM_PEAK_GBS,
                                        "us": scan["bwd_ms"] * 1e3, "algorithmic_bytes": 12 * scan["elements"],
                                        "traffic": tb},
                           "note": "achieved = (6 + 12) B/element x 2^28 / (forward + backward mean launch time "
                                   "of the timed launches; HIP events on the launch stream, after ~30 ms of "
                                   "warm-up); traffic = calibrated FETCH_SIZE+WRITE_SIZE bytes per launch pair "
                                   "(profiles/scan_cfg2_traffic.md)"}
        out["scan"] = scan
    if train:
        out["step_roofline"] = {"bound": "mfma", "achieved": train["tflops"], "peak": BF16_PEAK_TFLOPS,
                                "unit": "TFLOP/s", "frac": train["tflops"] / BF16_PEAK_TFLOPS,
                                "flops_per_step": train["flops_per_step"]}
        out["tokens_per_s_predicted"] = train["tokens_per_step"] * (1 - 1 / (2048 if args.workload == "cfg3" else 4096)) \
            / (train["ms_per_step"] * 1e-3)
    if ceil:
        out["hbm_ceilings"] = ceil
    if kern:
        out["kernels"] = kern
    if dec:
        out["decode"] = dec
        out["decode_production"] = dec_prod
        out["decode_production_fp32"] = dec_prod32
        out["decode_production_fp16"] = dec_prod16
    if ref:
        out["reference_loop"] = ref
    if cfg1:
        out["cfg1"] = cfg1
    if cfg5:
        out["cfg5"] = cfg5
    if prod:
        out["production_train"] = prod
    if cpu:
        out["cpu_baseline"] = cpu
    if cpu_scan:
        out["cpu_baseline_scan"] = cpu_scan
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
