"""Schedule-Free AdamW (Defazio et al., 2024, "The Road Less Scheduled").

The reference trains with `schedulefree.AdamWScheduleFree` pinned at commit
d407c270af9eced81c9107c14783a34268559769 (requirements.txt:44; constructed
at train.py:635 with lr, betas=(sf_beta, sf_beta2), weight_decay; put in
train mode at train.py:642; stepped at train.py:808). That package is not
available offline, so this is a restatement of the published algorithm;
its parity with the pinned package is unpinned.

Per parameter, p holds y (the gradient-evaluation point) in train mode;
state z is the base sequence and v the second moment. With step k (from 0),
c = weight_k / sum(weight), weight_k = (k+1)^r * lr_max^weight_lr_power:
    v   <- b2 v + (1 - b2) g^2
    u    = g / (sqrt(v / bc) + eps) + wd * y
    y   <- (1 - c) y + c z  +  lr_k (b1 (1 - c) - 1) u
    z   <- z - lr_k u
bias_correction selects the scalar schedule: "denominator" (default; the
package's releases since late 2024): bc = 1 - b2^(k+1), lr_k = lr * warmup;
"lr" (Algorithm 1 of the paper, the package's first releases): bc = 1,
lr_k = lr * warmup * sqrt(1 - b2^(k+1)), so the average weights follow
lr_k^2. The element-wise update is the same kernel either way.
eval() moves p to x = (y - (1 - b1) z) / b1 and train() moves it back,
exactly as the package's mode switch does.

step() runs the whole update as one mg_sf_adamw_step launch (all parameter
tensors, one pass over p, g, z, v), which also refreshes the bf16 copies of
the weights used by the bf16 linear layers (gruboros_amd.linear). Its tensor
table (pointers and sizes) goes to the device from two pinned host buffers
kept across steps, used in turn, so a step allocates no host memory.
"""
import torch

from . import scan as _scan
from ._lib import check, lib, require_cuda, stream_of


class _TableBuffers:
    """Pinned host rows for mg_sf_adamw_step's table, two buffers used in turn:
    a buffer is rewritten only after the copy that last read it has run.

    The rows are pointers and sizes, which repeat from step to step (the caching
    allocator hands the gradients the same blocks), so a table equal to the one
    last sent is not sent again: the kernel that reads it is queued behind that
    copy. A host-to-device copy in the step is not free even when small: in the
    cfg3 step profile the GPU sat idle ~0.33 ms before each one."""

    def __init__(self, rows, device):
        self.host = [torch.empty((rows, 8), dtype=torch.int64).pin_memory() for _ in range(2)]
        self.done = [None, None]
        self.dev = torch.empty((rows, 8), dtype=torch.int64, device=device)
        self.turn = 0
        self.sent = None  # the rows of the last copy into self.dev

    def upload(self, rows, stream):
        if rows == self.sent:
            return self.dev
        self.sent = [list(r) for r in rows]
        i = self.turn
        self.turn ^= 1
        if self.done[i] is not None:
            self.done[i].synchronize()
        n = len(rows)
        self.host[i][:n].copy_(torch.tensor(rows, dtype=torch.int64))
        self.dev[:n].copy_(self.host[i][:n], non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(stream)
        self.done[i] = ev
        return self.dev


class AdamWScheduleFree(torch.optim.Optimizer):
    def __init__(self, params, lr=0.0025, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0, warmup_steps=0,
                 r=0.0, weight_lr_power=2.0, bias_correction="denominator"):
        if bias_correction not in ("denominator", "lr"):
            raise ValueError(f"bias_correction must be 'denominator' or 'lr', got {bias_correction!r}")
        defaults = dict(lr=lr, betas=betas, eps=eps, weight_decay=weight_decay, warmup_steps=warmup_steps, r=r,
                        k=0, train_mode=False, weight_sum=0.0, lr_max=-1.0, weight_lr_power=weight_lr_power)
        super().__init__(params, defaults)
        self.bias_correction = bias_correction
        self._tables = {}

    @torch.no_grad()
    def eval(self):
        for group in self.param_groups:
            if group["train_mode"]:
                b1 = group["betas"][0]
                for p in group["params"]:
                    st = self.state[p]
                    if "z" in st:
                        p.lerp_(st["z"], 1 - 1 / b1)
                group["train_mode"] = False

    @torch.no_grad()
    def train(self):
        for group in self.param_groups:
            if not group["train_mode"]:
                b1 = group["betas"][0]
                for p in group["params"]:
                    st = self.state[p]
                    if "z" in st:
                        p.lerp_(st["z"], 1 - b1)
                group["train_mode"] = True

    @torch.no_grad()
    def step(self, closure=None):
        if not self.param_groups[0]["train_mode"]:
            raise RuntimeError("AdamWScheduleFree.step() called in eval mode; call optimizer.train() first")
        _scan.raise_pending_errors()  # a scan error reported by an earlier poll: do not apply its gradients
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        for group in self.param_groups:
            b1, b2 = group["betas"]
            k = group["k"]
            warm = group["warmup_steps"]
            sched = (k + 1) / warm if k < warm else 1.0
            bc2 = 1 - b2 ** (k + 1)
            lr = group["lr"] * sched
            if self.bias_correction == "lr":
                lr, bc2 = lr * bc2 ** 0.5, 1.0
            group["scheduled_lr"] = lr
            lr_max = group["lr_max"] = max(lr, group["lr_max"])
            weight = ((k + 1) ** group["r"]) * (lr_max ** group["weight_lr_power"])
            group["weight_sum"] = group["weight_sum"] + weight
            ckp1 = weight / group["weight_sum"] if group["weight_sum"] != 0 else 0.0
            y_lr = lr * (b1 * (1 - ckp1) - 1)
            rows, keep = [], []
            chunk = lib().mg_sf_adamw_chunk_elems()
            nchunks = 0
            for p in group["params"]:
                if p.grad is None:
                    continue
                require_cuda(p)
                if p.dtype != torch.float32 or not p.is_contiguous():
                    raise TypeError("AdamWScheduleFree: parameters must be contiguous float32")
                st = self.state[p]
                if "z" not in st:
                    st["z"] = p.detach().clone(memory_format=torch.preserve_format)
                    st["exp_avg_sq"] = torch.zeros_like(p, memory_format=torch.preserve_format)
                g = p.grad if (p.grad.is_contiguous() and p.grad.dtype == torch.float32) else \
                    p.grad.float().contiguous()
                keep.append(g)  # a converted copy must outlive the enqueue below
                pb, pair_cols = 0, 0
                pair = getattr(p, "_mg_pair", None)
                cache = getattr(p, "_mg_bf16", None)
                if pair is not None and pair[0] == p._version and p.dim() == 2 and p.shape[1] % 4 == 0 \
                        and p.numel() < (1 << 31) and pair[1].shape == (p.shape[0], 2 * p.shape[1]) \
                        and pair[1].is_contiguous():
                    # the kernel keeps the hi/lo pair (and with it the bf16 copy, its hi half) current
                    pb, pair_cols = pair[1].data_ptr(), p.shape[1]
                elif cache is not None and cache[0] == p._version and cache[1].shape == p.shape \
                        and cache[1].is_contiguous():
                    pb = cache[1].data_ptr()
                n = p.numel()
                rows.append([p.data_ptr(), g.data_ptr(), st["z"].data_ptr(), st["exp_avg_sq"].data_ptr(), pb, n,
                             nchunks, pair_cols])
                nchunks += (n + chunk - 1) // chunk
            if rows:
                dev = group["params"][0].device
                key = id(group)
                buf = self._tables.get(key)
                if buf is None or buf.dev.shape[0] < len(rows) or buf.dev.device != dev:
                    buf = self._tables[key] = _TableBuffers(len(group["params"]), dev)
                table = buf.upload(rows, torch.cuda.current_stream(dev))
                rc = lib().mg_sf_adamw_step(table.data_ptr(), len(rows), nchunks, b2, 1 - b2, bc2, group["eps"],
                                            group["weight_decay"], ckp1, y_lr, lr,
                                            stream_of(group["params"][0]))
                check(rc, "mg_sf_adamw_step")
                for p, row in zip([q for q in group["params"] if q.grad is not None], rows):
                    if row[7] == 0 and hasattr(p, "_mg_pair"):  # a pair the kernel did not update is re-made
                        del p._mg_pair
                    if row[7] != 0 and hasattr(p, "_mg_bf16"):  # and so is a dense copy beside a pair it did
                        del p._mg_bf16
            del keep
            group["k"] = k + 1
        if _scan._WORKSPACES:
            _scan.poll_workspaces()  # this step's backward scans, read at the next forward or step
        return loss
