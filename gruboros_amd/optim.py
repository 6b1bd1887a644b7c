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
    u    = g / (sqrt(v / (1 - b2^(k+1))) + eps) + wd * y
    y   <- (1 - c) y + c z  +  lr (b1 (1 - c) - 1) u
    z   <- z - lr u
eval() moves p to x = (y - (1 - b1) z) / b1 and train() moves it back,
exactly as the package's mode switch does.
"""
import torch


class AdamWScheduleFree(torch.optim.Optimizer):
    def __init__(self, params, lr=0.0025, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0, warmup_steps=0,
                 r=0.0, weight_lr_power=2.0):
        defaults = dict(lr=lr, betas=betas, eps=eps, weight_decay=weight_decay, warmup_steps=warmup_steps, r=r,
                        k=0, train_mode=False, weight_sum=0.0, lr_max=-1.0, weight_lr_power=weight_lr_power)
        super().__init__(params, defaults)

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
            group["scheduled_lr"] = lr
            lr_max = group["lr_max"] = max(lr, group["lr_max"])
            weight = ((k + 1) ** group["r"]) * (lr_max ** group["weight_lr_power"])
            group["weight_sum"] = group["weight_sum"] + weight
            ckp1 = weight / group["weight_sum"] if group["weight_sum"] != 0 else 0.0
            y_lr = lr * (b1 * (1 - ckp1) - 1)
            ps, gs, zs, vs = [], [], [], []
            for p in group["params"]:
                if p.grad is None:
                    continue
                st = self.state[p]
                if "z" not in st:
                    st["z"] = p.detach().clone(memory_format=torch.preserve_format)
                    st["exp_avg_sq"] = torch.zeros_like(p, memory_format=torch.preserve_format)
                ps.append(p)
                gs.append(p.grad)
                zs.append(st["z"])
                vs.append(st["exp_avg_sq"])
            if ps:
                torch._foreach_mul_(vs, b2)
                torch._foreach_addcmul_(vs, gs, gs, value=1 - b2)
                denom = torch._foreach_div(vs, bc2)
                torch._foreach_sqrt_(denom)
                torch._foreach_add_(denom, group["eps"])
                u = torch._foreach_div(gs, denom)
                if group["weight_decay"] != 0:
                    torch._foreach_add_(u, ps, alpha=group["weight_decay"])
                torch._foreach_lerp_(ps, zs, ckp1)
                torch._foreach_add_(ps, u, alpha=y_lr)
                torch._foreach_sub_(zs, u, alpha=lr)
            group["k"] = k + 1
        return loss
