"""CPU/torch restatement of Schedule-Free AdamW — TEST INFRASTRUCTURE ONLY.

The reference steps schedulefree.AdamWScheduleFree (train.py:635, :642,
:808; package pinned at requirements.txt:44, commit d407c270, not available
offline). This restates the published algorithm (Defazio et al., 2024, "The
Road Less Scheduled") with plain torch tensor ops, one parameter at a time,
as the checker for the fused kernel (mg_sf_adamw_step).

Parity with the pinned package is UNPINNED: no vectors from the package
exist in the reference tree and the package cannot be imported here. What
the tests pin instead (tests/test_oracle_sf.py): both scalar schedules below
against hand-derived steps, the y-form update against Algorithm 1's
z/x/y recursion written out step by step, and the schedule-free identity
x = (y - (1 - b1) z) / b1 under train()/eval().

Two forms of the per-step scalars, over the same element-wise update:
  * "denominator" (the package's AdamWScheduleFree in its releases since
    late 2024, the form the build uses by default): v is bias-corrected in
    the denominator, sqrt(v / (1 - b2^t)) + eps, the learning rate is
    lr * warmup, and the average weights are lr_max^2 (uniform, c = 1/t, at
    a constant lr);
  * "lr" (Algorithm 1 of the paper, and the package's first releases):
    gamma_t = lr * warmup * sqrt(1 - b2^t) carries the bias correction, the
    denominator is sqrt(v) + eps, and c_{t+1} = gamma_t^2 / sum gamma_i^2.
"""
import math

import torch


def sf_scalars(k, lr, b1, b2, warmup_steps=0, r=0.0, weight_lr_power=2.0, lr_max=-1.0, weight_sum=0.0,
               form="denominator"):
    """Per-step scalars of step k (0-based): returns (bc2, lr_k, ckp1, y_lr, lr_max, weight_sum).
    bc2 is the denominator's bias correction (1.0 in the "lr" form, where lr_k carries it)."""
    sched = (k + 1) / warmup_steps if k < warmup_steps else 1.0
    bc2 = 1 - b2 ** (k + 1)
    lr_k = lr * sched
    if form == "lr":
        lr_k, bc2 = lr_k * math.sqrt(bc2), 1.0
    elif form != "denominator":
        raise ValueError(f"unknown form {form!r}")
    lr_max = max(lr_k, lr_max)
    weight = ((k + 1) ** r) * (lr_max ** weight_lr_power)
    weight_sum = weight_sum + weight
    ckp1 = weight / weight_sum if weight_sum != 0 else 0.0
    y_lr = lr_k * (b1 * (1 - ckp1) - 1)
    return bc2, lr_k, ckp1, y_lr, lr_max, weight_sum


def sf_update(y, g, z, v, b2, bc2, eps, wd, ckp1, y_lr, lr):
    """One element-wise update in float64 or float32 tensors; returns new (y, z, v)."""
    v = b2 * v + (1 - b2) * g * g
    u = g / ((v / bc2).sqrt() + eps) + wd * y
    y_new = (1 - ckp1) * y + ckp1 * z + y_lr * u
    z_new = z - lr * u
    return y_new, z_new, v


class RefAdamWScheduleFree:
    """Minimal per-tensor restatement used to check the fused optimizer."""

    def __init__(self, params, lr=0.0025, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0, warmup_steps=0,
                 form="denominator"):
        self.form = form
        self.params = list(params)
        self.lr, self.b1, self.b2, self.eps, self.wd, self.warm = lr, betas[0], betas[1], eps, weight_decay, warmup_steps
        self.k = 0
        self.lr_max = -1.0
        self.weight_sum = 0.0
        self.z = [p.detach().clone() for p in self.params]
        self.v = [torch.zeros_like(p) for p in self.params]

    @torch.no_grad()
    def step(self, grads):
        bc2, lr_k, ckp1, y_lr, self.lr_max, self.weight_sum = sf_scalars(
            self.k, self.lr, self.b1, self.b2, self.warm, lr_max=self.lr_max, weight_sum=self.weight_sum,
            form=self.form)
        for i, (p, g) in enumerate(zip(self.params, grads)):
            y, z, v = sf_update(p, g, self.z[i], self.v[i], self.b2, bc2, self.eps, self.wd, ckp1, y_lr, lr_k)
            p.copy_(y)
            self.z[i], self.v[i] = z, v
        self.k += 1
