"""How far apart the two Schedule-Free AdamW scalar forms run — TEST/ANALYSIS ONLY.

Runs oracle.sf_adamw.RefAdamWScheduleFree in its "denominator" form (the
package's releases since late 2024; the build's default) and its "lr" form
(Algorithm 1 of Defazio et al. 2024) side by side, in float64, on the same
noisy quadratic, with train.py's defaults (train.py:453-461, :635: lr 1e-3,
betas (0.9, 0.999), weight decay 0.01, no warmup), and prints at chosen
steps: the two forms' learning rates gamma_t, their averaging weights
c_{t+1}, and the relative L2 distance between their y (the parameters the
model sees in train mode) and between their x (the averaged iterate eval()
exposes). The gradients are the same function of the parameters in both
runs (same seeds), so the distance is the forms' own divergence.

    python -m oracle.sf_forms_gap [--steps 1000] [--dim 65536]
"""
import argparse
import math

import torch

from .sf_adamw import RefAdamWScheduleFree, sf_scalars


def run(steps=1000, dim=65536, lr=1e-3, b1=0.9, b2=0.999, wd=0.01, noise=1.0, seed=0,
        report=(1, 10, 100, 300, 1000, 3000, 10000)):
    gen = torch.Generator().manual_seed(seed)
    curv = torch.exp(torch.empty(dim, dtype=torch.float64).uniform_(math.log(0.1), math.log(10.0), generator=gen))
    target = torch.randn(dim, dtype=torch.float64, generator=gen)
    w0 = torch.zeros(dim, dtype=torch.float64)
    opts, params = {}, {}
    for form in ("denominator", "lr"):
        params[form] = w0.clone()
        opts[form] = RefAdamWScheduleFree([params[form]], lr=lr, betas=(b1, b2), weight_decay=wd, form=form)
    rows = []
    scal = {f: dict(lr_max=-1.0, weight_sum=0.0) for f in opts}
    for k in range(steps):
        ngen = torch.Generator().manual_seed(seed * 1_000_003 + k)
        eps = torch.randn(dim, dtype=torch.float64, generator=ngen) * noise
        lrs, cs = {}, {}
        for form, opt in opts.items():
            _, lr_k, ckp1, _, scal[form]["lr_max"], scal[form]["weight_sum"] = sf_scalars(
                k, lr, b1, b2, lr_max=scal[form]["lr_max"], weight_sum=scal[form]["weight_sum"], form=form)
            lrs[form], cs[form] = lr_k, ckp1
            y = params[form]
            opt.step([curv * (y - target) + eps])
        if k + 1 in report:
            yd, yl = params["denominator"], params["lr"]
            xd = (yd - (1 - b1) * opts["denominator"].z[0]) / b1
            xl = (yl - (1 - b1) * opts["lr"].z[0]) / b1
            rows.append(dict(step=k + 1, lr_den=lrs["denominator"], lr_alg1=lrs["lr"], c_den=cs["denominator"],
                             c_alg1=cs["lr"],
                             y_gap=float((yd - yl).norm() / yd.norm()), x_gap=float((xd - xl).norm() / xd.norm()),
                             loss_den=float(0.5 * (curv * (xd - target) ** 2).mean()),
                             loss_alg1=float(0.5 * (curv * (xl - target) ** 2).mean())))
    return rows


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--dim", type=int, default=65536)
    args = ap.parse_args()
    print("| step | gamma (package) | gamma (Alg. 1) | c (package) | c (Alg. 1) | rel. gap y | rel. gap x | "
          "loss(x) package | loss(x) Alg. 1 |")
    print("|---:|---:|---:|---:|---:|---:|---:|---:|---:|")
    for r in run(args.steps, args.dim):
        print(f"| {r['step']} | {r['lr_den']:.3e} | {r['lr_alg1']:.3e} | {r['c_den']:.3e} | {r['c_alg1']:.3e} | "
              f"{r['y_gap']:.2e} | {r['x_gap']:.2e} | {r['loss_den']:.4f} | {r['loss_alg1']:.4f} |")


if __name__ == "__main__":
    main()
