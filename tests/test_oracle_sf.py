"""Pins the Schedule-Free AdamW restatement (oracle/sf_adamw.py) to the
paper's update written out by hand for single scalars, and to the
schedule-free interpolation identity. Parity with the pinned schedulefree
package itself is unpinned (not in the reference tree, not importable)."""
import math

import torch

from oracle import sf_adamw as S


def test_first_steps_by_hand():
    lr, b1, b2, eps, wd = 0.1, 0.9, 0.999, 1e-8, 0.01
    y0, g0, g1 = 0.5, 0.2, -0.3
    # step 0: c_1 = 1 (weight_sum = lr^2), y_lr = lr (b1 (1 - 1) - 1) = -lr
    bc2, lr_k, ckp1, y_lr, lr_max, wsum = S.sf_scalars(0, lr, b1, b2)
    assert math.isclose(ckp1, 1.0) and math.isclose(y_lr, -lr) and math.isclose(bc2, 1 - b2)
    v1 = (1 - b2) * g0 * g0
    u0 = g0 / (math.sqrt(v1 / (1 - b2)) + eps) + wd * y0
    z1 = y0 - lr * u0
    y1 = z1  # (1 - 1) y + 1 * z0 - lr u0 with z0 = y0
    y, z, v = S.sf_update(torch.tensor(y0, dtype=torch.float64), torch.tensor(g0, dtype=torch.float64),
                          torch.tensor(y0, dtype=torch.float64), torch.tensor(0.0, dtype=torch.float64),
                          b2, bc2, eps, wd, ckp1, y_lr, lr_k)
    assert math.isclose(float(y), y1, rel_tol=1e-12) and math.isclose(float(z), z1, rel_tol=1e-12)
    assert math.isclose(float(v), v1, rel_tol=1e-12)
    # step 1: c_2 = lr^2 / (2 lr^2) = 1/2
    bc2b, _, ckp1b, y_lrb, _, _ = S.sf_scalars(1, lr, b1, b2, lr_max=lr_max, weight_sum=wsum)
    assert math.isclose(ckp1b, 0.5) and math.isclose(y_lrb, lr * (b1 * 0.5 - 1))
    v2 = b2 * v1 + (1 - b2) * g1 * g1
    u1 = g1 / (math.sqrt(v2 / (1 - b2 ** 2)) + eps) + wd * y1
    y2 = 0.5 * y1 + 0.5 * z1 + y_lrb * u1
    z2 = z1 - lr * u1
    y, z, v = S.sf_update(y, torch.tensor(g1, dtype=torch.float64), z, v, b2, bc2b, eps, wd, ckp1b, y_lrb, lr)
    assert math.isclose(float(y), y2, rel_tol=1e-12) and math.isclose(float(z), z2, rel_tol=1e-12)


def test_warmup_schedule():
    _, lr_k, _, _, _, _ = S.sf_scalars(0, 1.0, 0.9, 0.999, warmup_steps=4)
    assert math.isclose(lr_k, 0.25)
    _, lr_k, _, _, _, _ = S.sf_scalars(5, 1.0, 0.9, 0.999, warmup_steps=4)
    assert lr_k == 1.0


def test_x_is_the_average_iterate():
    # with constant gradients the y/z/x sequences obey y = (1 - b1) z + b1 x
    torch.manual_seed(0)
    p = torch.randn(5, dtype=torch.float64)
    opt = S.RefAdamWScheduleFree([p], lr=0.01, betas=(0.9, 0.999))
    x = p.clone()  # x_1 = z_1 = y_1 initially
    g = torch.randn(5, dtype=torch.float64)
    for k in range(6):
        opt.step([g])
        c = 1.0 / (k + 1)  # uniform weights (r = 0, constant lr): step k averages with c = 1/(k+1)
        x = (1 - c) * x + c * opt.z[0]
        # the iterate p is y = (1 - b1) z + b1 x
    torch.testing.assert_close(p, (1 - 0.9) * opt.z[0] + 0.9 * x, rtol=1e-10, atol=1e-12)
