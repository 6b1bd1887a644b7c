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


def _algorithm1(p0, grads, lr, b1, b2, eps, wd, warmup=0):
    """Algorithm 1 of Defazio et al. (2024), "The Road Less Scheduled", for one
    scalar, written out as the paper states it (x, z, y sequences, t from 1):
      y_t = (1 - b1) z_t + b1 x_t;  g_t = grad at y_t
      v_t = b2 v_{t-1} + (1 - b2) g_t^2
      gamma_t = lr sqrt(1 - b2^t) min(1, t / warmup)
      z_{t+1} = z_t - gamma_t g_t / (sqrt(v_t) + eps) - gamma_t wd y_t
      c_{t+1} = gamma_t^2 / sum_{i <= t} gamma_i^2
      x_{t+1} = (1 - c_{t+1}) x_t + c_{t+1} z_{t+1}
    grads: callable y -> gradient. Returns the list of y_{t+1}."""
    x = z = p0
    v = 0.0
    gsum = 0.0
    ys = []
    for t in range(1, len(grads) + 1):
        y = (1 - b1) * z + b1 * x
        g = grads[t - 1](y)
        v = b2 * v + (1 - b2) * g * g
        gamma = lr * math.sqrt(1 - b2 ** t) * (min(1.0, t / warmup) if warmup else 1.0)
        z = z - gamma * g / (math.sqrt(v) + eps) - gamma * wd * y
        gsum += gamma * gamma
        c = gamma * gamma / gsum
        x = (1 - c) * x + c * z
        ys.append((1 - b1) * z + b1 * x)
    return ys


def test_paper_algorithm1_three_steps_by_hand():
    """The restatement's "lr" form equals Algorithm 1 step by step. The
    gradients depend on the point y (g = 3 y - 1 + a step constant), so a
    wrong evaluation point, a dropped weight-decay term, a wrong c or a wrong
    bias correction changes the sequence. The first step is also checked
    against its value derived by hand: v_1 = (1 - b2) g_1^2 and c_2 = 1, so
    y_2 = z_2 = p0 - gamma_1 (g_1 / (sqrt(1 - b2) |g_1| + eps) + wd p0) with
    gamma_1 = lr sqrt(1 - b2), i.e. about p0 - lr (sign(g_1) + sqrt(1 - b2) wd p0)."""
    lr, b1, b2, eps, wd = 0.05, 0.9, 0.999, 1e-8, 0.1
    p0 = 0.7
    grads = [lambda y: 3 * y - 1, lambda y: 3 * y - 0.5, lambda y: -2 * y + 0.25]
    ys = _algorithm1(p0, grads, lr, b1, b2, eps, wd)
    g1 = 3 * p0 - 1
    y2 = p0 - lr * math.sqrt(1 - b2) * (g1 / (math.sqrt(1 - b2) * abs(g1) + eps) + wd * p0)
    assert math.isclose(ys[0], y2, rel_tol=1e-14)
    # restatement, one tensor, "lr" form
    p = torch.tensor([p0], dtype=torch.float64)
    opt = S.RefAdamWScheduleFree([p], lr=lr, betas=(b1, b2), eps=eps, weight_decay=wd, form="lr")
    for t, grad in enumerate(grads):
        opt.step([torch.tensor([grad(float(p))], dtype=torch.float64)])
        assert math.isclose(float(p), ys[t], rel_tol=1e-12), (t, float(p), ys[t])
    # the averaging weights of the "lr" form are gamma_t^2: c_3 = (1 - b2^2) / ((1 - b2) + (1 - b2^2))
    _, _, c2, _, lm, ws = S.sf_scalars(0, lr, b1, b2, form="lr")
    _, _, c3, _, _, _ = S.sf_scalars(1, lr, b1, b2, lr_max=lm, weight_sum=ws, form="lr")
    assert math.isclose(c2, 1.0) and math.isclose(c3, (1 - b2 ** 2) / ((1 - b2) + (1 - b2 ** 2)), rel_tol=1e-12)


def test_package_form_differs_from_algorithm1():
    """The default ("denominator") form is not Algorithm 1: after the first
    step they part (uniform c = 1/2 against gamma-weighted c, and the eps
    term scaled differently), so the pin above would catch a silent switch."""
    lr, b1, b2, eps, wd = 0.05, 0.9, 0.999, 1e-8, 0.1
    grads = [lambda y: 3 * y - 1, lambda y: 3 * y - 0.5, lambda y: -2 * y + 0.25]
    ys = _algorithm1(0.7, grads, lr, b1, b2, eps, wd)
    p = torch.tensor([0.7], dtype=torch.float64)
    opt = S.RefAdamWScheduleFree([p], lr=lr, betas=(b1, b2), eps=eps, weight_decay=wd, form="denominator")
    got = []
    for grad in grads:
        opt.step([torch.tensor([grad(float(p))], dtype=torch.float64)])
        got.append(float(p))
    assert abs(got[2] - ys[2]) > 1e-4
