"""Pins the layer definition of oracle/mace.py (CPU; no GPU)."""
import math

import numpy as np
import torch

from oracle import mace as om
from oracle import tp as otp

from helpers import gen


def test_envelope_values_and_smooth_cutoff():
    d = torch.tensor([0.0, 0.5, 1.0 - 1e-12, 1.0, 1.5], dtype=torch.float64, requires_grad=True)
    f = om.envelope(d, xp=torch)
    assert f[0].item() == 1.0 and f[3].item() == 0.0 and f[4].item() == 0.0
    # f(1) = 0 with vanishing first and second derivatives (p = 6 envelope)
    (g,) = torch.autograd.grad(f.sum(), d, create_graph=True)
    (h,) = torch.autograd.grad(g[2], d)
    assert abs(f[2].item()) < 1e-9 and abs(g[2].item()) < 1e-8 and abs(h[2].item()) < 1e-6
    x = np.linspace(0, 1, 1001)
    assert np.all(np.diff(om.envelope(x)) <= 1e-15)   # monotone on [0, 1]


def test_bessel_basis_is_orthonormal_with_weight_r2():
    rc = 5.0
    r = np.linspace(1e-6, rc, 200001)
    b = om.bessel_bare(r, rc)
    gram = np.trapezoid(b[:, :, None] * b[:, None, :] * (r * r)[:, None, None], r, axis=0)
    np.testing.assert_allclose(gram, np.eye(om.N_BASIS), atol=1e-6)


def test_unit_weights_reduce_to_the_simple_product():
    e, c = 40, 3
    xs = torch.randn(e, c, 16, generator=gen(3), dtype=torch.float64)
    y = torch.randn(e, 16, generator=gen(4), dtype=torch.float64)
    m = om.channelwise_tp(xs, y, torch.ones(e, c, om.NUM_PATHS, dtype=torch.float64))
    for ch in range(c):
        np.testing.assert_allclose(m[:, ch].numpy(),
                                   otp.tensor_product_simple(xs[:, ch].numpy(), y.numpy()),
                                   rtol=1e-12, atol=1e-12)
    # a single path weight selects that path (its l_out block only)
    r1 = torch.zeros(e, c, om.NUM_PATHS, dtype=torch.float64)
    r1[:, :, 0] = 1.0   # path (0, 0, 0): out[0] = x[0] y[0]
    m1 = om.channelwise_tp(xs, y, r1)
    np.testing.assert_allclose(m1[:, :, 0].numpy(), (xs[:, :, 0] * y[:, None, 0]).numpy(), atol=1e-12)
    assert torch.count_nonzero(m1[:, :, 1:]).item() == 0


def _tiny_system(n=8, c=2, seed=5):
    g = gen(seed)
    box = np.array([7.0, 7.5, 8.0])
    pos = torch.rand(n, 3, generator=g, dtype=torch.float64) * torch.as_tensor(box)
    src, dst = [], []
    for i in range(n):
        for j in range(n):
            if i != j:
                src.append(j)
                dst.append(i)
    x = torch.randn(n, c, 16, generator=g, dtype=torch.float64)
    w1 = torch.randn(8, 64, generator=g, dtype=torch.float64) / math.sqrt(8)
    b1 = torch.randn(64, generator=g, dtype=torch.float64) * 0.1
    w2 = torch.randn(64, 34 * c, generator=g, dtype=torch.float64) / 8.0
    go = torch.randn(n, c, 16, generator=g, dtype=torch.float64)
    return pos, box, x, np.array(src), np.array(dst), w1, b1, w2, go


def test_position_gradient_matches_finite_differences_and_is_translation_invariant():
    pos, box, x, src, dst, w1, b1, w2, go = _tiny_system()
    rc = 6.0
    out, grad = om.layer_and_position_grad(pos, box, x, src, dst, w1, b1, w2, rc, go)
    s_t, d_t = torch.as_tensor(src), torch.as_tensor(dst)

    def energy(p):
        return float((om.layer(p, box, x, s_t, d_t, w1, b1, w2, rc) * go).sum())

    h = 1e-6
    for a in range(pos.shape[0]):
        for k in range(3):
            dp = pos.clone()
            dp[a, k] += h
            dm = pos.clone()
            dm[a, k] -= h
            fd = (energy(dp) - energy(dm)) / (2 * h)
            assert abs(fd - grad[a, k]) <= 1e-6 * max(1.0, abs(fd))
    np.testing.assert_allclose(grad.sum(axis=0), 0.0, atol=1e-9 * np.abs(grad).sum())
