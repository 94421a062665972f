"""Size-independent properties of the fused kernels at the configs[3] size (N = 5000,
C = 64, about 150k edges), beside the oracle comparisons on sampled destinations:
linearity in the features and in W, rotation equivariance (edge vectors rotated by R
and features by the Wigner matrices D(R), fitted from the oracle's SH), and invariance
under relabelling the atoms (the graph rebuilt from permuted positions).  Each holds
exactly in real arithmetic; the tolerance covers fp32 rounding (1e-5 normwise).
"""
import numpy as np
import pytest
import torch

from helpers import gen, normwise_err, periodic_box, random_rotation, wigner_d

pytestmark = pytest.mark.gpu
TOL = 1e-5


@pytest.fixture(scope="module")
def cfg3(dev):
    import batmobile
    pos, cell = periodic_box(5000, 3)
    g = batmobile.Graph(pos.to(dev), cell, 5.0, 64)
    x = torch.randn(5000, 64, 16, generator=gen(50)).to(dev)
    w = (torch.randn(34, 64, 64, generator=gen(51)) / 8.0).to(dev)
    return pos, cell, g, x, w


def _rotate_features(x, d):
    return (x.reshape(-1, 16) @ d.T).reshape(x.shape)


@pytest.mark.parametrize("weighted", [False, True])
def test_linear_in_features(cfg3, weighted):
    _, _, g, x, w = cfg3
    x2 = torch.randn(x.shape, generator=gen(52)).to(x.device)
    kw = {"weights": w} if weighted else {}
    lhs = g.sh_tp_scatter(0.75 * x - 1.5 * x2, **kw)
    rhs = 0.75 * g.sh_tp_scatter(x, **kw) - 1.5 * g.sh_tp_scatter(x2, **kw)
    assert normwise_err(lhs.cpu(), rhs.cpu()) <= TOL


def test_weighted_linear_in_weights(cfg3):
    _, _, g, x, w = cfg3
    w2 = (torch.randn(w.shape, generator=gen(53)) / 8.0).to(w.device)
    lhs = g.sh_tp_scatter(x, weights=w + 2.0 * w2)
    rhs = g.sh_tp_scatter(x, weights=w) + 2.0 * g.sh_tp_scatter(x, weights=w2)
    assert normwise_err(lhs.cpu(), rhs.cpu()) <= TOL


@pytest.mark.parametrize("weighted", [False, True])
def test_rotation_equivariance(cfg3, weighted):
    """out(R v, D x) = D out(v, x): the kernels are SO(3)-equivariant at full size."""
    _, _, g, x, w = cfg3
    rot = random_rotation(5)
    d = torch.tensor(wigner_d(rot), dtype=torch.float32, device=x.device)
    kw = {"weights": w} if weighted else {}
    out = g.sh_tp_scatter(x, **kw)
    vec0 = g.vec
    try:
        g.vec = (vec0 @ torch.tensor(rot.T, dtype=torch.float32, device=x.device)).contiguous()
        out_r = g.sh_tp_scatter(_rotate_features(x, d), **kw)
    finally:
        g.vec = vec0
    assert normwise_err(out_r.cpu(), _rotate_features(out, d).cpu()) <= TOL


def test_rotation_test_catches_a_wrong_matrix(cfg3):
    """The same comparison with D of another rotation fails (the test is not vacuous)."""
    _, _, g, x, _ = cfg3
    rot = random_rotation(5)
    d = torch.tensor(wigner_d(rot), dtype=torch.float32, device=x.device)
    d_wrong = torch.tensor(wigner_d(random_rotation(6)), dtype=torch.float32, device=x.device)
    out = g.sh_tp_scatter(x)
    vec0 = g.vec
    try:
        g.vec = (vec0 @ torch.tensor(rot.T, dtype=torch.float32, device=x.device)).contiguous()
        out_r = g.sh_tp_scatter(_rotate_features(x, d))
    finally:
        g.vec = vec0
    assert normwise_err(out_r.cpu(), _rotate_features(out, d_wrong).cpu()) > 1e-2


@pytest.mark.parametrize("weighted", [False, True])
def test_invariant_under_relabelled_atoms(cfg3, dev, weighted):
    """The graph rebuilt from permuted positions gives the permuted output: the neighbor
    list, the schedule and the kernel agree on the physics, whatever the atom labels."""
    import batmobile
    pos, cell, g, x, w = cfg3
    perm = torch.randperm(5000, generator=gen(54))
    g2 = batmobile.Graph(pos[perm].to(dev), cell, 5.0, 64)
    assert g2.num_edges == g.num_edges
    kw = {"weights": w} if weighted else {}
    out = g.sh_tp_scatter(x, **kw)
    out2 = g2.sh_tp_scatter(x[perm.to(dev)], **kw)
    assert normwise_err(out2.cpu(), out[perm.to(dev)].cpu()) <= TOL
