"""GPU parity on raw (non-unit) edge vectors.

The reference evaluates the SH polynomials on the vectors as given
(src/spherical_harmonics/spherical_harmonics.cu:50-96; the fused kernels,
src/message_passing/fused_sh_tp.cu:88-94 and fused_message_passing.cu:222-227,
335-340, likewise): Y_l is homogeneous of degree l in v.  Every entry point that
does not normalise is checked here on vectors of length 0.2 .. 5 against the
float64 oracle, which evaluates on the given vector; a kernel that normalised
inside would be off by |v|^l.

Tolerances: SH forward 1e-5 normwise per l block (the blocks scale as |v|^l);
gradients 1e-4 normwise; fused products and scatters 1e-5 normwise.
"""
import json
import os

import numpy as np
import pytest
import torch

from helpers import gen, normwise_err, periodic_box
from oracle import mp as omp
from oracle import sh as osh

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def raw_vectors(n, seed, lo=0.2, hi=5.0):
    v = torch.randn(n, 3, generator=gen(seed))
    v = v / v.norm(dim=1, keepdim=True)
    return v * (lo + (hi - lo) * torch.rand(n, 1, generator=gen(seed + 1)))


def _per_l_block_err(got, want, lmax):
    return max(normwise_err(got[:, l * l:(l + 1) ** 2], want[:, l * l:(l + 1) ** 2])
               for l in range(lmax + 1))


@pytest.mark.parametrize("lmax", range(7))
def test_sh_forward_raw_vectors(bm, dev, lmax):
    v = raw_vectors(20000, 61)
    y = bm.spherical_harmonics(v.to(dev), lmax).cpu().numpy()
    want = osh.spherical_harmonics(v.double().numpy(), lmax)
    assert _per_l_block_err(y, want, lmax) <= 1e-5
    # homogeneity: the l block of 2v is 2^l times that of v (exact in fp32 up to rounding)
    y2 = bm.spherical_harmonics((2.0 * v).to(dev), lmax).cpu().numpy()
    for l in range(lmax + 1):
        b = slice(l * l, (l + 1) ** 2)
        assert normwise_err(y2[:, b], (2.0 ** l) * y[:, b].astype(np.float64)) <= 1e-5


@pytest.mark.parametrize("lmax", [3, 6])
def test_sh_known_inputs_as_given(bm, dev, lmax):
    """The reference's near-pole list passed in without normalising, and the axis and
    diagonal lists scaled by 2.5 (tests/test_spherical_harmonics.py:55-99)."""
    inp = json.load(open(os.path.join(GOLDEN, "sh_known_inputs.json")))
    for key, scale in (("near_pole_unnormalised", 1.0), ("axis", 2.5), ("diagonal", 2.5)):
        v = torch.tensor(inp[key], dtype=torch.float32) * scale
        y = bm.spherical_harmonics(v.to(dev), lmax).cpu().numpy()
        want = osh.spherical_harmonics(v.double().numpy(), lmax)
        assert _per_l_block_err(y, want, lmax) <= 1e-5, key


@pytest.mark.parametrize("lmax", range(7))
def test_sh_backward_raw_vectors(bm, dev, lmax):
    v = raw_vectors(6000, 63)
    g = torch.randn(6000, (lmax + 1) ** 2, generator=gen(65))
    got = bm.spherical_harmonics_backward(v.to(dev), g.to(dev)).cpu().numpy()
    want = osh.spherical_harmonics_backward(v.double().numpy(), g.double().numpy())
    assert normwise_err(got, want) <= 1e-4


@pytest.mark.parametrize("n,e,c", [(100, 3000, 16), (40, 500, 64), (9, 70, 5)])
def test_fused_sh_tp_simple_raw_vectors(bm, dev, n, e, c):
    vec = raw_vectors(e, 71)
    x = torch.randn(n, c, 16, generator=gen(73))
    src = torch.randint(0, n, (e,), generator=gen(74))
    msg = bm.fused_sh_tp_simple(vec.to(dev), x.to(dev), src.to(dev)).cpu().numpy()
    want = omp.fused_sh_tp_simple(vec.double().numpy(), x.double().numpy(), src.numpy())
    assert normwise_err(msg, want) <= 1e-5
    # edge by edge, so that short vectors are checked too
    per_edge = np.abs(msg - want).max(axis=(1, 2)) / np.abs(want).max(axis=(1, 2))
    assert per_edge.max() <= 1e-4


def _csr(dst, n):
    rp = torch.zeros(n + 1, dtype=torch.int64)
    rp[1:] = torch.cumsum(torch.bincount(dst, minlength=n), 0)
    return rp


@pytest.mark.parametrize("n,e,c", [(300, 6000, 32), (50, 700, 80)])
def test_sh_tp_scatter_raw_vectors(bm, dev, n, e, c):
    vec = raw_vectors(e, 81)
    x = torch.randn(n, c, 16, generator=gen(83))
    src = torch.randint(0, n, (e,), generator=gen(84))
    dst, _ = torch.sort(torch.randint(0, n, (e,), generator=gen(85)))
    out = bm.sh_tp_scatter(vec.to(dev), x.to(dev), src.to(dev), _csr(dst, n).to(dev), None, False)
    want = omp.sh_tp_scatter(vec.double().numpy(), x.double().numpy(), src.numpy(), dst.numpy(), n,
                             normalize=False)
    assert normwise_err(out.cpu(), want) <= 1e-5


def test_fused_message_passing_raw_vectors(bm, dev):
    n, e, c, cout = 200, 4000, 16, 24
    vec = raw_vectors(e, 91)
    x = torch.randn(n, c, 16, generator=gen(93))
    src = torch.randint(0, n, (e,), generator=gen(94))
    tgt = torch.randint(0, n, (e,), generator=gen(95))
    ei = torch.stack([src, tgt]).to(dev)
    rp, ci = bm.edge_index_to_csr(ei, n)
    out = bm.fused_message_passing_simple(x.to(dev), vec.to(dev), ei, rp, ci).cpu()
    want = omp.fused_message_passing_simple(x.double().numpy(), vec.double().numpy(), ei.cpu().numpy(),
                                            rp.cpu().numpy(), ci.cpu().numpy())
    assert normwise_err(out, want) <= 1e-5
    # dense-weight variant: col_idx read as the source atom, vectors by CSR slot
    w = torch.randn(c, cout, generator=gen(96)) / 4.0
    col = torch.randint(0, n, (e,), generator=gen(97))
    tg, _ = torch.sort(tgt)
    rp2 = _csr(tg, n)
    out2 = bm.fused_message_passing(x.to(dev), vec.to(dev), w.to(dev), rp2.to(dev), col.to(dev)).cpu()
    want2 = omp.fused_message_passing(x.double().numpy(), vec.double().numpy(), w.double().numpy(),
                                      rp2.numpy(), col.numpy())
    assert normwise_err(out2, want2) <= 1e-5


def test_scheduled_scatter_raw_neighbor_vectors(bm, dev):
    """Graph.sh_tp_scatter(normalize=False) on the neighbor list's own vectors (|v| <= 5 A)."""
    import batmobile
    n, c = 1200, 32
    pos, cell = periodic_box(n, 99)
    graph = batmobile.Graph(pos.to(dev), cell, 5.0, c)
    x = torch.randn(n, c, 16, generator=gen(100)).to(dev)
    out = graph.sh_tp_scatter(x, normalize=False).cpu()
    want = omp.sh_tp_scatter(graph.vec.cpu().double().numpy(), x.cpu().double().numpy(),
                             graph.src.cpu().numpy(), graph.dst.cpu().numpy(), n, normalize=False)
    assert normwise_err(out, want) <= 1e-5
