"""GPU parity of the autograd wrappers (reference python/batmobile/autograd.py).

Gradients within 1e-4 normwise of the float64 oracle.
"""
import numpy as np
import pytest
import torch

from helpers import gen, normwise_err, unit_vectors
from oracle import sh as osh
from oracle import tp as otp

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("normalize", [True, False])
@pytest.mark.parametrize("lmax", [1, 3, 5])
def test_spherical_harmonics_function(dev, normalize, lmax):
    import batmobile
    v = torch.randn(2000, 3, generator=gen(1)) * 2.0
    if not normalize:
        v = v / v.norm(dim=1, keepdim=True)
    g = torch.randn(2000, (lmax + 1) ** 2, generator=gen(2))
    vd = v.to(dev).requires_grad_(True)
    y = batmobile.spherical_harmonics_autograd(vd, lmax, normalize)
    (y * g.to(dev)).sum().backward()
    vv = v.double().numpy()
    if normalize:
        want_y = osh.spherical_harmonics(osh.normalize(vv)[0], lmax)
        want_g = osh.spherical_harmonics_normalized_backward(vv, g.double().numpy())
    else:
        want_y = osh.spherical_harmonics(vv, lmax)
        want_g = osh.spherical_harmonics_backward(vv, g.double().numpy())
    assert normwise_err(y.detach().cpu(), want_y) <= 1e-5
    assert normwise_err(vd.grad.cpu(), want_g) <= 1e-4


def test_tensor_product_simple_function(dev):
    import batmobile
    x, y, g = (torch.randn(1500, 16, generator=gen(s)) for s in (3, 4, 5))
    xd, yd = x.to(dev).requires_grad_(True), y.to(dev).requires_grad_(True)
    out = batmobile.tensor_product_simple_autograd(xd, yd)
    (out * g.to(dev)).sum().backward()
    wx, wy = otp.tensor_product_simple_backward(*(t.double().numpy() for t in (x, y, g)))
    assert normwise_err(xd.grad.cpu(), wx) <= 1e-4
    assert normwise_err(yd.grad.cpu(), wy) <= 1e-4


@pytest.mark.parametrize("needs", [(True, True, True), (False, True, True), (True, False, False)])
def test_tensor_product_function(dev, needs):
    import batmobile
    n, cin, cout = 600, 8, 12
    x = torch.randn(n, cin, 16, generator=gen(6))
    y = torch.randn(n, 16, generator=gen(7))
    w = torch.randn(34, cin, cout, generator=gen(8)) / np.sqrt(cin)
    g = torch.randn(n, cout, 16, generator=gen(9))
    ts = [t.to(dev).requires_grad_(r) for t, r in zip((x, y, w), needs)]
    out = batmobile.tensor_product_autograd(ts[0], ts[1], ts[2], cin, cout)
    (out * g.to(dev)).sum().backward()
    want = otp.tensor_product_backward(*(t.double().numpy() for t in (x, y, w, g)))
    for t, r, wg in zip(ts, needs, want):
        if r:
            assert normwise_err(t.grad.cpu(), wg) <= 1e-4
        else:
            assert t.grad is None


def test_layer_composition_gradients_wrt_positions(dev):
    """SH(normalised r_dst - r_src) -> weighted TP -> index_add_, backward to positions
    (the pattern of reference benchmarks/benchmark_e2e_mace.py:308-356,885-946)."""
    import batmobile
    n, e, c = 60, 600, 8
    pos = torch.randn(n, 3, generator=gen(10)) * 3.0
    src = torch.randint(0, n, (e,), generator=gen(11))
    dst = (src + 1 + torch.randint(0, n - 1, (e,), generator=gen(12))) % n
    x = torch.randn(n, c, 16, generator=gen(13))
    w = torch.randn(34, c, c, generator=gen(14)) / np.sqrt(c)
    pd = pos.to(dev).requires_grad_(True)
    vec = pd[dst.to(dev)] - pd[src.to(dev)]
    y = batmobile.spherical_harmonics_autograd(vec, 3, True)
    msg = batmobile.tensor_product_autograd(x.to(dev)[src.to(dev)], y, w.to(dev), c, c)
    out = torch.zeros(n, c, 16, device=dev).index_add_(0, dst.to(dev), msg)
    energy = (out ** 2).sum()
    energy.backward()
    # float64 CPU autograd of the same composition through the oracle SH/TP formulas
    p64 = pos.double().requires_grad_(True)
    v64 = p64[dst] - p64[src]
    u64 = v64 / v64.norm(dim=1, keepdim=True).clamp(min=1e-10)
    y64 = osh.spherical_harmonics(u64, 3, xp=torch)
    cp, _ = __import__("oracle.cg", fromlist=["dense_paths"]).dense_paths()
    cp = torch.as_tensor(cp)
    t64 = torch.einsum("abq,nb,nia->niq", cp, y64, x.double()[src])
    from oracle import cg as ocg
    wq = w.double()[torch.as_tensor(ocg.slot_to_path())]
    s = torch.zeros(cp.shape[2], 16, dtype=torch.float64)
    s[torch.arange(cp.shape[2]), torch.as_tensor(ocg.slot_to_output())] = 1.0
    m64 = torch.einsum("niq,qic->ncq", t64, wq) @ s
    o64 = torch.zeros(n, c, 16, dtype=torch.float64).index_add_(0, dst, m64)
    (o64 ** 2).sum().backward()
    assert normwise_err(pd.grad.cpu(), p64.grad.numpy()) <= 1e-4
