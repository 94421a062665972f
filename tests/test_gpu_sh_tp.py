"""GPU parity: spherical harmonics and tensor products vs the float64 oracle.

Tolerances (written per test): forward fp32 outputs within 1e-5 normwise
(max|gpu - oracle| <= 1e-5 * max|oracle|) or the reference's own elementwise
atol = rtol = 1e-5 for SH (tests/test_spherical_harmonics.py:49); gradients
within 1e-4 normwise.
"""
import json
import os

import numpy as np
import pytest
import torch

from helpers import gen, normwise_err, unit_vectors
from oracle import sh as osh
from oracle import tp as otp

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_mfma_lane_layout(bm, dev):
    a = torch.randn(16, 4, generator=gen(0))
    b = torch.randn(4, 16, generator=gen(1))
    d = bm.selftest_mfma_16x16x4(a.to(dev), b.to(dev)).cpu()
    torch.testing.assert_close(d, a @ b, rtol=1e-5, atol=1e-5)


def test_mfma_4x4_broadcast_lane_layout(bm, dev):
    """The weighted scatter's mixing step: v_mfma_f32_4x4x1_16b_f32 with CBSZ = 4 and
    ABID = k gives lane 4b + j the products A[4k + r] * B[4b + j], r = 0..3."""
    a = torch.randn(64, generator=gen(2))
    b = torch.randn(64, generator=gen(3))
    d = bm.selftest_mfma_4x4x1_bcast(a.to(dev), b.to(dev)).cpu()
    want = torch.empty(16, 64, 4)
    for k in range(16):
        for lane in range(64):
            for r in range(4):
                want[k, lane, r] = a[4 * k + r] * b[lane]
    torch.testing.assert_close(d, want, rtol=1e-6, atol=0)


@pytest.mark.parametrize("lmax", range(7))
@pytest.mark.parametrize("n", [1, 10, 100, 1000, 100000])
def test_sh_forward_random(bm, dev, lmax, n):
    v = unit_vectors(n, 42)
    y = bm.spherical_harmonics(v.to(dev), lmax).cpu().numpy()
    want = osh.spherical_harmonics(v.double().numpy(), lmax)
    assert y.shape == want.shape
    np.testing.assert_allclose(y, want, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("lmax", [3, 6])
def test_sh_known_inputs(bm, dev, lmax):
    inp = json.load(open(os.path.join(GOLDEN, "sh_known_inputs.json")))
    for key, tol in (("axis", 1e-5), ("diagonal", 1e-5), ("near_pole_unnormalised", 1e-4)):
        v = torch.tensor(inp[key], dtype=torch.float32)
        if key.startswith("near_pole"):
            v = v / v.norm(dim=1, keepdim=True)
        y = bm.spherical_harmonics(v.to(dev), lmax).cpu().numpy()
        np.testing.assert_allclose(y, osh.spherical_harmonics(v.double().numpy(), lmax), rtol=tol, atol=tol)


def test_sh_inplace_empty_and_shapes(bm, dev):
    v = unit_vectors(300, 1).to(dev)
    out = torch.full((300, 16), -7.0, device=dev)
    bm.spherical_harmonics_inplace(v, out, 3)
    torch.testing.assert_close(out, bm.spherical_harmonics(v, 3), rtol=0, atol=0)
    for lmax in range(7):
        assert tuple(bm.spherical_harmonics(v[:0], lmax).shape) == (0, (lmax + 1) ** 2)
        assert tuple(bm.spherical_harmonics(v, lmax).shape) == (300, (lmax + 1) ** 2)
    with pytest.raises(RuntimeError):
        bm.spherical_harmonics_inplace(v, torch.empty(300, 9, device=dev), 3)


@pytest.mark.parametrize("lmax", range(7))
def test_sh_normalized_forward(bm, dev, lmax):
    v = torch.randn(5000, 3, generator=gen(3)) * 3.0
    y = bm.spherical_harmonics_normalized(v.to(dev), lmax).cpu().numpy()
    u, _ = osh.normalize(v.double().numpy())
    np.testing.assert_allclose(y, osh.spherical_harmonics(u, lmax), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("lmax", range(7))
def test_sh_backward(bm, dev, lmax):
    v = unit_vectors(4000, 5)
    g = torch.randn(4000, (lmax + 1) ** 2, generator=gen(6))
    got = bm.spherical_harmonics_backward(v.to(dev), g.to(dev)).cpu().numpy()
    want = osh.spherical_harmonics_backward(v.double().numpy(), g.double().numpy())
    assert normwise_err(got, want) <= 1e-4


@pytest.mark.parametrize("lmax", [0, 3, 6])
def test_sh_normalized_backward(bm, dev, lmax):
    v = torch.randn(4000, 3, generator=gen(7)) * 2.5
    g = torch.randn(4000, (lmax + 1) ** 2, generator=gen(8))
    got = bm.spherical_harmonics_normalized_backward(v.to(dev), g.to(dev)).cpu().numpy()
    want = osh.spherical_harmonics_normalized_backward(v.double().numpy(), g.double().numpy())
    assert normwise_err(got, want) <= 1e-4


@pytest.mark.parametrize("n", [1, 257, 20000, 65536, 65537, 100003])
def test_tp_simple_forward(bm, dev, n):
    # configs[0] workload at n = 20000: Y of unit Gaussian vectors, x ~ N(0,1)
    v = unit_vectors(n, 0)
    y = bm.spherical_harmonics(v.to(dev), 3)
    x = torch.randn(n, 16, generator=gen(10)).to(dev)
    out = bm.tensor_product_simple(x, y).cpu().numpy()
    want = otp.tensor_product_simple(x.cpu().double().numpy(), y.cpu().double().numpy())
    assert normwise_err(out, want) <= 1e-5
    np.testing.assert_allclose(out, want, rtol=1e-4, atol=1e-5)


def test_tp_simple_small_and_large_kernels_agree(bm, dev):
    """Up to 65,536 rows the product runs one row per lane from global memory, above that
    through LDS-staged coalesced rows: the same rows give the same bits either way."""
    n = 65537
    v = unit_vectors(n, 5)
    y = bm.spherical_harmonics(v.to(dev), 3)
    x = torch.randn(n, 16, generator=gen(11)).to(dev)
    big = bm.tensor_product_simple(x, y)
    small = bm.tensor_product_simple(x[:n - 1].contiguous(), y[:n - 1].contiguous())
    assert torch.equal(big[:n - 1], small)
    last = bm.tensor_product_simple(x[n - 1:].contiguous(), y[n - 1:].contiguous())
    assert torch.equal(big[n - 1:], last)


def test_tp_simple_large_input_chunks(bm, dev):
    """At 700,001 rows (LDS-staged workgroups of 256 rows, the last one partial) the rows
    equal the one-row-per-lane kernel's bit for bit, chunk by chunk."""
    n = 700001
    g = gen(12)
    x = torch.randn(n, 16, generator=g).to(dev)
    y = torch.randn(n, 16, generator=g).to(dev)
    big = bm.tensor_product_simple(x, y)
    for s0 in range(0, n, 65536):
        s1 = min(n, s0 + 65536)
        small = bm.tensor_product_simple(x[s0:s1].contiguous(), y[s0:s1].contiguous())
        assert torch.equal(big[s0:s1], small)


def test_tp_simple_backward(bm, dev):
    n = 3000
    x, y, g = (torch.randn(n, 16, generator=gen(s)) for s in (11, 12, 13))
    gx, gy = bm.tensor_product_simple_backward(x.to(dev), y.to(dev), g.to(dev))
    wx, wy = otp.tensor_product_simple_backward(*(t.double().numpy() for t in (x, y, g)))
    assert normwise_err(gx.cpu(), wx) <= 1e-5
    assert normwise_err(gy.cpu(), wy) <= 1e-5


@pytest.mark.parametrize("n,cin,cout", [(1000, 32, 64), (37, 3, 5), (64, 16, 16), (5, 64, 128),
                                         (17, 40, 200), (256, 24, 64), (129, 16, 80)])
def test_tp_weighted_forward(bm, dev, n, cin, cout):
    # row tiles are dealt to workgroups eight at a time (one per XCD): 256 rows fill
    # two rounds exactly, 129 rows leave one row in a ninth tile and seven idle ones
    # (1000, 32, 64) is configs[1]: x ~ N(0,1), Y of normalised Gaussian vectors, W ~ N(0, 1/C_in)
    x = torch.randn(n, cin, 16, generator=gen(1))
    y = bm.spherical_harmonics(unit_vectors(n, 2).to(dev), 3).cpu()
    w = torch.randn(34, cin, cout, generator=gen(3)) / np.sqrt(cin)
    out = bm.tensor_product(x.to(dev), y.to(dev), w.to(dev)).cpu().numpy()
    want = otp.tensor_product(x.double().numpy(), y.double().numpy(), w.double().numpy())
    assert out.shape == (n, cout, 16)
    assert normwise_err(out, want) <= 1e-5


def _tp_backward_oracle_chunked(x, y, w, g, chunk=2000):
    gx, gy, gw = [], [], 0.0
    for s in range(0, x.shape[0], chunk):
        a, b, c = otp.tensor_product_backward(x[s:s + chunk], y[s:s + chunk], w, g[s:s + chunk])
        gx.append(a)
        gy.append(b)
        gw = gw + c
    return np.concatenate(gx), np.concatenate(gy), gw


@pytest.mark.parametrize("n,cin,cout", [
    (20000, 32, 64),   # configs[2]
    (300, 5, 7),
    (1, 16, 16),
    (40, 20, 100),     # C_out in (64, 128]: the 128-channel grad_output tile
    (20, 8, 160),      # C_out > 128: the per-(row, channel) grad_x / grad_y kernel
    (9, 24, 320),      # C_out above the reference binding's sizes, g staged in LDS
    (5, 12, 1100),     # g of two rows over 64 KB: one row per workgroup, g read from memory
    (33, 80, 24),      # 15 (group, channel-tile) units on 8 waves: waves loop over units
    (45, 32, 48),      # single-tile workgroups of the two-tile kernel, the last tile partly past N
    (35, 64, 20),      # the same with C_in = 64 and C_out not a multiple of 16
    (12810, 32, 16),   # 801 tiles: two-tile workgroups throughout, the last pair half past N
])
def test_tp_weighted_backward(bm, dev, n, cin, cout):
    # (20000, 32, 64) is configs[2]: upstream grad ~ N(0,1)
    x = torch.randn(n, cin, 16, generator=gen(21))
    y = bm.spherical_harmonics(unit_vectors(n, 22).to(dev), 3).cpu()
    w = torch.randn(34, cin, cout, generator=gen(23)) / np.sqrt(cin)
    g = torch.randn(n, cout, 16, generator=gen(24))
    gx, gy, gw = bm.tensor_product_backward(x.to(dev), y.to(dev), w.to(dev), g.to(dev))
    wx, wy, ww = _tp_backward_oracle_chunked(*(t.double().numpy() for t in (x, y, w, g)))
    assert normwise_err(gx.cpu(), wx) <= 1e-4
    assert normwise_err(gy.cpu(), wy) <= 1e-4
    assert normwise_err(gw.cpu(), ww) <= 1e-4


def test_tp_weighted_backward_flags_and_empty(bm, dev):
    n, cin, cout = 50, 4, 6
    x = torch.randn(n, cin, 16, generator=gen(31)).to(dev)
    y = torch.randn(n, 16, generator=gen(32)).to(dev)
    w = torch.randn(34, cin, cout, generator=gen(33)).to(dev)
    g = torch.randn(n, cout, 16, generator=gen(34)).to(dev)
    full = bm.tensor_product_backward(x, y, w, g)
    only_w = bm.tensor_product_backward(x, y, w, g, False, False, True)
    assert only_w[0] is None and only_w[1] is None
    torch.testing.assert_close(only_w[2], full[2], rtol=0, atol=0)
    only_x = bm.tensor_product_backward(x, y, w, g, True, False, False)
    assert only_x[2] is None and only_x[1] is None
    torch.testing.assert_close(only_x[0], full[0], rtol=0, atol=0)
    e = bm.tensor_product_backward(x[:0], y[:0], w, g[:0])
    assert tuple(e[0].shape) == (0, cin, 16) and tuple(e[1].shape) == (0, 16)
    assert torch.count_nonzero(e[2]).item() == 0 and tuple(e[2].shape) == (34, cin, cout)


def test_tp_weighted_backward_is_deterministic(bm, dev):
    n, cin, cout = 4000, 8, 16
    x = torch.randn(n, cin, 16, generator=gen(41)).to(dev)
    y = torch.randn(n, 16, generator=gen(42)).to(dev)
    w = torch.randn(34, cin, cout, generator=gen(43)).to(dev)
    g = torch.randn(n, cout, 16, generator=gen(44)).to(dev)
    a = bm.tensor_product_backward(x, y, w, g)
    b = bm.tensor_product_backward(x, y, w, g)
    for u, v in zip(a, b):
        assert torch.equal(u, v)
