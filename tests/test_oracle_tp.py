"""Pins the tensor-product oracle (oracle/tp.py).

Independent checks: explicit loops over the 611 table entries on tiny inputs
(the reference's own formula, tests/test_tensor_product.py:57-81,230-282),
the adjoint identity <TP(x, y; W), g> = <x, gx> = <y, gy> = <W, gW>, finite
differences, and equivariance of the weighted product.
"""
import numpy as np
import pytest

from oracle import cg, tp


def _loop_simple(x, y):
    out = np.zeros_like(x)
    for p, a, b, o, c in cg.entries():
        out[:, int(o)] += c * x[:, int(a)] * y[:, int(b)]
    return out


def _loop_weighted(x, y, w):
    n, ci, _ = x.shape
    co = w.shape[2]
    out = np.zeros((n, co, 16))
    for p, a, b, o, c in cg.entries():
        p, a, b, o = int(p), int(a), int(b), int(o)
        t = c * x[:, :, a] * y[:, b][:, None]          # [n, ci]
        out[:, :, o] += t @ w[p]
    return out


def test_simple_matches_entry_loop():
    rng = np.random.default_rng(0)
    x, y = rng.normal(size=(7, 16)), rng.normal(size=(7, 16))
    np.testing.assert_allclose(tp.tensor_product_simple(x, y), _loop_simple(x, y), rtol=1e-12, atol=1e-12)


def test_weighted_matches_entry_loop():
    rng = np.random.default_rng(1)
    x, y, w = rng.normal(size=(5, 3, 16)), rng.normal(size=(5, 16)), rng.normal(size=(34, 3, 4))
    np.testing.assert_allclose(tp.tensor_product(x, y, w), _loop_weighted(x, y, w), rtol=1e-12, atol=1e-12)


def test_weighted_with_identity_mixing_reduces_to_simple():
    rng = np.random.default_rng(2)
    x, y = rng.normal(size=(6, 1, 16)), rng.normal(size=(6, 16))
    w = np.ones((34, 1, 1))
    np.testing.assert_allclose(tp.tensor_product(x, y, w)[:, 0], tp.tensor_product_simple(x[:, 0], y),
                               rtol=1e-12, atol=1e-12)


def test_simple_backward_adjoint():
    rng = np.random.default_rng(3)
    x, y, g = (rng.normal(size=(9, 16)) for _ in range(3))
    gx, gy = tp.tensor_product_simple_backward(x, y, g)
    ref = np.sum(tp.tensor_product_simple(x, y) * g)
    assert np.isclose(np.sum(gx * x), ref) and np.isclose(np.sum(gy * y), ref)


def test_weighted_backward_adjoint_and_fd():
    rng = np.random.default_rng(4)
    x, y, w = rng.normal(size=(6, 3, 16)), rng.normal(size=(6, 16)), rng.normal(size=(34, 3, 5))
    g = rng.normal(size=(6, 5, 16))
    gx, gy, gw = tp.tensor_product_backward(x, y, w, g)
    ref = np.sum(tp.tensor_product(x, y, w) * g)
    # the product is linear in each of x, y, W separately
    assert np.isclose(np.sum(gx * x), ref)
    assert np.isclose(np.sum(gy * y), ref)
    assert np.isclose(np.sum(gw * w), ref)
    h = 1e-6
    for (arr, grad) in ((x, gx), (y, gy), (w, gw)):
        idx = tuple(rng.integers(0, s) for s in arr.shape)
        orig = arr[idx]
        arr[idx] = orig + h
        up = np.sum(tp.tensor_product(x, y, w) * g)
        arr[idx] = orig - h
        dn = np.sum(tp.tensor_product(x, y, w) * g)
        arr[idx] = orig
        assert abs((up - dn) / (2 * h) - grad[idx]) < 1e-6 * max(1.0, abs(grad[idx]))


def test_weight_gradient_on_every_path():
    """Each of the 34 path blocks of grad_W is checked (the reference kernel is
    wrong on 15 of them, tensor_product_backward.cu:159-872)."""
    rng = np.random.default_rng(6)
    x, y, w = rng.normal(size=(4, 2, 16)), rng.normal(size=(4, 16)), rng.normal(size=(34, 2, 3))
    g = rng.normal(size=(4, 3, 16))
    _, _, gw = tp.tensor_product_backward(x, y, w, g)
    for p in range(34):
        e = np.zeros_like(w)
        e[p] = rng.normal(size=w[p].shape)
        # d/dt <TP(x,y;W+tE), g> = <E, gW>; the product is linear in W
        got = np.sum(tp.tensor_product(x, y, e) * g)
        assert np.isclose(got, np.sum(e * gw), rtol=1e-10, atol=1e-10)
