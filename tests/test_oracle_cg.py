"""Pins the CG table (oracle/cg.py) and the product's generated copy of it.

The fixture is the reference's own table (tests/golden/cg_l3_ref.json, values of
include/cg_coefficients_l3.cuh).  The checks below are independent of it:
mathematics (orthonormality, exact +-sqrt(p/q) values, equivariance, the
spherical-harmonic product rule) and the product's table, which
batmobile-evo_amd/csrc/gen_tables.py derives from the Racah formula.
"""
import os
import re

import numpy as np
import pytest

from oracle import cg, sh

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GEN = os.path.join(REPO, "batmobile-evo_amd", "csrc", "generated_tables.h")


def _product_entries():
    txt = open(GEN).read()
    body = txt[txt.index("constexpr CGEntry kCG"):]
    body = body[:body.index("};")]
    rows = re.findall(r"\{(\d+), (\d+), (\d+), (\d+), (\d+), (-?[0-9.eE+-]+)f\}", body)
    return np.array([[float(v) for v in r] for r in rows])


def test_paths_follow_triangle_rule():
    # reference tests/test_tensor_product.py:315-340
    want = [(l1, l2, l3) for l1 in range(4) for l2 in range(4) for l3 in range(4)
            if abs(l1 - l2) <= l3 <= l1 + l2]
    assert [tuple(p) for p in cg.path_info()] == want
    assert len(want) == cg.NUM_PATHS == 34
    assert cg.entries().shape == (cg.NUM_ENTRIES, 5)


def test_entry_counts_per_path():
    counts = np.bincount(cg.entries()[:, 0].astype(int), minlength=34)
    assert counts.tolist() == [1, 3, 5, 7, 3, 3, 6, 11, 11, 16, 21, 21, 26, 5, 11, 16, 21, 5, 16,
                               25, 28, 21, 28, 41, 7, 21, 26, 21, 28, 41, 7, 26, 41, 42]


def test_product_table_equals_reference_table():
    prod = _product_entries()
    ref = cg.entries()
    assert prod.shape == (611, 6)
    # same (path, a, b, o) in the same order
    np.testing.assert_array_equal(prod[:, :4], ref[:, :4])
    # values agree to fp32 rounding (the reference prints 10 digits)
    assert np.abs(prod[:, 5] - ref[:, 4]).max() <= 6e-8
    # slot index q = first slot of the path + m_out
    _, slots = cg.dense_paths()
    l_out = cg.path_info()[prod[:, 0].astype(int), 2]
    np.testing.assert_array_equal(prod[:, 4], slots[prod[:, 0].astype(int)] + prod[:, 3] - l_out ** 2)


def test_orthonormal_per_path():
    cp, slots = cg.dense_paths()
    for p, (l1, l2, l3) in enumerate(cg.path_info()):
        blk = cp[l1 * l1:(l1 + 1) ** 2, l2 * l2:(l2 + 1) ** 2, slots[p]:slots[p + 1]]
        gram = np.einsum("abq,abr->qr", blk, blk)
        np.testing.assert_allclose(gram, np.eye(2 * l3 + 1), atol=2e-7)


def test_values_are_signed_square_roots_of_rationals():
    c2 = cg.entries()[:, 4] ** 2 * 840.0
    assert np.abs(c2 - np.round(c2)).max() < 2e-4
    assert (np.round(c2) >= 1).all()


def _fit_wigner_d(rot, lmax=3, n=400, seed=0):
    """D_l(R) with Y_l(R r) = D_l Y_l(r), fitted by least squares from the oracle SH."""
    rng = np.random.default_rng(seed)
    r = rng.normal(size=(n, 3))
    r /= np.linalg.norm(r, axis=1, keepdims=True)
    y0 = sh.spherical_harmonics(r, lmax)
    y1 = sh.spherical_harmonics(r @ rot.T, lmax)
    d = np.zeros(((lmax + 1) ** 2, (lmax + 1) ** 2))
    for l in range(lmax + 1):
        s = slice(l * l, (l + 1) ** 2)
        sol, *_ = np.linalg.lstsq(y0[:, s], y1[:, s], rcond=None)
        d[s, s] = sol.T
    return d


def _random_rotation(seed):
    q, _ = np.linalg.qr(np.random.default_rng(seed).normal(size=(3, 3)))
    return q * np.sign(np.linalg.det(q))


def _equivariance_error(c):
    rot = _random_rotation(7)
    d = _fit_wigner_d(rot)
    rng = np.random.default_rng(1)
    x, y = rng.normal(size=(5, 16)), rng.normal(size=(5, 16))
    lhs = np.einsum("abo,na,nb->no", c, x @ d.T, y @ d.T)
    rhs = np.einsum("abo,na,nb->no", c, x, y) @ d.T
    return np.abs(lhs - rhs).max()


def test_fitted_wigner_matrices_are_orthogonal():
    d = _fit_wigner_d(_random_rotation(7))
    np.testing.assert_allclose(d @ d.T, np.eye(16), atol=1e-10)


def test_tensor_product_is_equivariant():
    assert _equivariance_error(cg.dense()) < 1e-6


def test_planted_sign_error_breaks_equivariance():
    """A flipped coefficient (planted in a copy of the oracle table) must be caught."""
    c = cg.dense().copy()
    e = cg.entries()[300]
    c[int(e[1]), int(e[2]), int(e[3])] *= -1.0
    assert _equivariance_error(c) > 1e-2


@pytest.mark.parametrize("p", range(34))
def test_product_rule(p):
    """CG_p(Y_l1(r), Y_l2(r)) = k_p Y_lo(r) if l1+l2+lo is even, else 0."""
    l1, l2, l3 = cg.path_info()[p]
    cp, slots = cg.dense_paths()
    blk = cp[l1 * l1:(l1 + 1) ** 2, l2 * l2:(l2 + 1) ** 2, slots[p]:slots[p + 1]]
    rng = np.random.default_rng(p)
    r = rng.normal(size=(64, 3))
    r /= np.linalg.norm(r, axis=1, keepdims=True)
    y = sh.spherical_harmonics(r, 3)
    out = np.einsum("abq,na,nb->nq", blk, y[:, l1 * l1:(l1 + 1) ** 2], y[:, l2 * l2:(l2 + 1) ** 2])
    ylo = y[:, l3 * l3:(l3 + 1) ** 2]
    if (l1 + l2 + l3) % 2:
        assert np.abs(out).max() < 1e-6
    else:
        k = np.sum(out * ylo) / np.sum(ylo * ylo)
        assert abs(k) > 0.1
        assert np.abs(out - k * ylo).max() < 1e-6
