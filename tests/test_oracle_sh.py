"""Pins the spherical-harmonic oracle (oracle/sh.py) and the product's SH tables.

Independent checks: closed-form values on the polar axis, component
normalisation, homogeneity and harmonicity of the polynomials, the CG
recurrence derived in batmobile-evo_amd/csrc/gen_tables.py, finite differences
for the backward, and the normalisation chain rule.
"""
import importlib.util
import json
import os
import re

import numpy as np
import pytest

from oracle import sh

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(REPO, "tests", "golden")
CSRC = os.path.join(REPO, "batmobile-evo_amd", "csrc")


def _unit(n, seed):
    v = np.random.default_rng(seed).normal(size=(n, 3))
    return v / np.linalg.norm(v, axis=1, keepdims=True)


def _gen_tables():
    spec = importlib.util.spec_from_file_location("gen_tables", os.path.join(CSRC, "gen_tables.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _eval_product_recurrence(v, lmax):
    """Evaluate the SH term table compiled into the kernels (generated_tables.h)."""
    txt = open(os.path.join(CSRC, "generated_tables.h")).read()
    starts = [int(s) for s in re.search(r"kSHTermStart\[\d+\] = \{([^}]*)\}", txt).group(1).split(",")]
    body = txt[txt.index("constexpr SHTerm kSHTerms"):]
    terms = re.findall(r"\{(\d+), (\d+), (\d+), (-?[0-9.eE+-]+)f\}", body[:body.index("};")])
    terms = [(int(a), int(b), int(c), float(d)) for a, b, c, d in terms]
    y = [np.ones(len(v))]
    cols = [y[0]]
    blocks = [[y[0]]]
    for l in range(lmax):
        cur = [np.zeros(len(v)) for _ in range(2 * l + 3)]
        for (M, m, j, c) in terms[starts[l]:starts[l + 1]]:
            cur[M] = cur[M] + c * blocks[l][m] * v[:, j]
        blocks.append(cur)
        cols.extend(cur)
    return np.stack(cols, axis=1)


@pytest.mark.parametrize("lmax", range(7))
def test_polar_axis_known_answer(lmax):
    # on +y only m = 0 survives, with value sqrt(2l+1); on -y, (-1)^l sqrt(2l+1)
    for sgn in (1.0, -1.0):
        y = sh.spherical_harmonics(np.array([[0.0, sgn, 0.0]]), lmax)[0]
        want = np.zeros((lmax + 1) ** 2)
        for l in range(lmax + 1):
            want[l * l + l] = (sgn ** l) * np.sqrt(2 * l + 1)
        np.testing.assert_allclose(y, want, atol=1e-12)


def test_axis_and_diagonal_known_answers():
    inp = json.load(open(os.path.join(GOLDEN, "sh_known_inputs.json")))
    s3, s5, s15 = np.sqrt(3), np.sqrt(5), np.sqrt(15)
    y = sh.spherical_harmonics(np.array(inp["axis"], float), 2)
    # +x: Y1 = sqrt3 (1,0,0); Y2 = (0, 0, -sqrt5/2, 0, -sqrt15/2)
    np.testing.assert_allclose(y[0], [1, s3, 0, 0, 0, 0, -s5 / 2, 0, -s15 / 2], atol=1e-12)
    # +z: Y2 = (0, 0, -sqrt5/2, 0, +sqrt15/2)
    np.testing.assert_allclose(y[4], [1, 0, 0, s3, 0, 0, -s5 / 2, 0, s15 / 2], atol=1e-12)
    d = np.array(inp["diagonal"], float)
    yd = sh.spherical_harmonics(d, 2)
    x_, y_, z_ = d[3]
    np.testing.assert_allclose(yd[3, 4:9], [s15 * x_ * z_, s15 * x_ * y_, s5 * (y_ * y_ - 0.5 * (x_ * x_ + z_ * z_)),
                                            s15 * y_ * z_, 0.5 * s15 * (z_ * z_ - x_ * x_)], atol=1e-12)


@pytest.mark.parametrize("lmax", range(7))
def test_component_normalisation(lmax):
    y = sh.spherical_harmonics(_unit(200, lmax), lmax)
    for l in range(lmax + 1):
        np.testing.assert_allclose((y[:, l * l:(l + 1) ** 2] ** 2).sum(1), 2 * l + 1, rtol=1e-12)


def test_homogeneous_and_harmonic():
    v = np.random.default_rng(3).normal(size=(20, 3))
    y1 = sh.spherical_harmonics(v, 6)
    y2 = sh.spherical_harmonics(2.0 * v, 6)
    for l in range(7):
        s = slice(l * l, (l + 1) ** 2)
        np.testing.assert_allclose(y2[:, s], (2.0 ** l) * y1[:, s], rtol=1e-10, atol=1e-10)
    h = 1e-3
    lap = -6.0 * y1
    for k in range(3):
        e = np.zeros(3)
        e[k] = h
        lap = lap + sh.spherical_harmonics(v + e, 6) + sh.spherical_harmonics(v - e, 6)
    lap /= h * h
    assert np.abs(lap).max() / np.abs(y1).max() < 1e-4


@pytest.mark.parametrize("lmax", range(1, 7))
def test_cg_recurrence_matches_oracle(lmax):
    """Y_{l+1} = k_l CG(l,1,l+1)(Y_l, r), CG from the Racah formula (gen_tables.py)."""
    gt = _gen_tables()
    v = np.random.default_rng(lmax).normal(size=(30, 3))
    want = sh.spherical_harmonics(v, lmax)
    steps = gt.sh_recurrence()
    blocks = [np.ones((30, 1))]
    for l in range(lmax):
        nxt = np.zeros((30, 2 * l + 3))
        for (M, m, j, c) in steps[l]:
            nxt[:, M] += c * blocks[-1][:, m] * v[:, j]
        blocks.append(nxt)
    np.testing.assert_allclose(np.concatenate(blocks, axis=1), want, rtol=1e-11, atol=1e-11)


def test_product_table_recurrence_matches_oracle():
    v = np.random.default_rng(11).normal(size=(50, 3))
    np.testing.assert_allclose(_eval_product_recurrence(v, 6), sh.spherical_harmonics(v, 6),
                               rtol=2e-7, atol=2e-6)


@pytest.mark.parametrize("lmax", [1, 3, 6])
def test_backward_matches_finite_differences(lmax):
    rng = np.random.default_rng(5)
    v = rng.normal(size=(8, 3))
    g = rng.normal(size=(8, (lmax + 1) ** 2))
    got = sh.spherical_harmonics_backward(v, g)
    h = 1e-6
    fd = np.zeros_like(v)
    for k in range(3):
        e = np.zeros(3)
        e[k] = h
        fd[:, k] = ((sh.spherical_harmonics(v + e, lmax) - sh.spherical_harmonics(v - e, lmax)) * g).sum(1) / (2 * h)
    np.testing.assert_allclose(got, fd, rtol=1e-6, atol=1e-6)


def test_normalised_backward_is_gradient_of_normalised_forward():
    rng = np.random.default_rng(9)
    v = rng.normal(size=(8, 3)) * 3.0
    g = rng.normal(size=(8, 16))
    got = sh.spherical_harmonics_normalized_backward(v, g)
    h = 1e-6
    fd = np.zeros_like(v)
    for k in range(3):
        e = np.zeros(3)
        e[k] = h
        up = sh.spherical_harmonics(sh.normalize(v + e)[0], 3)
        dn = sh.spherical_harmonics(sh.normalize(v - e)[0], 3)
        fd[:, k] = ((up - dn) * g).sum(1) / (2 * h)
    np.testing.assert_allclose(got, fd, rtol=1e-6, atol=1e-6)
