"""Shared helpers for the test-suite (inputs, tolerances, geometry)."""
import numpy as np
import torch

RHO = 30.0 / (4.0 / 3.0 * np.pi * 5.0 ** 3)   # ~30 neighbours within 5 A


def gen(seed):
    return torch.Generator().manual_seed(seed)


def unit_vectors(n, seed):
    v = torch.randn(n, 3, generator=gen(seed))
    return v / v.norm(dim=1, keepdim=True)


def normwise_err(got, want):
    """max|got - want| / max|want| (0 when both are empty or zero)."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    if want.size == 0:
        return 0.0
    den = np.abs(want).max()
    return float(np.abs(got - want).max() / (den if den > 0 else 1.0))


def periodic_box(n, seed):
    """Uniform positions in a cube with ~30 neighbours within 5 A."""
    L = float((n / RHO) ** (1.0 / 3.0))
    pos = torch.rand(n, 3, generator=gen(seed)) * L
    cell = torch.diag(torch.tensor([L, L, L]))
    return pos, cell


def dst_sorted_edges(src_i, dst_j, vec_ij):
    """NL output sorted by (i, j) -> edges sorted by destination.

    The neighbor relation is symmetric, so the message edge (src = j, dst = i)
    exists for every (i, j) and its vector r_dst - r_src is -vec_ij exactly.
    Returns (src, dst, vec) with dst non-decreasing and src ascending per dst.
    """
    return dst_j, src_i, -vec_ij


def random_rotation(seed):
    """A proper rotation matrix (det +1), float64."""
    q, _ = np.linalg.qr(np.random.default_rng(seed).normal(size=(3, 3)))
    return q * np.sign(np.linalg.det(q))


def wigner_d(rot, lmax=3, n=400, seed=0):
    """Block-diagonal D(R) with Y(R r) = D Y(r) for the real SH of the oracle, fitted by least
    squares per l from n random unit vectors (float64; exact to rounding)."""
    from oracle import sh
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
