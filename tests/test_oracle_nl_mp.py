"""Pins the neighbor-list oracle (oracle/nl_ref.c) and the message-passing oracle."""
import numpy as np
import pytest

from oracle import mp, nl, sh, tp

RHO = 30.0 / (4.0 / 3.0 * np.pi * 5.0 ** 3)


def _box(n, seed):
    L = (n / RHO) ** (1.0 / 3.0)
    pos = (np.random.default_rng(seed).random((n, 3)) * L).astype(np.float32)
    return pos, np.diag([L, L, L]).astype(np.float32)


@pytest.mark.parametrize("n", [10, 100, 1000])
def test_cell_list_equals_brute_force(n):
    pos, cell = _box(n, n)
    a = nl.cell_list(pos, cell, 5.0)
    b = nl.brute_force(pos, cell, 5.0)
    for u, v in zip(a, b):
        np.testing.assert_array_equal(u, v)


def reference_nl_cases():
    """Positions of the reference's correctness cases (tests/test_neighbor_list.cu:18-27,
    264-266: std::mt19937(42), density 0.05, N = 100, 500, 1000), written by
    tests/golden/make_nl_fixtures.py."""
    import json
    import os
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                        "nl_mt19937_positions.json")
    d = json.load(open(path))
    return [(c["N"], np.float32(c["box"]), np.asarray(c["positions"], dtype=np.float32))
            for c in d["cases"]], float(d["cutoff"])


def test_reference_cases_cell_list_equals_brute_force():
    """The reference's own cases: cell list == brute force (its check, :30-68), bit-exact."""
    cases, cutoff = reference_nl_cases()
    for n, box, pos in cases:
        assert pos.shape == (n, 3) and pos.min() >= 0 and pos.max() < box
        cell = np.diag([box, box, box]).astype(np.float32)
        a = nl.cell_list(pos, cell, cutoff)
        b = nl.brute_force(pos, cell, cutoff)
        for u, v in zip(a, b):
            np.testing.assert_array_equal(u, v)
        # ~ density * 4/3 pi r^3 = 26 neighbours per atom, symmetric
        assert 20 * n < a[0].size < 32 * n
        assert a[0].size == np.sum(a[0] != a[1])


def test_self_loops_and_symmetry():
    pos, cell = _box(300, 1)
    s, d, v = nl.cell_list(pos, cell, 5.0, self_loops=True)
    assert np.sum(s == d) == 300
    s, d, v = nl.cell_list(pos, cell, 5.0)
    fwd = {(int(i), int(j)): v[k] for k, (i, j) in enumerate(zip(s, d))}
    for (i, j), vec in fwd.items():
        np.testing.assert_array_equal(fwd[(j, i)], -vec)   # exact negation


def test_cubic_lattice_known_answer():
    # simple cubic lattice, spacing 2.0, 6^3 sites in a 12 A box: 6 neighbours at
    # r = 2 (inclusive cutoff), 6 + 12 at r = 2*sqrt(2) + eps
    g = np.arange(6) * 2.0 + 0.5
    pos = np.stack(np.meshgrid(g, g, g, indexing="ij"), -1).reshape(-1, 3).astype(np.float32)
    cell = np.diag([12.0, 12.0, 12.0]).astype(np.float32)
    s, _, v = nl.cell_list(pos, cell, 2.0)
    assert np.bincount(s, minlength=216).tolist() == [6] * 216
    np.testing.assert_allclose(np.linalg.norm(v, axis=1), 2.0)
    s, _, _ = nl.cell_list(pos, cell, 2.0 * np.sqrt(2.0) + 1e-3)
    assert np.bincount(s, minlength=216).tolist() == [18] * 216


def test_fused_equals_composition():
    rng = np.random.default_rng(0)
    n, e, c = 40, 300, 5
    vec = rng.normal(size=(e, 3))
    x = rng.normal(size=(n, c, 16))
    src = rng.integers(0, n, e)
    dst = rng.integers(0, n, e)
    msg = mp.fused_sh_tp_simple(vec, x, src)
    y = sh.spherical_harmonics(vec, 3)
    for k in range(0, e, 37):
        np.testing.assert_allclose(msg[k], tp.tensor_product_simple(x[src[k]], np.repeat(y[k:k + 1], c, 0)),
                                   rtol=1e-12, atol=1e-12)
    out = mp.scatter_add(msg, dst, n)
    np.testing.assert_allclose(mp.sh_tp_scatter(vec, x, src, dst, n), out, rtol=1e-12, atol=1e-12)
    # CSR single-kernel semantics (fused_message_passing.cu:174-255) agree as well
    ei = np.stack([src, dst])
    rp, ci = mp.edge_index_to_csr(ei, n)
    np.testing.assert_allclose(mp.fused_message_passing_simple(x, vec, ei, rp, ci), out,
                               rtol=1e-12, atol=1e-12)


def test_csr_is_stable_and_complete():
    rng = np.random.default_rng(1)
    ei = np.stack([rng.integers(0, 20, 200), rng.integers(0, 20, 200)])
    rp, ci = mp.edge_index_to_csr(ei, 25)
    assert rp[0] == 0 and rp[-1] == 200 and len(rp) == 26
    for t in range(25):
        row = ci[rp[t]:rp[t + 1]]
        assert (ei[1, row] == t).all() and (np.diff(row) > 0).all()


def test_dense_weight_message_passing():
    rng = np.random.default_rng(2)
    n, e, ci_, co = 12, 60, 3, 4
    vec = rng.normal(size=(e, 3))
    x = rng.normal(size=(n, ci_, 16))
    w = rng.normal(size=(ci_, co))
    tgt = np.sort(rng.integers(0, n, e))
    rp = np.concatenate([[0], np.cumsum(np.bincount(tgt, minlength=n))])
    col = rng.integers(0, n, e)     # read as source atoms by the reference kernel
    got = mp.fused_message_passing(x, vec, w, rp, col)
    want = np.zeros((n, co, 16))
    for k in range(e):
        t = tp.tensor_product_simple(x[col[k]], np.repeat(sh.spherical_harmonics(vec[k:k + 1], 3), ci_, 0))
        want[tgt[k]] += np.einsum("io,ic->co", t, w)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_weighted_message_passing_matches_per_edge_loop():
    rng = np.random.default_rng(3)
    n, e, ci_, co = 10, 40, 2, 3
    vec = rng.normal(size=(e, 3))
    x = rng.normal(size=(n, ci_, 16))
    w = rng.normal(size=(34, ci_, co))
    src, dst = rng.integers(0, n, e), rng.integers(0, n, e)
    got = mp.weighted_message_passing(vec, x, w, src, dst, n)
    u, _ = sh.normalize(vec)
    want = np.zeros((n, co, 16))
    for k in range(e):
        want[dst[k]] += tp.tensor_product(x[src[k]][None], sh.spherical_harmonics(u[k:k + 1], 3), w)[0]
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("normalize", [True, False])
def test_cpu_baseline_compositions_match_the_oracle(normalize):
    """The float32 torch compositions bench.py times as its CPU baselines
    (oracle/cpu_path.py) agree with the float64 message-passing oracle, the weighted one
    with chunks smaller than the edge list so that the chunked scatter is exercised."""
    import torch

    from oracle import cpu_path
    g = torch.Generator().manual_seed(11)
    n, e, c, co = 40, 700, 6, 10
    vec = torch.randn(e, 3, generator=g) * 2.0
    x = torch.randn(n, c, 16, generator=g)
    w = torch.randn(34, c, co, generator=g) / 3.0
    src = torch.randint(0, n, (e,), generator=g)
    dst = torch.randint(0, n, (e,), generator=g)
    got = cpu_path.weighted_sh_tp_scatter(vec, x, w, src, dst, n, normalize=normalize, chunk=128)
    want = mp.weighted_message_passing(vec.double().numpy(), x.double().numpy(),
                                       w.double().numpy(), src.numpy(), dst.numpy(), n,
                                       normalize=normalize)
    assert np.abs(got.numpy() - want).max() <= 1e-5 * np.abs(want).max()
    got = cpu_path.sh_tp_scatter(vec, x, src, dst, n, normalize=normalize)
    want = mp.sh_tp_scatter(vec.double().numpy(), x.double().numpy(), src.numpy(), dst.numpy(),
                            n, normalize=normalize)
    assert np.abs(got.numpy() - want).max() <= 1e-5 * np.abs(want).max()
