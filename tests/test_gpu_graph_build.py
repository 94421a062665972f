"""GPU parity of the four-kernel graph build (batteries_graph_build_count / _write,
_batmobile.graph_build, batmobile.Graph for up to 8192 atoms), and of the neighbor list
from the same cell kernels (batteries_neighbor_list_cells_*, _batmobile.neighbor_list
for up to 8192 atoms) against the general passes (row_capacity < 0).

Every array it returns (edges in the message-passing layout, vectors, row offsets,
spatial order, schedule and edge_perm) must equal, bit for bit, the general path's
(neighbor list passes, serpentine order, mp_schedule: batmobile.Graph with
fast_build=False), which the neighbor-list tests pin to the oracle; the edges are also
compared with the C restatement of the reference's cell list directly
(src/neighbor_list/neighbor_list.cu:242-430).  Cases: the configs[3] system, the
reference's own positions, self loops, boxes of three cells per axis (every cell's
stencil is the whole box: candidate lists past the 2048 staged per chunk and cells of
more than 256 atoms), sparse boxes with empty cells, one atom, positions outside the
box, a non-cubic box, rows past the slab row capacity (found again by the write
kernel), and max_edges (no host synchronisation) with and without overflow.
"""
import numpy as np
import pytest
import torch

from helpers import gen, periodic_box
from oracle import nl as onl

pytestmark = pytest.mark.gpu

FIELDS = ("src", "dst", "vec", "row_ptr", "order", "row_ptr_s", "row_dst", "edge_perm")


def _graphs(pos, cell, cutoff, c=64, self_loops=False, **kw):
    import batmobile
    fast = batmobile.Graph(pos, cell, cutoff, c, self_loops=self_loops, **kw)
    general = batmobile.Graph(pos, cell, cutoff, c, self_loops=self_loops, fast_build=False, **kw)
    return fast, general


def _assert_same(fast, general, e=None):
    for f in FIELDS:
        a, b = getattr(fast, f), getattr(general, f)
        if e is not None and f in ("src", "dst", "vec", "edge_perm"):
            a, b = a[:e], b[:e]
        assert torch.equal(a, b), f
    assert (fast.n_blocks, fast.rows_per_block) == (general.n_blocks, general.rows_per_block)


def _assert_oracle(g, pos, cell, cutoff, self_loops=False):
    s, d, v = onl.cell_list(pos.cpu().numpy(), cell.numpy(), cutoff, self_loops)
    # the neighbor list (i, j) read with roles swapped: grouped by destination i
    np.testing.assert_array_equal(g.dst.cpu().numpy(), s)
    np.testing.assert_array_equal(g.src.cpu().numpy(), d)
    np.testing.assert_array_equal(g.vec.cpu().numpy(), -v)


def _fast_taken(bm, pos, cell, cutoff, c=64):
    return bm.graph_build(pos, cell, cutoff, False, c) is not None


@pytest.mark.parametrize("n,seed", [(5000, 3), (1000, 11), (8192, 8192), (300, 5)])
def test_graph_build_equals_general_path_and_oracle(bm, dev, n, seed):
    pos, cell = periodic_box(n, seed)
    pos = pos.to(dev)
    print(f"graph build n={n} seed={seed}", flush=True)
    assert _fast_taken(bm, pos, cell, 5.0)
    fast, general = _graphs(pos, cell, 5.0)
    _assert_same(fast, general)
    _assert_oracle(fast, pos, cell, 5.0)
    rdst = fast.row_dst.cpu()
    assert torch.equal(torch.sort(rdst[rdst >= 0]).values, torch.arange(n))


def test_graph_build_reference_cases_and_self_loops(bm, dev):
    from test_oracle_nl_mp import reference_nl_cases
    cases, cutoff = reference_nl_cases()
    for n, box, p in cases:
        print(f"graph build reference case N={n}", flush=True)
        cell = torch.diag(torch.tensor([box, box, box], dtype=torch.float32))
        pos = torch.from_numpy(p).to(dev)
        for sl in (False, True):
            fast, general = _graphs(pos, cell, cutoff, self_loops=sl)
            _assert_same(fast, general)
            _assert_oracle(fast, pos, cell, cutoff, sl)


@pytest.mark.parametrize("n,box,cutoff,c", [
    (3000, 12.0, 4.0, 64),    # 3 cells per axis: each stencil is the whole box (> 2048)
    (8000, 12.0, 4.0, 32),    # ~296 atoms per cell: own atoms past 256 per chunk
    (10, 60.0, 5.0, 64),      # mostly empty cells
    (1, 20.0, 5.0, 16),       # one atom
    (700, 15.0, 5.0, 128),    # 3 cells per axis, two channel groups
])
def test_graph_build_dense_sparse_and_tiny(bm, dev, n, box, cutoff, c):
    pos = (torch.rand(n, 3, generator=gen(n + 7)) * box).to(dev)
    cell = torch.diag(torch.tensor([box, box, box]))
    print(f"graph build n={n} box={box} rc={cutoff} C={c}", flush=True)
    assert _fast_taken(bm, pos, cell, cutoff, c)
    fast, general = _graphs(pos, cell, cutoff, c)
    _assert_same(fast, general)
    _assert_oracle(fast, pos, cell, cutoff)


def test_graph_build_positions_outside_box_and_non_cubic(bm, dev):
    """Positions wrapped by the binning (negative, past the box), a non-cubic box."""
    L = torch.tensor([31.0, 22.5, 40.0])
    pos = (torch.rand(2500, 3, generator=gen(71)) * 3.0 - 1.0) * L
    cell = torch.diag(L)
    pos = pos.to(dev)
    assert _fast_taken(bm, pos, cell, 5.0)
    fast, general = _graphs(pos, cell, 5.0)
    _assert_same(fast, general)
    _assert_oracle(fast, pos, cell, 5.0)


@pytest.mark.parametrize("row_cap", [1, 4, 16])
def test_graph_build_rows_past_the_slab_capacity(bm, dev, row_cap):
    """A slab row capacity under the degrees (~30): most rows are found again, in index
    order, by the write kernel; the result is unchanged."""
    import batmobile
    pos, cell = periodic_box(3000, 12)
    pos = pos.to(dev)
    general = batmobile.Graph(pos, cell, 5.0, 64, fast_build=False)
    res = bm.graph_build(pos, cell, 5.0, False, 64, -1, row_cap)
    assert res is not None
    for f, a in zip(FIELDS[:3], res[:3]):
        assert torch.equal(a, getattr(general, f)), f
    for f, a in (("row_ptr", res[3]), ("order", res[4]), ("row_ptr_s", res[5]),
                 ("edge_perm", res[6]), ("row_dst", res[7])):
        assert torch.equal(a, getattr(general, f)), f
    # with self loops and max_edges as well
    gs = batmobile.Graph(pos, cell, 5.0, 64, self_loops=True, fast_build=False)
    e = gs.num_edges
    r2 = bm.graph_build(pos, cell, 5.0, True, 64, e + 10, row_cap)
    assert int(r2[10].item()) == 0
    assert torch.equal(r2[0][:e], gs.src) and torch.equal(r2[2][:e], gs.vec)
    assert torch.equal(r2[6][:e], gs.edge_perm)


def test_graph_build_max_edges(bm, dev):
    import batmobile
    pos, cell = periodic_box(5000, 3)
    pos = pos.to(dev)
    ex = batmobile.Graph(pos, cell, 5.0, 64)
    e = ex.num_edges
    for cap in (e, e + 999):
        fast, general = _graphs(pos, cell, 5.0, max_edges=cap)
        fast.check()
        assert fast.num_edges == e and fast.src.numel() == cap
        _assert_same(fast, general, e)
        _assert_same(fast, ex, e)
    x = torch.randn(5000, 64, 16, generator=gen(91)).to(dev)
    assert torch.equal(fast.sh_tp_scatter(x), ex.sh_tp_scatter(x))


@pytest.mark.parametrize("max_edges", [0, 1000, 150000])
def test_graph_build_max_edges_overflow(bm, dev, max_edges):
    """Too few max_edges: the flag is raised, every row is empty, the schedule still
    lists every destination (with no edges), and the kernels read nothing past the
    arrays (all-zero outputs)."""
    import batmobile
    pos, cell = periodic_box(5000, 3)
    g = batmobile.Graph(pos.to(dev), cell, 5.0, 64, max_edges=max_edges)
    with pytest.raises(RuntimeError, match="max_edges"):
        g.check()
    assert int(g.row_ptr.abs().sum().item()) == 0
    assert int(g.row_ptr_s.abs().sum().item()) == 0
    rdst = g.row_dst.cpu()
    assert torch.equal(torch.sort(rdst[rdst >= 0]).values, torch.arange(5000))
    x = torch.randn(5000, 64, 16, generator=gen(92)).to(dev)
    assert torch.count_nonzero(g.sh_tp_scatter(x)).item() == 0


def test_graph_build_repeated_builds_agree(bm, dev):
    """Back-to-back builds on one stream (workspaces reused by the allocator) and a
    rebuild after the positions moved give the general path's results each time."""
    import batmobile
    pos, cell = periodic_box(5000, 3)
    pos = pos.to(dev)
    first = [batmobile.Graph(pos, cell, 5.0, 64, max_edges=160000) for _ in range(3)]
    for g in first[1:]:
        _assert_same(g, first[0], first[0].num_edges)  # entries past E are not written
    pos2 = pos + 0.3 * torch.randn(pos.shape, generator=gen(93)).to(dev)
    fast, general = _graphs(pos2, cell, 5.0)
    _assert_same(fast, general)


@pytest.mark.parametrize("case", ["cfg3", "dense", "self_loops", "cap1", "cap8", "skewed", "tiny"])
def test_neighbor_list_cells_equal_general_passes(bm, dev, case):
    """_batmobile.neighbor_list through the cell kernels equals the general passes bit for
    bit ([2, E] int64 sorted by (i, j), vectors, row offsets), and the C oracle."""
    cutoff, sl, cap = 5.0, False, 0
    if case == "dense":
        pos = torch.rand(3000, 3, generator=gen(81)) * 12.0
        cell, cutoff = torch.diag(torch.tensor([12.0, 12.0, 12.0])), 4.0
    elif case == "skewed":
        L = torch.tensor([31.0, 22.5, 40.0])
        pos = (torch.rand(2500, 3, generator=gen(82)) * 3.0 - 1.0) * L
        cell = torch.diag(L)
    elif case == "tiny":
        pos = torch.rand(2, 3, generator=gen(83)) * 2.0
        cell = torch.diag(torch.tensor([20.0, 20.0, 20.0]))
    else:
        pos, cell = periodic_box(5000 if case == "cfg3" else 2000, 3 if case == "cfg3" else 84)
        sl = case == "self_loops"
        cap = {"cap1": 1, "cap8": 8}.get(case, 0)
    pos = pos.to(dev)
    a = bm.neighbor_list(pos, cell, cutoff, sl, cap)
    b = bm.neighbor_list(pos, cell, cutoff, sl, -1)
    for x, y, name in zip(a, b, ("edge_index", "vectors", "row_offsets")):
        assert torch.equal(x, y), name
    s, d, v = onl.cell_list(pos.cpu().numpy(), cell.numpy(), cutoff, sl)
    np.testing.assert_array_equal(a[0].cpu().numpy(), np.stack([s, d]))
    np.testing.assert_array_equal(a[1].cpu().numpy(), v)
