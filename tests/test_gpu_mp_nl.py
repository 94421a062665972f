"""GPU parity: fused SH+TP(+scatter), CSR conversion and the neighbor list.

Float outputs within 1e-5 normwise of the float64 oracle; neighbor lists
bit-exact (indices and fp32 vectors) against the C restatement of the
reference cell list after sorting by (i, j); CSR bit-exact.
"""
import ctypes
import os

import numpy as np
import pytest
import torch

from helpers import dst_sorted_edges, gen, normwise_err, periodic_box, unit_vectors
from oracle import mp as omp
from oracle import nl as onl

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(REPO, "batmobile-evo_amd", "lib", "libbatmobile_hip.so")
NL_LIB = os.path.join(REPO, "batmobile-evo_amd", "lib", "libbatteries_neighbor.so")


def _random_graph(n, e, c, seed):
    vec = unit_vectors(e, seed)
    x = torch.randn(n, c, 16, generator=gen(seed + 1))
    src = torch.randint(0, n, (e,), generator=gen(seed + 2))
    dst = torch.randint(0, n, (e,), generator=gen(seed + 3))
    return vec, x, src, dst


@pytest.mark.parametrize("n,e,c", [(100, 1000, 16), (50, 333, 64), (20, 77, 5), (10, 64, 128), (7, 1, 1)])
def test_fused_sh_tp_simple(bm, dev, n, e, c):
    vec, x, src, _ = _random_graph(n, e, c, 100 + c)
    msg = bm.fused_sh_tp_simple(vec.to(dev), x.to(dev), src.to(dev)).cpu().numpy()
    want = omp.fused_sh_tp_simple(vec.double().numpy(), x.double().numpy(), src.numpy())
    assert msg.shape == (e, c, 16)
    assert normwise_err(msg, want) <= 1e-5


def test_fused_vs_unfused_composition(bm, dev):
    """benchmarks/benchmark_fused_sh_tp.py:114-156: fused == SH -> gather -> TP_simple."""
    n, e, c = 300, 4000, 32
    vec, x, src, dst = _random_graph(n, e, c, 7)
    vec, x, src = vec.to(dev), x.to(dev), src.to(dev)
    fused = bm.fused_sh_tp_simple(vec, x, src)
    y = bm.spherical_harmonics(vec, 3)
    unf = bm.tensor_product_simple(x[src].reshape(e * c, 16),
                                   y.unsqueeze(1).expand(-1, c, -1).reshape(e * c, 16)).reshape(e, c, 16)
    assert (fused - unf).abs().max().item() <= 1e-4


@pytest.mark.parametrize("n,e,c,normalize", [(500, 6000, 64, False), (200, 3000, 16, True),
                                             (64, 500, 3, False), (33, 2000, 80, True)])
def test_sh_tp_scatter_random_graph(bm, dev, n, e, c, normalize):
    vec, x, src, dst = _random_graph(n, e, c, 9)
    if normalize:
        vec = vec * (1.0 + torch.rand(e, 1, generator=gen(5)) * 4.0)
    order = torch.argsort(dst, stable=True)
    rp = torch.zeros(n + 1, dtype=torch.int64)
    rp[1:] = torch.cumsum(torch.bincount(dst, minlength=n), 0)
    # permuted edge data (perm = CSR order), as fused_message_passing_simple uses it
    out = bm.sh_tp_scatter(vec.to(dev), x.to(dev), src.to(dev), rp.to(dev), order.to(dev), normalize)
    want = omp.sh_tp_scatter(vec.double().numpy(), x.double().numpy(), src.numpy(), dst.numpy(), n,
                             normalize=normalize)
    assert normwise_err(out.cpu(), want) <= 1e-5
    # the same edges stored in CSR order, no permutation
    out2 = bm.sh_tp_scatter(vec[order].to(dev), x.to(dev), src[order].to(dev), rp.to(dev), None, normalize)
    assert torch.equal(out, out2)


def test_sh_tp_scatter_empty_rows_and_edges(bm, dev):
    n, c = 40, 16
    x = torch.randn(n, c, 16, generator=gen(3)).to(dev)
    # odd destinations have no edges; destination 6 has 153 edges (> one 64-edge batch)
    dst = torch.cat([torch.arange(0, n, 2).repeat_interleave(3), torch.full((150,), 6)])
    dst, _ = torch.sort(dst)
    e = dst.numel()
    src = torch.randint(0, n, (e,), generator=gen(4))
    vec = unit_vectors(e, 5)
    rp = torch.zeros(n + 1, dtype=torch.int64)
    rp[1:] = torch.cumsum(torch.bincount(dst, minlength=n), 0)
    out = bm.sh_tp_scatter(vec.to(dev), x, src.to(dev), rp.to(dev)).cpu()
    want = omp.sh_tp_scatter(vec.double().numpy(), x.cpu().double().numpy(), src.numpy(), dst.numpy(), n)
    assert normwise_err(out, want) <= 1e-5
    assert torch.count_nonzero(out[1::2]).item() == 0
    # no edges at all -> zeros
    z = bm.sh_tp_scatter(vec[:0].to(dev), x, src[:0].to(dev), torch.zeros(n + 1, dtype=torch.int64, device=dev))
    assert torch.count_nonzero(z).item() == 0 and tuple(z.shape) == (n, c, 16)
    # no source rows and no edges -> zeros for every destination (simple and weighted)
    rp0 = torch.zeros(n + 1, dtype=torch.int64, device=dev)
    z = bm.sh_tp_scatter(vec[:0].to(dev), x[:0], src[:0].to(dev), rp0)
    assert torch.count_nonzero(z).item() == 0 and tuple(z.shape) == (n, c, 16)
    w = torch.randn(34, c, 8, generator=gen(6)).to(dev)
    z = bm.sh_tp_scatter_weighted(vec[:0].to(dev), x[:0], w, src[:0].to(dev), rp0)
    assert torch.count_nonzero(z).item() == 0 and tuple(z.shape) == (n, 8, 16)


def test_edge_index_to_csr(bm, dev):
    n, e = 1000, 30000
    ei = torch.stack([torch.randint(0, n, (e,), generator=gen(1)), torch.randint(0, n - 10, (e,), generator=gen(2))])
    rp, ci = bm.edge_index_to_csr(ei.to(dev), n)
    wrp, wci = omp.edge_index_to_csr(ei.numpy(), n)
    np.testing.assert_array_equal(rp.cpu().numpy(), wrp)
    np.testing.assert_array_equal(ci.cpu().numpy(), wci)
    rp0, ci0 = bm.edge_index_to_csr(ei[:, :0].to(dev), 7)
    assert rp0.cpu().tolist() == [0] * 8 and ci0.numel() == 0


def test_edge_index_to_csr_row_lengths(bm, dev):
    """Rows of 1, 63, 64, 65, 300 (several register chunks per lane) and 600 entries (past
    the register sort) next to random short rows, edges in a shuffled order: bit-exact
    against the stable sort of the oracle."""
    n = 200
    tgt = torch.cat([torch.full((600,), 0), torch.full((300,), 1), torch.full((64,), 2),
                     torch.full((65,), 3), torch.full((63,), 4), torch.full((1,), 5),
                     torch.randint(6, n, (5000,), generator=gen(61))])
    tgt = tgt[torch.randperm(tgt.numel(), generator=gen(62))]
    src = torch.randint(0, n, (tgt.numel(),), generator=gen(63))
    ei = torch.stack([src, tgt])
    rp, ci = bm.edge_index_to_csr(ei.to(dev), n)
    wrp, wci = omp.edge_index_to_csr(ei.numpy(), n)
    np.testing.assert_array_equal(rp.cpu().numpy(), wrp)
    np.testing.assert_array_equal(ci.cpu().numpy(), wci)


def test_fused_message_passing_simple(bm, dev):
    n, e, c = 400, 8000, 32
    vec, x, src, dst = _random_graph(n, e, c, 21)
    ei = torch.stack([src, dst]).to(dev)
    rp, ci = bm.edge_index_to_csr(ei, n)
    out = bm.fused_message_passing_simple(x.to(dev), vec.to(dev), ei, rp, ci).cpu()
    want = omp.scatter_add(omp.fused_sh_tp_simple(vec.double().numpy(), x.double().numpy(), src.numpy()),
                           dst.numpy(), n)
    assert normwise_err(out, want) <= 1e-5
    # and against the reference's own composition: fused_sh_tp_simple -> index_add_
    msg = bm.fused_sh_tp_simple(vec.to(dev), x.to(dev), src.to(dev))
    ref = torch.zeros(n, c, 16, device=dev).index_add_(0, dst.to(dev), msg).cpu()
    assert normwise_err(out, ref.numpy()) <= 1e-5


def test_fused_message_passing_dense_weights(bm, dev):
    n, e, cin, cout = 120, 2000, 16, 24
    vec = unit_vectors(e, 31)
    x = torch.randn(n, cin, 16, generator=gen(32))
    w = torch.randn(cin, cout, generator=gen(33)) / 4.0
    tgt, _ = torch.sort(torch.randint(0, n, (e,), generator=gen(34)))
    rp = torch.zeros(n + 1, dtype=torch.int64)
    rp[1:] = torch.cumsum(torch.bincount(tgt, minlength=n), 0)
    col = torch.randint(0, n, (e,), generator=gen(35))
    out = bm.fused_message_passing(x.to(dev), vec.to(dev), w.to(dev), rp.to(dev), col.to(dev)).cpu()
    want = omp.fused_message_passing(x.double().numpy(), vec.double().numpy(), w.double().numpy(),
                                     rp.numpy(), col.numpy())
    assert normwise_err(out, want) <= 1e-5


def _nl_gpu(bm, dev, pos, cell, cutoff=5.0, self_loops=False):
    ei, vec, off = bm.neighbor_list(pos.to(dev), cell, cutoff, self_loops)
    return ei.cpu().numpy(), vec.cpu().numpy(), off.cpu().numpy()


@pytest.mark.parametrize("n", [100, 1000, 5000, 50000])
def test_neighbor_list_bit_exact(bm, dev, n):
    pos, cell = periodic_box(n, 3 if n == 5000 else n)
    ei, vec, off = _nl_gpu(bm, dev, pos, cell)
    s, d, v = onl.cell_list(pos.numpy(), cell.numpy(), 5.0)
    np.testing.assert_array_equal(ei[0], s)
    np.testing.assert_array_equal(ei[1], d)
    np.testing.assert_array_equal(vec, v)      # bit-exact fp32
    np.testing.assert_array_equal(off, np.concatenate([[0], np.cumsum(np.bincount(s, minlength=n))]))
    if n <= 1000:
        bs, bd, bv = onl.brute_force(pos.numpy(), cell.numpy(), 5.0)
        np.testing.assert_array_equal(ei[0], bs)
        np.testing.assert_array_equal(vec, bv)


@pytest.mark.parametrize("n,box", [(8192, None), (8193, None), (500, 100.0), (0, 30.0)])
def test_neighbor_list_binning_paths(bm, dev, n, box):
    """Systems of up to 8192 atoms in up to 4096 bins are binned by one workgroup, larger
    ones by the multi-kernel sequence: both sides of each limit, bit-exact."""
    if box is None:
        pos, cell = periodic_box(n, n)
    else:
        pos = torch.rand(n, 3, generator=gen(n + 1)) * box
        cell = torch.diag(torch.tensor([box, box, box]))
    ei, vec, off = _nl_gpu(bm, dev, pos, cell)
    s, d, v = onl.cell_list(pos.numpy(), cell.numpy(), 5.0)
    np.testing.assert_array_equal(ei, np.stack([s, d]))
    np.testing.assert_array_equal(vec, v)
    assert off.shape == (n + 1,) and off[0] == 0 and off[-1] == len(s)


def test_neighbor_list_reference_cases(bm, dev):
    """The reference's correctness cases (tests/test_neighbor_list.cu:264-266: N = 100, 500,
    1000, density 0.05, cutoff 5, std::mt19937(42) positions from tests/golden/): bit-exact
    against the C restatement and against brute force."""
    from test_oracle_nl_mp import reference_nl_cases
    cases, cutoff = reference_nl_cases()
    for n, box, pos in cases:
        print(f"reference NL case N={n}", flush=True)
        cell = torch.diag(torch.tensor([box, box, box], dtype=torch.float32))
        ei, vec, off = _nl_gpu(bm, dev, torch.from_numpy(pos), cell, cutoff)
        s, d, v = onl.cell_list(pos, cell.numpy(), cutoff)
        np.testing.assert_array_equal(ei, np.stack([s, d]))
        np.testing.assert_array_equal(vec, v)
        bs, bd, bv = onl.brute_force(pos, cell.numpy(), cutoff)
        np.testing.assert_array_equal(ei, np.stack([bs, bd]))
        np.testing.assert_array_equal(vec, bv)


def test_neighbor_list_dense_long_rows_and_chunked_cells(bm, dev):
    """3000 atoms in a 12 A box with r_c = 4 A: 3 bins per axis, so every cell's
    27-cell candidate list is the whole system (> 2048 staged per chunk), and
    rows hold ~300 neighbours (> 64: ranked in registers, five entries per lane)."""
    pos = torch.rand(3000, 3, generator=gen(7)) * 12.0
    cell = torch.diag(torch.tensor([12.0, 12.0, 12.0]))
    ei, vec, off = _nl_gpu(bm, dev, pos, cell, 4.0)
    assert np.diff(off).max() > 64
    s, d, v = onl.cell_list(pos.numpy(), cell.numpy(), 4.0)
    np.testing.assert_array_equal(ei, np.stack([s, d]))
    np.testing.assert_array_equal(vec, v)
    bs, bd, bv = onl.brute_force(pos.numpy(), cell.numpy(), 4.0)
    np.testing.assert_array_equal(ei, np.stack([bs, bd]))


def test_neighbor_list_bin_over_1024_atoms_and_rows_over_512(bm, dev):
    """1100 atoms packed into one 5 A cell of a 30 A box (6 bins per axis) among 1500
    spread over the box: that bin holds > 1024 atoms (the bin sort ranks them from
    memory instead of LDS) and its atoms' rows hold > 512 neighbours (ranked from
    memory and written out to the int64 arrays of both torch layouts), the rows of
    atoms near it 65..512 (ranked in registers).  Both layouts bit-exact against the C
    restatement and brute force; the C ABI's in-place int32 sort of the same system is
    test_neighbor_list_c_abi_long_rows_in_place."""
    g = gen(11)
    dense = torch.rand(1100, 3, generator=g) * 4.6 + 0.2
    spread = torch.rand(1500, 3, generator=g) * 30.0
    pos = torch.cat([spread[:700], dense, spread[700:]])
    cell = torch.diag(torch.tensor([30.0, 30.0, 30.0]))
    ei, vec, off = _nl_gpu(bm, dev, pos, cell, 5.0)
    deg = np.diff(off)
    assert deg.max() > 512 and ((deg > 64) & (deg <= 512)).any()
    s, d, v = onl.cell_list(pos.numpy(), cell.numpy(), 5.0)
    np.testing.assert_array_equal(ei, np.stack([s, d]))
    np.testing.assert_array_equal(vec, v)
    bs, bd, bv = onl.brute_force(pos.numpy(), cell.numpy(), 5.0)
    np.testing.assert_array_equal(ei, np.stack([bs, bd]))
    np.testing.assert_array_equal(vec, bv)
    src, dst, gvec, goff, _ = bm.neighbor_graph(pos.to(dev), cell, 5.0, False)
    np.testing.assert_array_equal(src.cpu().numpy(), d)
    np.testing.assert_array_equal(dst.cpu().numpy(), s)
    np.testing.assert_array_equal(gvec.cpu().numpy(), -v)
    np.testing.assert_array_equal(goff.cpu().numpy(), off)


def test_neighbor_list_small_box_self_loops_and_lattice(bm, dev):
    pos, cell = periodic_box(40, 8)           # box ~ 8.8 A: 3 bins of < r_c
    ei, vec, _ = _nl_gpu(bm, dev, pos, cell, 5.0, True)
    s, d, v = onl.cell_list(pos.numpy(), cell.numpy(), 5.0, True)
    np.testing.assert_array_equal(ei, np.stack([s, d]))
    np.testing.assert_array_equal(vec, v)
    g = torch.arange(6, dtype=torch.float32) * 2.0 + 0.5
    lat = torch.stack(torch.meshgrid(g, g, g, indexing="ij"), -1).reshape(-1, 3)
    ei, vec, _ = _nl_gpu(bm, dev, lat, torch.diag(torch.tensor([12.0, 12.0, 12.0])), 2.0)
    assert np.bincount(ei[0], minlength=216).tolist() == [6] * 216


@pytest.mark.parametrize("n", [0, 1, 5, 16383, 16384, 16385, 50001, 300007])
def test_exclusive_scan_c_abi(bm, dev, n):
    """batteries_exclusive_scan_i64: out[i] = sum in[:i], out[n] = total, bit-exact; sizes
    around the 16384-element tile, values up to 2^40 (sums beyond 32 bits)."""
    lib = ctypes.CDLL(LIB)
    lib.batteries_exclusive_scan_i64.restype = ctypes.c_int
    lib.batteries_exclusive_scan_i64.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                                 ctypes.c_void_p]
    g = gen(900 + n)
    v = torch.randint(0, 1000, (n,), generator=g, dtype=torch.int64)
    if n:
        v[torch.randint(0, n, (max(1, n // 97),), generator=g)] = 1 << 40
    vd = v.to(dev)
    out = torch.full((n + 1,), -7, dtype=torch.int64, device=dev)
    torch.cuda.synchronize()
    assert lib.batteries_exclusive_scan_i64(vd.data_ptr() if n else None, out.data_ptr(), n, None) == 0
    torch.cuda.synchronize()
    want = np.zeros(n + 1, dtype=np.int64)
    want[1:] = np.cumsum(v.numpy())
    np.testing.assert_array_equal(out.cpu().numpy(), want)


class _NlResult(ctypes.Structure):
    _fields_ = [("edge_index", ctypes.c_void_p), ("edge_vectors", ctypes.c_void_p),
                ("num_edges", ctypes.c_int64), ("d_edge_index", ctypes.c_void_p),
                ("d_edge_vectors", ctypes.c_void_p)]


def _nl_c_abi(libpath, dev, pos, cell, cutoff=5.0):
    """neighbor_list_cuda through ctypes, as reference benchmarks/benchmark_neighbor_list.py:18-47
    uses it: int32 edge_index [2, E] and vectors copied out of the library-owned buffers."""
    lib = ctypes.CDLL(libpath)
    lib.neighbor_list_cuda.restype = ctypes.c_int
    lib.neighbor_list_cuda.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_float,
                                       ctypes.c_bool, ctypes.POINTER(_NlResult), ctypes.c_void_p]
    lib.neighbor_list_free.argtypes = [ctypes.POINTER(_NlResult)]
    n = pos.shape[0]
    pd, cd = pos.to(dev).contiguous(), cell.to(dev).contiguous()
    torch.cuda.synchronize()
    res = _NlResult()
    rc = lib.neighbor_list_cuda(pd.data_ptr(), cd.data_ptr(), n, cutoff, False, ctypes.byref(res), None)
    assert rc == 0
    e = res.num_edges
    ei = torch.empty(2 * e, dtype=torch.int32, device=dev)
    vv = torch.empty(e * 3, dtype=torch.float32, device=dev)
    hip = ctypes.CDLL("libamdhip64.so.7")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    assert hip.hipMemcpy(ei.data_ptr(), res.d_edge_index, 8 * e, 3) == 0
    assert hip.hipMemcpy(vv.data_ptr(), res.d_edge_vectors, 12 * e, 3) == 0
    lib.neighbor_list_free(ctypes.byref(res))
    assert res.num_edges == 0 and not res.d_edge_index
    return ei.cpu().numpy().reshape(2, e), vv.cpu().numpy().reshape(e, 3)


@pytest.mark.parametrize("libpath", [NL_LIB, LIB])
def test_neighbor_list_reference_c_abi(bm, dev, libpath):
    """ctypes use as in reference benchmarks/benchmark_neighbor_list.py:18-47, through the
    reference's library name (libbatteries_neighbor.so) and the full library."""
    pos, cell = periodic_box(2000, 4)
    ei, vv = _nl_c_abi(libpath, dev, pos, cell)
    s, d, v = onl.cell_list(pos.numpy(), cell.numpy(), 5.0)
    np.testing.assert_array_equal(ei[0], s)
    np.testing.assert_array_equal(ei[1], d)
    np.testing.assert_array_equal(vv, v)


@pytest.mark.parametrize("box", [30.0, 90.0])
def test_neighbor_list_c_abi_long_rows_in_place(bm, dev, box):
    """The dense cluster of test_neighbor_list_bin_over_1024_atoms_and_rows_over_512 through
    neighbor_list_cuda.  In a 30 A box (216 cells) it takes the cell kernels, whose slab rows
    (sized from the mean density) are far shorter than the cluster's rows: those are found
    again by the row kernel.  In a 90 A box (5832 cells, past the cell kernels' 4096) it
    takes the general passes, whose int32 layout sorts rows in place: rows of 65..512
    neighbours ranked in registers, longer ones ranked from memory and permuted by cycles
    (ranks held in the source column, which is restored)."""
    g = gen(11)
    dense = torch.rand(1100, 3, generator=g) * 4.6 + 0.2
    spread = torch.rand(1500, 3, generator=g) * box
    pos = torch.cat([spread[:700], dense, spread[700:]])
    cell = torch.diag(torch.tensor([box, box, box]))
    ei, vv = _nl_c_abi(LIB, dev, pos, cell)
    s, d, v = onl.cell_list(pos.numpy(), cell.numpy(), 5.0)
    assert np.bincount(s).max() > 512
    np.testing.assert_array_equal(ei, np.stack([s, d]))
    np.testing.assert_array_equal(vv, v)


def test_config4_scatter_full_size(bm, dev):
    """configs[3] geometry: N = 5000, ~30 neighbours, C = 64, edges sorted by destination."""
    pos, cell = periodic_box(5000, 3)
    ei, vec, off = bm.neighbor_list(pos.to(dev), cell, 5.0, False)
    src, dst, v = dst_sorted_edges(ei[0], ei[1], vec)
    x = torch.randn(5000, 64, 16, generator=gen(13)).to(dev)
    out = bm.sh_tp_scatter(v, x, src, off, None, True)
    want = omp.sh_tp_scatter(v.cpu().double().numpy(), x.cpu().double().numpy(), src.cpu().numpy(),
                             dst.cpu().numpy(), 5000, normalize=True)
    assert normwise_err(out.cpu(), want) <= 1e-5
    # deterministic: bitwise identical on a second run
    assert torch.equal(out, bm.sh_tp_scatter(v, x, src, off, None, True))


@pytest.mark.parametrize("n", [5000, 50000, 40])
def test_spatial_order_is_a_morton_permutation(bm, dev, n):
    pos, cell = periodic_box(n, 3)
    order = bm.spatial_order(pos.to(dev), cell).cpu().numpy()
    assert np.array_equal(np.sort(order), np.arange(n))
    L = float(cell[0, 0])
    bits = 1                              # 2^bits cells per axis: the largest bits <= 5
    while bits < 5 and 8 ** (bits + 1) <= n:   # with 8^bits <= N
        bits += 1
    q = np.clip((pos.numpy() / L * (1 << bits)).astype(int), 0, (1 << bits) - 1)

    def spread(v):
        r = np.zeros_like(v)
        for b in range(bits):
            r |= ((v >> b) & 1) << (3 * b)
        return r

    key = spread(q[:, 0]) | (spread(q[:, 1]) << 1) | (spread(q[:, 2]) << 2)
    k = key[order]
    assert (np.diff(k) >= 0).all()
    same = np.diff(k) == 0
    assert (np.diff(order)[same] > 0).all()     # ascending atom index inside a cell


@pytest.mark.parametrize("n,c", [(5000, 64), (1500, 16), (700, 128), (40, 5)])
def test_scheduled_scatter_equals_index_order(bm, dev, n, c):
    import batmobile
    pos, cell = periodic_box(n, 11 + n)
    g = batmobile.Graph(pos.to(dev), cell, 5.0, c)
    x = torch.randn(n, c, 16, generator=gen(12)).to(dev)
    a = g.sh_tp_scatter(x)
    b = g.sh_tp_scatter_index_order(x)
    # each destination is summed by one wave in CSR order in both: bitwise identical
    assert torch.equal(a, b)
    assert int(g.row_dst.ge(0).sum()) == n
    want = omp.sh_tp_scatter(g.vec.cpu().double().numpy(), x.cpu().double().numpy(), g.src.cpu().numpy(),
                             g.dst.cpu().numpy(), n, normalize=True)
    assert normwise_err(a.cpu(), want) <= 1e-5


def test_schedule_is_a_balanced_partition(bm, dev):
    """Every destination in exactly one slot, edge_perm a permutation, workgroup
    edge counts within 10% of the mean at the configs[3] density."""
    import batmobile
    n, c = 5000, 64
    pos, cell = periodic_box(n, 3)
    g = batmobile.Graph(pos.to(dev), cell, 5.0, c)
    rdst = g.row_dst.cpu()
    assert torch.equal(torch.sort(rdst[rdst >= 0]).values, torch.arange(n))
    assert torch.equal(torch.sort(g.edge_perm.cpu()).values, torch.arange(g.num_edges))
    R, nb = g.rows_per_block, g.n_blocks
    rps = g.row_ptr_s.cpu()
    per_wg = (rps[torch.arange(1, nb + 1) * R] - rps[torch.arange(nb) * R]).double()
    assert int(rps[-1]) == g.num_edges
    assert per_wg.max().item() <= 1.10 * per_wg.mean().item()
    # the slot degrees are the row lengths of the scheduled destinations
    deg = (g.row_ptr[1:] - g.row_ptr[:-1]).cpu()
    slot_deg = rps[1:] - rps[:-1]
    ok = rdst >= 0
    assert torch.equal(slot_deg[ok], deg[rdst[ok]])
    assert int(slot_deg[~ok].abs().sum()) == 0


@pytest.mark.parametrize("c", [64, 24])
def test_schedule_with_skewed_degrees(bm, dev, c):
    """One destination with more edges than a workgroup's share, rows of one
    edge and isolated destinations: the scheduled kernel still matches the
    oracle and the index-order kernel bit for bit."""
    n = 3000
    g = gen(61)
    hub_src = torch.randint(0, n, (900,), generator=g)
    hub_dst = torch.zeros(900, dtype=torch.int64)                 # destination 0: 900 edges
    one_dst = torch.arange(1, 600)                                # destinations 1..599: one edge
    one_src = torch.randint(0, n, (599,), generator=g)
    mid_dst = torch.randint(600, 2000, (40000,), generator=g)     # 600..1999: ~29 edges each
    mid_src = torch.randint(0, n, (40000,), generator=g)          # 2000..2999: no edges
    src = torch.cat([hub_src, one_src, mid_src])
    dst = torch.cat([hub_dst, one_dst, mid_dst])
    e = src.numel()
    vec = unit_vectors(e, 62) * (1.0 + torch.rand(e, 1, generator=g))
    x = torch.randn(n, c, 16, generator=gen(63))
    ei = torch.stack([src, dst]).to(dev)
    rp, ci = bm.edge_index_to_csr(ei, n)
    order = torch.randperm(n, generator=gen(64)).to(dev)
    rps, ep, rdst, nb, rpb = bm.mp_schedule(rp, order, c, ci)
    out = bm.sh_tp_scatter_scheduled(vec.to(dev), x.to(dev), ei[0].contiguous(), rps, ep, rdst, nb,
                                     rpb, n, True)
    idx = bm.sh_tp_scatter(vec.to(dev), x.to(dev), ei[0].contiguous(), rp, ci, True)
    assert torch.equal(out, idx)
    want = omp.sh_tp_scatter(vec.double().numpy(), x.double().numpy(), src.numpy(), dst.numpy(), n,
                             normalize=True)
    assert normwise_err(out.cpu(), want) <= 1e-5
    assert out[2000:].abs().max().item() == 0.0
    assert torch.equal(torch.sort(rdst[rdst >= 0].cpu()).values, torch.arange(n))


def _schedule_groups_expected(deg, P, Q, R):
    """Group bounds of the spatial schedule from the degrees in processing order: each
    group ends where the cumulative edge count reaches its share of the edges (or one
    position earlier when that is closer), then the ends are clamped in order so that
    every group fits its Qg * R slots and leaves room for the groups after it."""
    n = len(deg)
    cum = np.concatenate([[0], np.cumsum(deg, dtype=np.int64)])
    G = (P + Q - 1) // Q
    gb = np.zeros(8 * G + 1, dtype=np.int64)
    start = 0
    for gi in range(8 * G):
        x, gen_ = divmod(gi, G)
        qg = min(Q, P - gen_ * Q)
        w_end = x * P + gen_ * Q + qg
        target = float(cum[n]) * float(w_end) / (8.0 * float(P))
        lo = int(np.searchsorted(cum[:n].astype(np.float64), target, side="left"))
        if lo > 0 and target - float(cum[lo - 1]) < float(cum[lo]) - target:
            lo -= 1
        low = max(start, n - (8 * P - w_end) * R)
        high = min(n, start + qg * R)
        gb[gi + 1] = max(low, min(high, lo))
        start = int(gb[gi + 1])
    return gb


@pytest.mark.parametrize("case", ["box5000", "box16384", "box16385", "box20000", "skewed", "empty"])
def test_schedule_groups_through_c_abi(bm, dev, case):
    """batteries_mp_schedule's processing-order degrees, their running sums and the group
    bounds (read from its workspace: degm [N], cum [N + 1], gb [8 G + 1]) against a numpy
    restatement, and its slot offsets against the running sums of the slot degrees, on both
    sides of the one-workgroup preparation's limit of 16,384 destinations."""
    import batmobile
    c = 64
    if case.startswith("box"):
        n = int(case[3:])
        pos, cell = periodic_box(n, 5 + n % 97)
        g = batmobile.Graph(pos.to(dev), cell, 5.0, c)
        row_ptr, order, e = g.row_ptr, g.order, g.num_edges
    elif case == "skewed":
        n = 3000
        dst = torch.cat([torch.zeros(900, dtype=torch.int64), torch.arange(1, 600),
                         torch.randint(600, 2000, (40000,), generator=gen(71))])
        src = torch.randint(0, n, (dst.numel(),), generator=gen(72))
        row_ptr, _ = bm.edge_index_to_csr(torch.stack([src, dst]).to(dev), n)
        order = torch.randperm(n, generator=gen(73)).to(dev)
        e = dst.numel()
    else:
        n, e = 0, 0
        row_ptr = torch.zeros(1, dtype=torch.int64, device=dev)
        order = torch.zeros(1, dtype=torch.int64, device=dev)
    lib = ctypes.CDLL(LIB)
    nb, rpb = ctypes.c_int(), ctypes.c_int()
    assert lib.batteries_mp_schedule_shape(ctypes.c_int64(n), ctypes.c_int(c), ctypes.byref(nb),
                                           ctypes.byref(rpb)) == 0
    nb, rpb = nb.value, rpb.value
    lib.batteries_mp_schedule_workspace_bytes.restype = ctypes.c_size_t
    wsb = lib.batteries_mp_schedule_workspace_bytes(ctypes.c_int(nb), ctypes.c_int(rpb))
    ws = torch.full((wsb // 8,), -7, dtype=torch.int64, device=dev)
    ns = nb * rpb
    rps = torch.empty(ns + 1, dtype=torch.int64, device=dev)
    rdst = torch.empty(ns, dtype=torch.int64, device=dev)
    ep = torch.empty(max(e, 1), dtype=torch.int64, device=dev)
    P = nb // 8
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    Q = min(P, max(1, 2 * cus // ((c + 63) // 64) // 8), 256)
    G = (P + Q - 1) // Q
    stream = torch.cuda.current_stream().cuda_stream
    lib.batteries_mp_schedule.restype = ctypes.c_int
    rc = lib.batteries_mp_schedule(
        ctypes.c_void_p(row_ptr.data_ptr()), None, ctypes.c_void_p(order.data_ptr()),
        ctypes.c_int64(n), ctypes.c_int64(e), ctypes.c_int(c), ctypes.c_int(nb), ctypes.c_int(rpb),
        ctypes.c_void_p(rps.data_ptr()), ctypes.c_void_p(rdst.data_ptr()),
        ctypes.c_void_p(ep.data_ptr()), ctypes.c_void_p(ws.data_ptr()), ctypes.c_size_t(wsb),
        ctypes.c_void_p(stream))
    torch.cuda.synchronize()
    assert rc == 0
    w = ws.cpu().numpy()
    rp = row_ptr.cpu().numpy()
    od = order.cpu().numpy()[:n]
    deg = (rp[1:] - rp[:-1])[od] if n else np.zeros(0, dtype=np.int64)
    assert np.array_equal(w[:n], deg)
    assert np.array_equal(w[n:2 * n + 1], np.concatenate([[0], np.cumsum(deg)]))
    gb = w[2 * n + 1: 2 * n + 1 + 8 * G + 1]
    assert np.array_equal(gb, _schedule_groups_expected(deg, P, Q, rpb))
    # and the schedule built on them covers every destination once, its slot offsets
    # the running sums of the scheduled rows' degrees
    r = rdst.cpu()
    assert torch.equal(torch.sort(r[r >= 0]).values, torch.arange(n))
    slot_deg = torch.zeros(ns, dtype=torch.int64)
    slot_deg[r >= 0] = torch.from_numpy(rp[1:] - rp[:-1])[r[r >= 0]]
    assert torch.equal(rps.cpu(), torch.cat([torch.zeros(1, dtype=torch.int64), torch.cumsum(slot_deg, 0)]))
    assert int(rps[-1]) == e


def test_schedule_with_col_perm_matches_fused_message_passing_simple(bm, dev):
    n, e, c = 900, 20000, 32
    vec, x, src, dst = _random_graph(n, e, c, 51)
    ei = torch.stack([src, dst]).to(dev)
    rp, ci = bm.edge_index_to_csr(ei, n)
    order = torch.randperm(n, generator=gen(52)).to(dev)
    rps, ep, rdst, nb, rpb = bm.mp_schedule(rp, order, c, ci)
    out = bm.sh_tp_scatter_scheduled(vec.to(dev), x.to(dev), ei[0].contiguous(), rps, ep, rdst, nb, rpb, n,
                                     False)
    ref = bm.fused_message_passing_simple(x.to(dev), vec.to(dev), ei, rp, ci)
    assert torch.equal(out, ref)


@pytest.mark.parametrize("seed", range(24))
def test_scheduled_scatter_random_degree_patterns(bm, dev, seed):
    """Random graphs whose row lengths mix empty rows, one-edge rows, rows around the
    32- and 64-edge boundaries and long rows, in random orders: the scheduled kernel
    (gather indices read ahead across halves and batches) equals the index-order kernel
    bit for bit, and the oracle within 1e-5 on every fourth case."""
    g = torch.Generator().manual_seed(1000 + seed)
    n = int(torch.randint(1, 600, (1,), generator=g))
    c = [16, 64, 24, 80][seed % 4]
    kind = torch.randint(0, 6, (n,), generator=g)
    deg = torch.where(kind == 0, torch.zeros(n, dtype=torch.int64),
          torch.where(kind == 1, torch.ones(n, dtype=torch.int64),
          torch.where(kind == 2, torch.randint(28, 37, (n,), generator=g),
          torch.where(kind == 3, torch.randint(60, 69, (n,), generator=g),
          torch.where(kind == 4, torch.randint(2, 20, (n,), generator=g),
                      torch.randint(100, 300, (n,), generator=g))))))
    if seed % 3 == 0:
        deg[torch.rand(n, generator=g) < 0.5] = 0        # long runs of empty rows
    dst = torch.repeat_interleave(torch.arange(n), deg)
    e = int(dst.numel())
    src = torch.randint(0, n, (e,), generator=g)
    perm = torch.randperm(e, generator=g)                # edges in random order
    src, dst = src[perm], dst[perm]
    vec = unit_vectors(e, 2000 + seed) * (0.5 + torch.rand(e, 1, generator=g)) if e else torch.zeros(0, 3)
    x = torch.randn(n, c, 16, generator=g)
    ei = torch.stack([src, dst]).to(dev)
    rp, ci = bm.edge_index_to_csr(ei, n)
    order = torch.randperm(n, generator=g).to(dev)
    rps, ep, rdst, nb, rpb = bm.mp_schedule(rp, order, c, ci)
    out = bm.sh_tp_scatter_scheduled(vec.to(dev), x.to(dev), ei[0].contiguous(), rps, ep, rdst, nb, rpb,
                                     n, True)
    idx = bm.sh_tp_scatter(vec.to(dev), x.to(dev), ei[0].contiguous(), rp, ci, True)
    assert torch.equal(out, idx)
    assert out[deg.to(dev) == 0].abs().sum().item() == 0.0
    if seed % 4 == 0 and e:
        want = omp.sh_tp_scatter(vec.double().numpy(), x.double().numpy(), src.numpy(), dst.numpy(), n,
                                 normalize=True)
        assert normwise_err(out.cpu(), want) <= 1e-5


def test_scatter_batch_boundaries(bm, dev):
    """Index order with 11 destinations per workgroup (n = 512 * 11, C = 16) and
    degree patterns that put row ends on both sides of the 32- and 64-edge
    boundaries: rows of exactly 32, 64, 96 edges, a batch whose last edge closes a
    row, batches with more closing rows than staging slots (written as they
    close) next to staged ones, empty rows between, and single long rows."""
    patterns = [
        [64] + [0] * 10, [32] + [0] * 10, [33], [31], [63], [65], [96], [127], [128], [200],
        [1] * 11, [5] * 11, [10, 10, 10, 10, 10, 10, 4], [20, 20, 20, 4], [21, 21, 22],
        [64, 64, 64], [0, 0, 30, 0, 34, 0], [100, 1, 1, 1, 1, 1], [30] * 11,
        [16, 16, 16, 16, 16, 16, 16, 16], [3, 61, 3, 61], [0] * 11,
    ]
    n_wg = 512
    deg = []
    for k in range(n_wg):
        p = patterns[k % len(patterns)]
        deg += (p + [0] * 11)[:11]
    deg = torch.tensor(deg, dtype=torch.int64)
    n = deg.numel()
    c = 16
    dst = torch.repeat_interleave(torch.arange(n), deg)
    e = dst.numel()
    src = torch.randint(0, n, (e,), generator=gen(71))
    vec = unit_vectors(e, 72) * (0.5 + torch.rand(e, 1, generator=gen(73)))
    x = torch.randn(n, c, 16, generator=gen(74))
    rp = torch.zeros(n + 1, dtype=torch.int64)
    rp[1:] = torch.cumsum(deg, 0)
    out = bm.sh_tp_scatter(vec.to(dev), x.to(dev), src.to(dev), rp.to(dev), None, True)
    want = omp.sh_tp_scatter(vec.double().numpy(), x.double().numpy(), src.numpy(), dst.numpy(), n,
                             normalize=True)
    assert normwise_err(out.cpu(), want) <= 1e-5
    assert out[deg == 0].abs().max().item() == 0.0
    assert torch.equal(out, bm.sh_tp_scatter(vec.to(dev), x.to(dev), src.to(dev), rp.to(dev), None, True))


def _bin_coords_f32(pos, L, rc):
    """The cell list's bin coordinates in float32, with the cell-list kernels' operations
    (no contraction): t = p / L, wrapped p - floor(t) L, divided by the bin width."""
    L32, rc32 = np.float32(L), np.float32(rc)
    nb = max(3, int(L32 / rc32))
    inv = np.float32(1.0) / L32
    binw = L32 / np.float32(nb)
    p = pos.astype(np.float32)
    fl = (np.floor(p * inv).astype(np.float32) * L32).astype(np.float32)
    w = (p - fl).astype(np.float32)
    v = (w / binw).astype(np.int64)
    return np.clip(v, 0, nb - 1), nb


@pytest.mark.parametrize("n", [5000, 700, 20000])
def test_graph_order_is_a_serpentine_cell_order(bm, dev, n):
    """Graph.order: a permutation of the atoms, the cell list's cells along a serpentine
    path (x fastest, every other row and every other plane reversed) and the atoms of a
    cell in ascending index."""
    import batmobile
    pos, cell = periodic_box(n, 5)
    g = batmobile.Graph(pos.to(dev), cell, 5.0, 16)
    order = g.order.cpu().numpy()
    assert np.array_equal(np.sort(order), np.arange(n))
    b, nb = _bin_coords_f32(pos.numpy(), float(cell[0, 0]), 5.0)
    bx, by, bz = b[:, 0], b[:, 1], b[:, 2]
    py = np.where(bz % 2 == 1, nb - 1 - by, by)
    row = bz * nb + py
    px = np.where(row % 2 == 1, nb - 1 - bx, bx)
    path = row * nb + px                      # serpentine position of each atom's cell
    key = path[order] * n + order             # path position, then atom index
    assert (np.diff(key) > 0).all()


def test_graph_with_max_edges_matches_exact_build(bm, dev):
    """Graph(max_edges=...) builds without a host synchronisation into arrays of max_edges
    edges: the first E entries, the row pointers, the order and the schedule equal the exact
    build's, and the fused kernels give bit-identical results."""
    import batmobile
    pos, cell = periodic_box(5000, 3)
    pos = pos.to(dev)
    ex = batmobile.Graph(pos, cell, 5.0, 64)
    e = ex.num_edges
    cap = batmobile.Graph(pos, cell, 5.0, 64, max_edges=e + 1000)
    assert cap.src.numel() == e + 1000
    assert cap.num_edges == e
    cap.check()
    for a, b in ((cap.src[:e], ex.src), (cap.dst[:e], ex.dst), (cap.vec[:e], ex.vec),
                 (cap.row_ptr, ex.row_ptr), (cap.order, ex.order), (cap.row_ptr_s, ex.row_ptr_s),
                 (cap.row_dst, ex.row_dst), (cap.edge_perm[:e], ex.edge_perm)):
        assert torch.equal(a, b)
    x = torch.randn(5000, 64, 16, generator=gen(40)).to(dev)
    assert torch.equal(cap.sh_tp_scatter(x), ex.sh_tp_scatter(x))
    w = (torch.randn(34, 64, 64, generator=gen(41)) / 8.0).to(dev)
    assert torch.equal(cap.sh_tp_scatter(x, weights=w), ex.sh_tp_scatter(x, weights=w))
    assert torch.equal(cap.sh_tp_scatter_index_order(x), ex.sh_tp_scatter_index_order(x))
    cap.exact()
    assert cap.src.numel() == e and torch.equal(cap.src, ex.src)
    # exactly full
    full = batmobile.Graph(pos, cell, 5.0, 64, max_edges=e)
    full.check()
    assert torch.equal(full.sh_tp_scatter(x), ex.sh_tp_scatter(x))


@pytest.mark.parametrize("max_edges", [0, 1000, 150000])
def test_graph_with_too_few_max_edges_flags_and_stays_in_bounds(bm, dev, max_edges):
    """Edges beyond max_edges: check() raises, every row is empty (row pointers all zero), and
    the kernels that follow read nothing past the arrays (zero outputs)."""
    import batmobile
    pos, cell = periodic_box(5000, 3)   # about 150,480 edges
    g = batmobile.Graph(pos.to(dev), cell, 5.0, 64, max_edges=max_edges)
    with pytest.raises(RuntimeError, match="max_edges"):
        g.check()
    assert int(g.row_ptr.abs().sum().item()) == 0
    x = torch.randn(5000, 64, 16, generator=gen(42)).to(dev)
    assert torch.count_nonzero(g.sh_tp_scatter(x)).item() == 0
    w = (torch.randn(34, 64, 64, generator=gen(43)) / 8.0).to(dev)
    assert torch.count_nonzero(g.sh_tp_scatter(x, weights=w)).item() == 0


def test_graph_with_max_edges_and_no_atoms(bm, dev):
    import batmobile
    g = batmobile.Graph(torch.zeros(0, 3, device=dev), torch.diag(torch.tensor([20.0, 20.0, 20.0])),
                        5.0, 16, max_edges=10)
    g.check()
    assert g.num_edges == 0 and g.row_ptr.cpu().tolist() == [0]
