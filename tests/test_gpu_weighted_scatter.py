"""GPU parity: the weighted scatter (fused SH + weighted TP + scatter-add).

out[d] = sum_{e -> d} tensor_product(X[src_e], Y(v_e), W) with one W [34, C_in, C_out],
the reference interaction block's SH -> tensor_product -> scatter_add
(benchmarks/benchmark_e2e_mace.py:308-349).  Compared with the float64 oracle
composition (oracle.mp.weighted_message_passing) within 1e-5 normwise; at the full
configs[3] size through a sampled set of destinations, the reduction to the simple
scatter for identity mixing, and linearity in W.
"""
import numpy as np
import pytest
import torch

from helpers import gen, normwise_err, periodic_box, unit_vectors
from oracle import mp as omp

pytestmark = pytest.mark.gpu


def _csr(dst, n):
    order = torch.argsort(dst, stable=True)
    rp = torch.zeros(n + 1, dtype=torch.int64)
    rp[1:] = torch.cumsum(torch.bincount(dst, minlength=n), 0)
    return order, rp


def _weights(ci, co, seed):
    return torch.randn(34, ci, co, generator=gen(seed)) / np.sqrt(ci)


@pytest.mark.parametrize("n,e,ci,co,normalize", [
    (200, 3000, 32, 64, True),
    (150, 2500, 16, 16, False),
    (64, 900, 5, 3, True),      # channels below one 16-channel chunk
    (50, 700, 20, 70, True),    # a partial input chunk, two output-channel groups
    (33, 400, 48, 8, False),    # an odd number of input chunks
    (70, 1200, 128, 128, True),  # eight input chunks in four groups, two output-channel tiles
])
def test_weighted_scatter_random_graph(bm, dev, n, e, ci, co, normalize):
    vec = unit_vectors(e, 40 + ci)
    if normalize:
        vec = vec * (0.5 + torch.rand(e, 1, generator=gen(41)) * 3.0)
    x = torch.randn(n, ci, 16, generator=gen(42))
    w = _weights(ci, co, 43)
    src = torch.randint(0, n, (e,), generator=gen(44))
    dst = torch.randint(0, n, (e,), generator=gen(45))
    order, rp = _csr(dst, n)
    want = omp.weighted_message_passing(vec.double().numpy(), x.double().numpy(),
                                        w.double().numpy(), src.numpy(), dst.numpy(), n,
                                        normalize=normalize)
    # edge data in its original order, reached through perm
    out = bm.sh_tp_scatter_weighted(vec.to(dev), x.to(dev), w.to(dev), src.to(dev), rp.to(dev),
                                    order.to(dev), None, normalize)
    assert out.shape == (n, co, 16)
    assert normwise_err(out.cpu(), want) <= 1e-5
    # the same edges stored in CSR order, destinations processed in a shuffled order
    shuffle = torch.randperm(n, generator=gen(46))
    out2 = bm.sh_tp_scatter_weighted(vec[order].to(dev), x.to(dev), w.to(dev),
                                     src[order].to(dev), rp.to(dev), None, shuffle.to(dev),
                                     normalize)
    assert torch.equal(out, out2)


def test_weighted_scatter_empty_rows_long_rows_and_no_edges(bm, dev):
    n, ci, co = 30, 32, 64
    x = torch.randn(n, ci, 16, generator=gen(50))
    w = _weights(ci, co, 51)
    # odd destinations have no edges; destination 4 has 203 edges (several 64-edge groups)
    dst = torch.cat([torch.arange(0, n, 2).repeat_interleave(3), torch.full((200,), 4)])
    dst, _ = torch.sort(dst)
    e = dst.numel()
    src = torch.randint(0, n, (e,), generator=gen(52))
    vec = unit_vectors(e, 53)
    _, rp = _csr(dst, n)
    out = bm.sh_tp_scatter_weighted(vec.to(dev), x.to(dev), w.to(dev), src.to(dev), rp.to(dev))
    want = omp.weighted_message_passing(vec.double().numpy(), x.double().numpy(),
                                        w.double().numpy(), src.numpy(), dst.numpy(), n)
    assert normwise_err(out.cpu(), want) <= 1e-5
    assert torch.count_nonzero(out[1::2]).item() == 0
    # no edges at all: zeros; no destinations: empty
    z = bm.sh_tp_scatter_weighted(torch.zeros(0, 3, device=dev), x.to(dev), w.to(dev),
                                  torch.zeros(0, dtype=torch.int64, device=dev),
                                  torch.zeros(n + 1, dtype=torch.int64, device=dev))
    assert z.shape == (n, co, 16) and torch.count_nonzero(z).item() == 0
    z = bm.sh_tp_scatter_weighted(torch.zeros(0, 3, device=dev), x.to(dev), w.to(dev),
                                  torch.zeros(0, dtype=torch.int64, device=dev),
                                  torch.zeros(1, dtype=torch.int64, device=dev))
    assert z.shape == (0, co, 16)


@pytest.mark.parametrize("ci,co", [(32, 64), (20, 70)])
def test_weighted_scatter_step_and_segment_boundaries(bm, dev, ci, co):
    """Destinations whose edge counts sit on both sides of the kernel's boundaries: the
    4-edge k-steps (padded to an even number), the 12-step (48-edge) staging segments,
    and several segments; in a shuffled processing order, against the oracle, and the
    same bits as with the edges stored in CSR order."""
    degs = [0, 1, 2, 3, 4, 5, 7, 8, 9, 47, 48, 49, 52, 95, 96, 97, 100, 143, 144, 145]
    n = len(degs)
    dst = torch.repeat_interleave(torch.arange(n), torch.tensor(degs))
    e = dst.numel()
    perm = torch.randperm(e, generator=gen(80))
    dst = dst[perm]
    src = torch.randint(0, n, (e,), generator=gen(81))
    vec = unit_vectors(e, 82) * (0.5 + torch.rand(e, 1, generator=gen(83)))
    x = torch.randn(n, ci, 16, generator=gen(84))
    w = _weights(ci, co, 85)
    order, rp = _csr(dst, n)
    shuffle = torch.randperm(n, generator=gen(86))
    out = bm.sh_tp_scatter_weighted(vec.to(dev), x.to(dev), w.to(dev), src.to(dev), rp.to(dev),
                                    order.to(dev), shuffle.to(dev), True)
    want = omp.weighted_message_passing(vec.double().numpy(), x.double().numpy(),
                                        w.double().numpy(), src.numpy(), dst.numpy(), n,
                                        normalize=True)
    assert normwise_err(out.cpu(), want) <= 1e-5
    assert torch.count_nonzero(out[0]).item() == 0
    out2 = bm.sh_tp_scatter_weighted(vec[order].to(dev), x.to(dev), w.to(dev), src[order].to(dev),
                                     rp.to(dev), None, None, True)
    assert torch.equal(out, out2)


def test_weighted_scatter_matches_reference_composition_on_gpu(bm, dev):
    """SH -> tensor_product(X[src], Y, W) -> index_add_, the reference's own calls, on this GPU."""
    n, e, c = 300, 5000, 32
    vec = unit_vectors(e, 60).to(dev)
    x = torch.randn(n, c, 16, generator=gen(61)).to(dev)
    w = _weights(c, c, 62).to(dev)
    src = torch.randint(0, n, (e,), generator=gen(63)).to(dev)
    dst = torch.randint(0, n, (e,), generator=gen(64)).to(dev)
    order, rp = _csr(dst.cpu(), n)
    fused = bm.sh_tp_scatter_weighted(vec, x, w, src, rp.to(dev), order.to(dev), None, True)
    msg = bm.tensor_product(x[src], bm.spherical_harmonics(vec, 3), w)
    ref = torch.zeros(n, c, 16, device=dev).index_add_(0, dst, msg)
    assert normwise_err(fused.cpu(), ref.cpu()) <= 1e-5


def test_config3_weighted_full_size(bm, dev):
    """configs[3] weighted variant: N = 5000, C = 64, W [34, 64, 64] ~ N(0, 1/64)."""
    import batmobile
    n, c = 5000, 64
    pos, cell = periodic_box(n, 3)
    graph = batmobile.Graph(pos.to(dev), cell, 5.0, c)
    x = torch.randn(n, c, 16, generator=gen(70)).to(dev)
    w = _weights(c, c, 71).to(dev)
    out = graph.sh_tp_scatter(x, weights=w)
    # identity mixing reduces the weighted product to the simple one
    eye = torch.eye(c).expand(34, c, c).contiguous().to(dev)
    simple = graph.sh_tp_scatter(x)
    assert normwise_err(graph.sh_tp_scatter(x, weights=eye).cpu(), simple.cpu()) <= 1e-5
    # linearity in W
    w2 = _weights(c, c, 72).to(dev)
    both = graph.sh_tp_scatter(x, weights=w + w2)
    sep = out + graph.sh_tp_scatter(x, weights=w2)
    assert normwise_err(both.cpu(), sep.cpu()) <= 1e-5
    # oracle on a sample of destinations (all of their edges)
    rp = graph.row_ptr.cpu()
    pick = torch.randperm(n, generator=gen(73))[:120].sort().values
    ks = torch.cat([torch.arange(int(rp[d]), int(rp[d + 1])) for d in pick.tolist()])
    dloc = torch.repeat_interleave(torch.arange(pick.numel()), rp[pick + 1] - rp[pick])
    want = omp.weighted_message_passing(graph.vec.cpu()[ks].double().numpy(),
                                        x.cpu().double().numpy(), w.cpu().double().numpy(),
                                        graph.src.cpu()[ks].numpy(), dloc.numpy(), pick.numel())
    assert normwise_err(out.cpu()[pick], want) <= 1e-5


def _tile_order_expected(order, deg, n):
    """Each XCD range of 4-destination tiles (P = ceil(tiles / 8) per range, as the weighted
    kernel deals them): destinations sorted by decreasing edge count inside windows of 16
    positions from the range start, then tiles sorted by decreasing edge count, ties by
    position in both; a partial last tile stays last; ranges of more than 2048 tiles are
    left as they are."""
    ntile = (n + 3) // 4
    per = (ntile + 7) // 8
    out = order.copy()
    if per > 2048:
        return out
    for x in range(8):
        t0, t1 = x * per, min(ntile, (x + 1) * per)
        if t0 >= t1:
            continue
        ts = t1 - 1 if (t1 == ntile and n % 4) else t1
        seg = order[4 * t0:4 * ts].copy()
        for wb in range(0, len(seg), 16):
            win = seg[wb:wb + 16]
            seg[wb:wb + 16] = win[sorted(range(len(win)), key=lambda i: (-deg[win[i]], i))]
        w = [int(deg[seg[4 * t:4 * t + 4]].sum()) for t in range(ts - t0)]
        idx = sorted(range(ts - t0), key=lambda k: (-w[k], k))
        for j, k in enumerate(idx):
            out[4 * (t0 + j):4 * (t0 + j) + 4] = seg[4 * k:4 * k + 4]
    return out


@pytest.mark.parametrize("n", [1, 3, 4, 31, 33, 130, 1001, 5000, 16390, 65529, 65541])
def test_weighted_tile_order(bm, dev, n):
    """batteries_weighted_tile_order against a direct statement of the rule, for sizes with
    empty XCD ranges, a partial last tile and ranges of one tile; and the weighted scatter
    is bit-identical in the sorted and the spatial order."""
    g = gen(80 + n)
    deg = torch.randint(0, 60, (n,), generator=g)
    deg[torch.rand(n, generator=g) < 0.1] = 0
    rp = torch.zeros(n + 1, dtype=torch.int64)
    rp[1:] = torch.cumsum(deg, 0)
    order = torch.randperm(n, generator=g)
    got = bm.weighted_tile_order(order.to(dev), rp.to(dev)).cpu().numpy()
    want = _tile_order_expected(order.numpy(), deg.numpy(), n)
    np.testing.assert_array_equal(got, want)
    got_id = bm.weighted_tile_order(None, rp.to(dev)).cpu().numpy()
    np.testing.assert_array_equal(got_id, _tile_order_expected(np.arange(n), deg.numpy(), n))
    if n <= 1001:
        e = int(rp[-1])
        dst = torch.repeat_interleave(torch.arange(n), deg)
        src = torch.randint(0, n, (e,), generator=g)
        vec = unit_vectors(e, 81) * 1.5 if e else torch.zeros(0, 3)
        x = torch.randn(n, 16, 16, generator=g)
        w = _weights(16, 16, 82)
        a = bm.sh_tp_scatter_weighted(vec.to(dev), x.to(dev), w.to(dev), src.to(dev), rp.to(dev),
                                      None, order.to(dev), True)
        b = bm.sh_tp_scatter_weighted(vec.to(dev), x.to(dev), w.to(dev), src.to(dev), rp.to(dev),
                                      None, torch.from_numpy(got).to(dev), True)
        assert torch.equal(a, b)
