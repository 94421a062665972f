"""Channel-half scheduled scatter (batteries_sh_tp_scatter_scheduled_chsplit,
`sh_tp_scatter_scheduled(..., channel_split=True)`): the sums of the scheduled kernel with
each half of the XCDs on one half of the channels and the edges of a workgroup in two
parts, each part's two waves on one 16-channel tile.

Rows that a part boundary cuts are summed in pieces, so they may differ from the scheduled
kernel within rounding.  Every other row is summed in the same order; with unnormalised
vectors it is bit-identical (with normalize=True the two kernels' reciprocal square roots
may round differently).  Shapes the kernel does not take (C not a multiple of 64) run the
scheduled kernel itself."""
import numpy as np
import pytest
import torch

from helpers import gen, normwise_err, unit_vectors
from oracle import mp as omp

pytestmark = pytest.mark.gpu


PARTS = 2  # edge parts of a channel-half workgroup (kHalfParts in mp.hip)


def _cut_rows(rps, rdst, nb, rpb):
    """Destinations whose edge range a workgroup's part boundary crosses: a block's edges
    [e0, e1) are cut at e0 + len * w // PARTS for w = 1 .. PARTS - 1."""
    rps = rps.cpu().numpy()
    rdst = rdst.cpu().numpy()
    cut = set()
    for b in range(nb):
        s0 = b * rpb
        e0, e1 = int(rps[s0]), int(rps[s0 + rpb])
        n = e1 - e0
        cuts = [e0 + n * w // PARTS for w in range(1, PARTS)]
        for i in range(s0, s0 + rpb):
            rs, re = int(rps[i]), int(rps[i + 1])
            if rdst[i] >= 0 and any(rs < c < re for c in cuts):
                cut.add(int(rdst[i]))
    return cut


def _degrees(kind_seed, n, g):
    kind = torch.randint(0, 6, (n,), generator=g)
    deg = torch.where(kind == 0, torch.zeros(n, dtype=torch.int64),
          torch.where(kind == 1, torch.ones(n, dtype=torch.int64),
          torch.where(kind == 2, torch.randint(2, 6, (n,), generator=g),
          torch.where(kind == 3, torch.randint(14, 19, (n,), generator=g),
          torch.where(kind == 4, torch.randint(25, 40, (n,), generator=g),
                      torch.randint(60, 300, (n,), generator=g))))))
    if kind_seed % 3 == 0:
        deg[torch.rand(n, generator=g) < 0.5] = 0
    return deg


def _run(bm, dev, vec, x, src, dst, n, normalize):
    ei = torch.stack([src, dst]).to(dev)
    rp, ci = bm.edge_index_to_csr(ei, n)
    order = torch.arange(n, device=dev)
    c = x.shape[1]
    rps, ep, rdst, nb, rpb = bm.mp_schedule(rp, order, c, ci)
    args = (vec.to(dev), x.to(dev), ei[0].contiguous(), rps, ep, rdst, nb, rpb, n, normalize)
    ref = bm.sh_tp_scatter_scheduled(*args)
    out = bm.sh_tp_scatter_scheduled(*args, channel_split=True)
    return out, ref, _cut_rows(rps, rdst, nb, rpb)


def _check(out, ref, cut, n, deg, normalize):
    keep = torch.ones(n, dtype=torch.bool)
    if cut:
        keep[torch.tensor(sorted(cut))] = False
    keep = keep.to(out.device)
    if not normalize:
        assert torch.equal(out[keep], ref[keep])
    assert normwise_err(out.cpu(), ref.double().cpu().numpy()) <= 1e-5
    assert out[deg.to(out.device) == 0].abs().sum().item() == 0.0


@pytest.mark.parametrize("seed", range(14))
def test_chsplit_random_degree_patterns(bm, dev, seed):
    """Empty rows, one-edge rows, rows shorter and longer than a part of a workgroup's
    edges, long rows cut into pieces, in random order; C = 64, 128 and 192 (the channel-half
    kernel) and 16, 80, 256 (not a multiple of 64, or rows past the index-mode stride: the
    scheduled kernel)."""
    g = torch.Generator().manual_seed(3000 + seed)
    n = int(torch.randint(1, 700, (1,), generator=g))
    c = [64, 128, 192, 64, 16, 80, 256][seed % 7]
    deg = _degrees(seed, n, g)
    dst = torch.repeat_interleave(torch.arange(n), deg)
    e = int(dst.numel())
    src = torch.randint(0, n, (e,), generator=g)
    perm = torch.randperm(e, generator=g)
    src, dst = src[perm], dst[perm]
    vec = unit_vectors(e, 4000 + seed) * (0.5 + torch.rand(e, 1, generator=g)) if e else torch.zeros(0, 3)
    x = torch.randn(n, c, 16, generator=g)
    normalize = seed % 2 == 0
    out, ref, cut = _run(bm, dev, vec, x, src, dst, n, normalize)
    if c % 64 or c * 64 > 16383:
        assert torch.equal(out, ref)  # the scheduled kernel itself
    else:
        _check(out, ref, cut, n, deg, normalize)
    if seed % 4 == 0 and e:
        want = omp.sh_tp_scatter(vec.double().numpy(), x.double().numpy(), src.numpy(), dst.numpy(), n,
                                 normalize=normalize)
        assert normwise_err(out.cpu(), want) <= 1e-5


def test_chsplit_reference_random_graph(bm, dev):
    """The reference benchmark's kind of graph (sources uniform over all atoms, ~30 per
    destination, edges scrambled) at N = 3000, C = 64, against the scheduled kernel and the
    oracle."""
    n, c = 3000, 64
    g = gen(71)
    k = torch.randint(1, 60, (n,), generator=g)
    dst = torch.repeat_interleave(torch.arange(n), k)
    src = torch.randint(0, n, (dst.numel(),), generator=g)
    keep = src != dst
    src, dst = src[keep], dst[keep]
    p = torch.randperm(src.numel(), generator=g)
    src, dst = src[p], dst[p]
    e = src.numel()
    vec = unit_vectors(e, 72)
    x = torch.randn(n, c, 16, generator=gen(73))
    out, ref, cut = _run(bm, dev, vec, x, src, dst, n, False)
    deg = torch.bincount(dst, minlength=n)
    _check(out, ref, cut, n, deg, False)
    assert len(cut) > 0
    want = omp.sh_tp_scatter(vec.double().numpy(), x.double().numpy(), src.numpy(), dst.numpy(), n,
                             normalize=False)
    assert normwise_err(out.cpu(), want) <= 1e-5


@pytest.mark.parametrize("hub", [3, 900, 5000])
def test_chsplit_long_rows_and_tiny_blocks(bm, dev, hub):
    """One destination with more edges than a workgroup's parts (cut into pieces, some parts
    lying inside it), destinations with one edge (workgroups with fewer edges than parts:
    empty parts), isolated destinations."""
    n, c = 1200, 64
    g = gen(81 + hub)
    hub_src = torch.randint(0, n, (hub,), generator=g)
    hub_dst = torch.zeros(hub, dtype=torch.int64)
    one_dst = torch.arange(1, 400)
    one_src = torch.randint(0, n, (399,), generator=g)
    mid_dst = torch.randint(400, 800, (9000,), generator=g)
    mid_src = torch.randint(0, n, (9000,), generator=g)          # 800..1199: no edges
    src = torch.cat([hub_src, one_src, mid_src])
    dst = torch.cat([hub_dst, one_dst, mid_dst])
    e = src.numel()
    vec = unit_vectors(e, 82) * (1.0 + torch.rand(e, 1, generator=g))
    x = torch.randn(n, c, 16, generator=gen(83))
    out, ref, cut = _run(bm, dev, vec, x, src, dst, n, True)
    deg = torch.bincount(dst, minlength=n)
    _check(out, ref, cut, n, deg, True)
    want = omp.sh_tp_scatter(vec.double().numpy(), x.double().numpy(), src.numpy(), dst.numpy(), n,
                             normalize=True)
    assert normwise_err(out.cpu(), want) <= 1e-5
    assert out[800:].abs().max().item() == 0.0


def test_chsplit_deterministic(bm, dev):
    """Two calls give the same bits."""
    n, c = 2000, 128
    g = gen(91)
    dst = torch.repeat_interleave(torch.arange(n), torch.randint(0, 70, (n,), generator=g))
    src = torch.randint(0, n, (dst.numel(),), generator=g)
    vec = unit_vectors(src.numel(), 92)
    x = torch.randn(n, c, 16, generator=gen(93))
    a, _, _ = _run(bm, dev, vec, x, src, dst, n, True)
    b, _, _ = _run(bm, dev, vec, x, src, dst, n, True)
    assert torch.equal(a, b)
