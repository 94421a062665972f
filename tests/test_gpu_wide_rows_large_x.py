"""GPU parity for the gather variants that the narrow, small tests do not reach.

The message-passing kernels pick their source-row gather by shape:
  - rows of C * 64 bytes that fit a buffer descriptor's stride field (C <= 255) are
    gathered in index mode; wider rows (C >= 256) take the per-edge lane-read form;
  - node features of 2 GiB or more are gathered with 64-bit global loads instead of
    buffer loads (the simple kernels and the weighted scatter alike).
Each case here is compared with the float64 oracle within 1e-5 normwise (the simple
and weighted compositions of oracle.mp) on all or on a sample of the destinations.
The reference bounds neither C nor the feature size on these entry points
(python/bindings.cpp:402-489, 555-595).

Also here: the weighted TP backward at C_in > 1023 with C_out > 128 (the VALU path
whose per-row LDS once bounded C_in), against the oracle's exact adjoint.
"""
import numpy as np
import pytest
import torch

from helpers import gen, normwise_err, periodic_box, unit_vectors
from oracle import mp as omp
from oracle import tp as otp

pytestmark = pytest.mark.gpu


def _random_edges(n_src, n_dst, deg, seed, force_last=True):
    """Random edges into n_dst destinations (degrees 0..2*deg), sources uniform over
    n_src rows; the last source row is used by some edges (its offset is the largest)."""
    g = gen(seed)
    degs = torch.randint(0, 2 * deg + 1, (n_dst,), generator=g)
    dst = torch.repeat_interleave(torch.arange(n_dst), degs)
    e = dst.numel()
    src = torch.randint(0, n_src, (e,), generator=g)
    if force_last and e > 8:
        src[::max(1, e // 8)] = n_src - 1
    vec = unit_vectors(e, seed + 1) * (0.5 + torch.rand(e, 1, generator=g) * 4.0)
    rp = torch.zeros(n_dst + 1, dtype=torch.int64)
    rp[1:] = torch.cumsum(degs, 0)
    return vec, src, dst, rp


@pytest.mark.parametrize("c", [256, 320])
def test_wide_rows_scatter_index_order_and_scheduled(bm, dev, c):
    """C >= 256: rows wider than the index-mode stride; index order, a permuted edge
    order and the scheduled kernel, all against the oracle."""
    n = 90
    vec, src, dst, rp = _random_edges(n, n, 20, 500 + c)
    x = torch.randn(n, c, 16, generator=gen(501 + c))
    want = omp.sh_tp_scatter(vec.double().numpy(), x.double().numpy(), src.numpy(), dst.numpy(),
                             n, normalize=True)
    vd, xd, sd, rpd = vec.to(dev), x.to(dev), src.to(dev), rp.to(dev)
    out = bm.sh_tp_scatter(vd, xd, sd, rpd, None, True)
    assert normwise_err(out.cpu(), want) <= 1e-5
    # the same edges stored shuffled and read through perm (perm[k] = CSR slot k's edge)
    shuf = torch.randperm(vec.shape[0], generator=gen(502 + c))
    inv = torch.argsort(shuf)
    outp = bm.sh_tp_scatter(vd[shuf], xd, sd[shuf], rpd, inv.to(dev), True)
    assert torch.equal(out, outp)
    # scheduled: destinations in a shuffled processing order
    order = torch.randperm(n, generator=gen(503 + c)).to(dev)
    rps, ep, rdst, nb, rpb = bm.mp_schedule(rpd, order, c, None, int(vec.shape[0]))
    outs = bm.sh_tp_scatter_scheduled(vd, xd, sd, rps, ep, rdst, nb, rpb, n, True)
    assert torch.equal(out, outs)


@pytest.mark.parametrize("c", [256, 320])
def test_wide_rows_fused_messages_and_csr_passes(bm, dev, c):
    n, e = 70, 900
    vec = unit_vectors(e, 510 + c)
    x = torch.randn(n, c, 16, generator=gen(511 + c))
    src = torch.randint(0, n, (e,), generator=gen(512 + c))
    tgt = torch.randint(0, n, (e,), generator=gen(513 + c))
    msg = bm.fused_sh_tp_simple(vec.to(dev), x.to(dev), src.to(dev))
    want = omp.fused_sh_tp_simple(vec.double().numpy(), x.double().numpy(), src.numpy())
    assert normwise_err(msg.cpu(), want) <= 1e-5
    ei = torch.stack([src, tgt])
    rp, col = bm.edge_index_to_csr(ei.to(dev), n)
    out = bm.fused_message_passing_simple(x.to(dev), vec.to(dev), ei.to(dev), rp, col)
    want2 = omp.fused_message_passing_simple(x.double().numpy(), vec.double().numpy(), ei.numpy(),
                                             rp.cpu().numpy(), col.cpu().numpy())
    assert normwise_err(out.cpu(), want2) <= 1e-5


@pytest.mark.parametrize("ci,co", [(256, 64), (320, 80)])
def test_wide_rows_weighted_scatter(bm, dev, ci, co):
    n = 40
    vec, src, dst, rp = _random_edges(n, n, 16, 520 + ci)
    x = torch.randn(n, ci, 16, generator=gen(521 + ci))
    w = torch.randn(34, ci, co, generator=gen(522 + ci)) / np.sqrt(ci)
    out = bm.sh_tp_scatter_weighted(vec.to(dev), x.to(dev), w.to(dev), src.to(dev), rp.to(dev),
                                    None, None, True)
    want = omp.weighted_message_passing(vec.double().numpy(), x.double().numpy(),
                                        w.double().numpy(), src.numpy(), dst.numpy(), n)
    assert normwise_err(out.cpu(), want) <= 1e-5


# ---------------------------------------------------------------------------
# node features of 2 GiB and more: 64-bit gathers
# ---------------------------------------------------------------------------
N_BIG = 140_000   # x [140000, 256, 16] fp32 = 2.29 GB > 2 GiB
C_BIG = 256


@pytest.fixture(scope="module")
def big_x(dev):
    g = torch.Generator(device=dev).manual_seed(530)
    x = torch.randn(N_BIG, C_BIG, 16, device=dev, generator=g)
    assert x.numel() * 4 > 2 ** 31
    yield x
    del x
    torch.cuda.empty_cache()


def _sampled_check(out, x, vec, src, rp, sample, weights=None):
    """Oracle on the sampled destinations' edges, the source rows they use copied back."""
    rpc = rp.cpu()
    es = torch.cat([torch.arange(int(rpc[d]), int(rpc[d + 1])) for d in sample])
    ds = torch.cat([torch.full((int(rpc[d + 1] - rpc[d]),), i) for i, d in enumerate(sample)])
    used, local = torch.unique(src[es], return_inverse=True)
    xs = x[used.to(x.device)].cpu().double().numpy()
    v = vec[es].double().numpy()
    if weights is None:
        want = omp.sh_tp_scatter(v, xs, local.numpy(), ds.numpy(), len(sample), normalize=True)
    else:
        want = omp.weighted_message_passing(v, xs, weights.double().numpy(), local.numpy(),
                                            ds.numpy(), len(sample))
    got = out[torch.tensor(sample, device=out.device)].cpu().numpy()
    return normwise_err(got, want)


def test_large_x_scatter_index_order_and_scheduled(bm, dev, big_x):
    n_dst = 3000
    vec, src, dst, rp = _random_edges(N_BIG, n_dst, 12, 531)
    vd, sd, rpd = vec.to(dev), src.to(dev), rp.to(dev)
    out = bm.sh_tp_scatter(vd, big_x, sd, rpd, None, True)
    # sampled destinations, including the ones whose edges use the last source row
    rows_last = torch.unique(dst[src == N_BIG - 1])[:6].tolist()
    sample = sorted(set([0, 1, n_dst - 1] + list(range(17, n_dst, 211)) + rows_last))
    assert _sampled_check(out, big_x, vec, src, rp, sample) <= 1e-5
    order = torch.randperm(n_dst, generator=gen(532)).to(dev)
    rps, ep, rdst, nb, rpb = bm.mp_schedule(rpd, order, C_BIG, None, int(vec.shape[0]))
    outs = bm.sh_tp_scatter_scheduled(vd, big_x, sd, rps, ep, rdst, nb, rpb, n_dst, True)
    assert torch.equal(out, outs)


def test_large_x_fused_messages(bm, dev, big_x):
    e = 2500
    src = torch.randint(0, N_BIG, (e,), generator=gen(533))
    src[::97] = N_BIG - 1
    vec = unit_vectors(e, 534)
    msg = bm.fused_sh_tp_simple(vec.to(dev), big_x, src.to(dev))
    used, local = torch.unique(src, return_inverse=True)
    want = omp.fused_sh_tp_simple(vec.double().numpy(), big_x[used.to(dev)].cpu().double().numpy(),
                                  local.numpy())
    assert normwise_err(msg.cpu(), want) <= 1e-5


def test_large_x_weighted_scatter(bm, dev, big_x):
    n_dst, co = 1500, 64
    vec, src, dst, rp = _random_edges(N_BIG, n_dst, 12, 535)
    w = torch.randn(34, C_BIG, co, generator=gen(536)) / np.sqrt(C_BIG)
    out = bm.sh_tp_scatter_weighted(vec.to(dev), big_x, w.to(dev), src.to(dev), rp.to(dev),
                                    None, None, True)
    rows_last = torch.unique(dst[src == N_BIG - 1])[:4].tolist()
    sample = sorted(set([0, n_dst - 1] + list(range(5, n_dst, 173)) + rows_last))
    assert _sampled_check(out, big_x, vec, src, rp, sample, weights=w) <= 1e-5


# ---------------------------------------------------------------------------
# weighted TP backward with C_in > 1023 and C_out > 128
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("n,ci,co", [(3, 1100, 160), (2, 2050, 129)])
def test_tp_backward_wide_input_channels(bm, dev, n, ci, co):
    x = torch.randn(n, ci, 16, generator=gen(540 + ci))
    y = torch.randn(n, 16, generator=gen(541))
    w = torch.randn(34, ci, co, generator=gen(542)) / np.sqrt(ci)
    go = torch.randn(n, co, 16, generator=gen(543))
    gx, gy, gw = bm.tensor_product_backward(x.to(dev), y.to(dev), w.to(dev), go.to(dev))
    wx, wy, ww = otp.tensor_product_backward(x.double().numpy(), y.double().numpy(),
                                             w.double().numpy(), go.double().numpy())
    assert normwise_err(gx.cpu(), wx) <= 1e-4
    assert normwise_err(gy.cpu(), wy) <= 1e-4
    assert normwise_err(gw.cpu(), ww) <= 1e-4
    # each gradient alone gives the same values
    gx1, gy1, gw1 = bm.tensor_product_backward(x.to(dev), y.to(dev), w.to(dev), go.to(dev),
                                               True, False, False)
    assert gy1 is None and gw1 is None and torch.equal(gx1, gx)
