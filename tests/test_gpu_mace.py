"""MACE-style layer with per-edge radial weights on the GPU vs the
float64 composition of oracle/mace.py; the fp32 MFMA GEMM vs float64."""
import numpy as np
import pytest
import torch

from oracle import mace as om

from helpers import gen, normwise_err, periodic_box

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("m,n,k,tb", [(100, 70, 64, False), (65, 64, 300, True), (1, 1, 1, False),
                                      (130, 4352, 64, False)])
def test_gemm_f32(bm, dev, m, n, k, tb):
    a = torch.randn(m, k, generator=gen(1))
    b = torch.randn(n, k, generator=gen(2)) if tb else torch.randn(k, n, generator=gen(2))
    c = bm.gemm_f32(a.to(dev), b.to(dev), tb).cpu()
    ref = a.double() @ (b.double().T if tb else b.double())
    assert normwise_err(c, ref.numpy()) <= 1e-6


def _layer_inputs(dev, n, c, seed):
    import batmobile
    pos, cell = periodic_box(n, seed)
    graph = batmobile.Graph(pos.to(dev), cell, 5.0, c)
    layer = batmobile.MACEInteraction(c, 5.0, device=dev, generator=gen(seed + 1))
    x = torch.randn(n, c, 16, generator=gen(seed + 2))
    go = torch.randn(n, c, 16, generator=gen(seed + 3))
    return pos, cell, graph, layer, x, go


def _oracle(pos, cell, graph, layer, x, go):
    box = torch.diagonal(cell).numpy().astype(np.float64)
    return om.layer_and_position_grad(pos.numpy(), box, x.numpy(), graph.src.cpu().numpy(),
                                      graph.dst.cpu().numpy(), layer.W1.cpu().numpy(),
                                      layer.b1.cpu().numpy(), layer.W2.cpu().numpy(), 5.0,
                                      go.numpy())


@pytest.mark.parametrize("n,c", [(80, 16), (300, 5), (80, 64), (60, 128), (40, 256)])
def test_mace_layer_forward_and_forces(bm, dev, n, c):
    pos, cell, graph, layer, x, go = _layer_inputs(dev, n, c, 11)
    p = pos.to(dev).requires_grad_(True)
    out = layer(graph, p, x.to(dev))
    out.backward(go.to(dev))
    ref_out, ref_grad = _oracle(pos, cell, graph, layer, x, go)
    assert normwise_err(out.detach().cpu(), ref_out) <= 1e-5
    assert normwise_err(p.grad.cpu(), ref_grad) <= 1e-4
    # translation invariance: the forces sum to zero
    assert p.grad.sum(0).abs().max().item() <= 1e-5 * p.grad.abs().sum().item()


def test_mace_layer_many_tiles(bm, dev):
    """~285k edges over every position range of the launch, C = 2 (one channel quad,
    half of it past C)."""
    pos, cell, graph, layer, x, go = _layer_inputs(dev, 9500, 2, 21)
    assert graph.num_edges > 262144
    p = pos.to(dev).requires_grad_(True)
    out = layer(graph, p, x.to(dev))
    out.backward(go.to(dev))
    ref_out, ref_grad = _oracle(pos, cell, graph, layer, x, go)
    assert normwise_err(out.detach().cpu(), ref_out) <= 1e-5
    assert normwise_err(p.grad.cpu(), ref_grad) <= 1e-4


def test_mace_layer_dense_cluster_long_rows(bm, dev):
    """125 of 300 atoms on a jittered 0.7 A lattice (a 2.8 A cube): their rows hold 124
    or more edges, so a destination's sum runs over eight or more 16-edge tiles (the
    running sum carried from tile to tile), next to ordinary rows and rows with no edge."""
    import batmobile
    n, c = 300, 12
    L = 30.0
    g = gen(71)
    pos = torch.rand(n, 3, generator=g) * L
    grid = torch.stack(torch.meshgrid(*[torch.arange(5.0)] * 3, indexing="ij"), -1).reshape(-1, 3)
    pos[:125] = torch.tensor([10.0, 12.0, 14.0]) + 0.7 * grid + \
        (torch.rand(125, 3, generator=g) - 0.5) * 0.1
    pos[-1] = torch.tensor([25.0, 25.0, 25.0])
    cell = torch.diag(torch.tensor([L, L, L]))
    graph = batmobile.Graph(pos.to(dev), cell, 5.0, c)
    deg = graph.row_ptr[1:] - graph.row_ptr[:-1]
    assert int(deg.max()) >= 124
    layer = batmobile.MACEInteraction(c, 5.0, device=dev, generator=gen(72))
    x = torch.randn(n, c, 16, generator=gen(73))
    go = torch.randn(n, c, 16, generator=gen(74))
    p = pos.to(dev).requires_grad_(True)
    out = layer(graph, p, x.to(dev))
    out.backward(go.to(dev))
    ref_out, ref_grad = _oracle(pos, cell, graph, layer, x, go)
    assert normwise_err(out.detach().cpu(), ref_out) <= 1e-5
    assert normwise_err(p.grad.cpu(), ref_grad) <= 1e-4
    empty = (deg == 0).cpu()
    assert torch.equal(out.detach().cpu()[empty], torch.zeros(int(empty.sum()), c, 16))


def test_reverse_edges(bm, dev):
    import batmobile
    pos, cell = periodic_box(400, 31)
    graph = batmobile.Graph(pos.to(dev), cell, 5.0, 8)
    rev = graph.reverse_edges().cpu()
    src, dst = graph.src.cpu(), graph.dst.cpu()
    assert torch.equal(rev[rev], torch.arange(rev.numel()))
    assert torch.equal(src[rev], dst) and torch.equal(dst[rev], src)
    # a non-symmetric edge list is refused
    with pytest.raises(RuntimeError, match="not symmetric"):
        bm.mace_reverse_edges(graph.row_ptr, torch.zeros_like(graph.src))


def test_mace_layer_is_deterministic(bm, dev):
    pos, cell, graph, layer, x, go = _layer_inputs(dev, 500, 8, 41)
    outs, grads = [], []
    for _ in range(2):
        p = pos.to(dev).requires_grad_(True)
        o = layer(graph, p, x.to(dev))
        o.backward(go.to(dev))
        outs.append(o.detach().cpu())
        grads.append(p.grad.cpu())
    assert torch.equal(outs[0], outs[1]) and torch.equal(grads[0], grads[1])


def test_mace_row_order_does_not_change_results(bm, dev):
    """Destinations in the graph's spatial order (as MACEInteraction runs them) and in
    index order give bit-identical outputs and forces: every destination is summed in
    ascending edge order, whatever tile its edges fall in.  A malformed order is
    refused."""
    pos, cell, graph, layer, x, go = _layer_inputs(dev, 9500, 6, 61)
    p, xd, god = pos.to(dev), x.to(dev), go.to(dev)
    args = (p, cell, xd, layer.W1, layer.b1, layer.W2, graph.src, graph.dst, graph.row_ptr)
    out_idx = bm.mace_forward(*args, 5.0)
    rev = graph.reverse_edges()
    g_idx = bm.mace_backward(*args, rev, god, 5.0)
    for order in (graph.fine_order(), graph.order):   # as MACEInteraction runs them, and the cell order
        out_sp = bm.mace_forward(*args, 5.0, order)
        assert torch.equal(out_idx, out_sp)
        g_sp = bm.mace_backward(*args, rev, god, 5.0, order)
        assert torch.equal(g_idx, g_sp)
    # a reversed order as well (any permutation)
    assert torch.equal(bm.mace_forward(*args, 5.0, graph.order.flip(0).contiguous()), out_idx)
    with pytest.raises(RuntimeError, match="order"):
        bm.mace_forward(*args, 5.0, graph.order[:-1].contiguous())
    with pytest.raises(RuntimeError, match="order"):
        bm.mace_forward(*args, 5.0, graph.order.to(torch.int32))


def test_config4_full_size(bm, dev):
    """configs[4] as bench.py runs it: N = 50,000, C = 128, ~1.5M edges.  Outputs of 100
    sampled destinations against the float64 oracle restricted to their incoming edges;
    forces on 100 sampled atoms against the oracle over the edges incident to them (no
    other edge depends on their positions); the forces sum to zero; two runs are bitwise
    identical; forward and backward stay under 12 GB of device memory (the per-edge
    weights, 26 GB, are never stored)."""
    import batmobile
    n, c = 50000, 128
    pos, cell = periodic_box(n, 4)
    graph = batmobile.Graph(pos.to(dev), cell, 5.0, c)
    layer = batmobile.MACEInteraction(c, 5.0, device=dev, generator=gen(5))
    x = torch.randn(n, c, 16, generator=gen(6))
    go = torch.randn(n, c, 16, generator=gen(7))
    e = graph.num_edges
    assert e > 1_400_000, e
    torch.cuda.reset_peak_memory_stats(dev)
    outs, grads = [], []
    for _ in range(2):
        p = pos.to(dev).requires_grad_(True)
        o = layer(graph, p, x.to(dev))
        o.backward(go.to(dev))
        outs.append(o.detach().cpu())
        grads.append(p.grad.cpu())
        del o, p
    peak = torch.cuda.max_memory_allocated(dev)
    print(f"configs[4] E={e} peak device memory {peak / 1e9:.2f} GB", flush=True)
    assert peak <= 12e9
    assert torch.equal(outs[0], outs[1]) and torch.equal(grads[0], grads[1])
    out, grad = outs[0], grads[0]
    # the forces sum to zero (translation invariance)
    assert grad.sum(0).abs().max().item() <= 1e-5 * grad.abs().sum().item()

    src, dst = graph.src.cpu(), graph.dst.cpu()
    box = torch.diagonal(cell).numpy().astype(np.float64)
    w1, b1, w2 = (t.cpu().numpy() for t in (layer.W1, layer.b1, layer.W2))
    sample = torch.randperm(n, generator=gen(8))[:100]
    # outputs: the sampled destinations' incoming edges only
    sel = torch.isin(dst, sample)
    ref_out, _ = om.layer_and_position_grad(pos.numpy(), box, x.numpy(), src[sel].numpy(),
                                            dst[sel].numpy(), w1, b1, w2, 5.0,
                                            np.zeros((n, c, 16)))
    assert normwise_err(out[sample], ref_out[sample.numpy()]) <= 1e-5
    # forces: every edge whose source or destination is a sampled atom
    sel = torch.isin(dst, sample) | torch.isin(src, sample)
    _, ref_grad = om.layer_and_position_grad(pos.numpy(), box, x.numpy(), src[sel].numpy(),
                                             dst[sel].numpy(), w1, b1, w2, 5.0, go.numpy())
    assert normwise_err(grad[sample], ref_grad[sample.numpy()]) <= 1e-4
