"""MACE-style interaction layer with per-edge radial weights.

Not a reference API.  The reference's interaction block
(benchmarks/benchmark_e2e_mace.py:281-355) composes SH -> tensor product ->
scatter_add with one weight tensor W[34, C, C] shared by all edges and takes
forces by backward through the edge vectors (:412-420, :885-946).  This layer
is the per-edge-weight form of the same pattern:

    v_e   = minimum image of pos[dst_e] - pos[src_e]
    B(r)  = 8 Bessel functions sqrt(2/rc) sin(k pi r/rc)/r times the envelope
            1 - 28 d^6 + 48 d^7 - 21 d^8 (d = r/rc)
    R_e   = silu(B(r_e) W1 + b1) W2      -> [C, 34] weights per edge
    out_d = sum_{e -> d} sum_p R_e[c, p] TP_p(x[src_e, c], Y(v_e / r_e))

computed by the HIP kernels of the library: one fused kernel per pass that forms
each tile of per-edge weights R on MFMA (h W2) and consumes it in the channel-wise
CG product and the scatter-add without storing it (R would take 34 C floats per
edge, 26 GB at configs[4]); the backward runs the transpose GEMM of the MLP on
MFMA in the same tiles and ends in per-edge position gradients.
Gradients are provided for the positions only (forces); the layer's weights
and the node features are treated as constants.
"""
import math

import torch

import _batmobile

N_BASIS = 8
HIDDEN = 64
NUM_PATHS = 34


class MaceLayerFunction(torch.autograd.Function):
    """out = layer(positions); backward returns d<out, grad>/d positions."""

    @staticmethod
    def forward(ctx, positions, node_features, w1, b1, w2, graph, cutoff):
        graph.exact()  # edge arrays of the edge count (a graph built with max_edges)
        pos = positions.detach().contiguous()
        x = node_features.detach().contiguous()
        # destinations in the graph's Morton order: neighbouring destinations share
        # source rows, which then stay in cache (the results do not depend on the order)
        out = _batmobile.mace_forward(pos, graph.cell, x, w1, b1, w2, graph.src, graph.dst,
                                      graph.row_ptr, float(cutoff), graph.fine_order())
        ctx.save_for_backward(pos, x, w1, b1, w2)
        ctx.graph = graph
        ctx.cutoff = float(cutoff)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        pos, x, w1, b1, w2 = ctx.saved_tensors
        if any(ctx.needs_input_grad[1:5]):
            raise NotImplementedError(
                "MaceLayerFunction: only the gradient with respect to positions is provided")
        grad_pos = None
        if ctx.needs_input_grad[0]:
            g = ctx.graph
            grad_pos = _batmobile.mace_backward(pos, g.cell, x, w1, b1, w2, g.src, g.dst,
                                                g.row_ptr, g.reverse_edges(),
                                                grad_out.contiguous(), ctx.cutoff,
                                                g.fine_order())
        return grad_pos, None, None, None, None, None, None


class MACEInteraction(torch.nn.Module):
    """Interaction layer with per-edge radial weights (weights as buffers).

    W1 [8, 64] ~ N(0, 1/8), b1 = 0, W2 [64, 34 C] ~ N(0, 1/64), column p * C + c
    weighting path p of channel c.
    """

    def __init__(self, channels, cutoff=5.0, device=None, generator=None):
        super().__init__()
        self.channels = int(channels)
        self.cutoff = float(cutoff)
        g = generator
        w1 = torch.randn(N_BASIS, HIDDEN, generator=g) / math.sqrt(N_BASIS)
        w2 = torch.randn(HIDDEN, NUM_PATHS * self.channels, generator=g) / math.sqrt(HIDDEN)
        self.register_buffer("W1", w1.to(device))
        self.register_buffer("b1", torch.zeros(HIDDEN, device=device))
        self.register_buffer("W2", w2.to(device))

    def forward(self, graph, positions, node_features):
        return MaceLayerFunction.apply(positions, node_features, self.W1, self.b1, self.W2,
                                       graph, self.cutoff)
