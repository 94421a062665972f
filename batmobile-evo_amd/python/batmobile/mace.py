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

computed by the HIP kernels of the library (radial MLP, MFMA GEMM, channel-wise
CG product + scatter-add, and the gradient with respect to positions).
Gradients are provided for the positions only (forces); the layer's weights
and the node features are treated as constants.
"""
import math

import torch

import _batmobile

N_BASIS = 8
HIDDEN = 64
NUM_PATHS = 34


def edge_weight_bytes(num_edges, channels):
    """Device bytes of the per-edge weights R kept from the forward for the backward:
    mace_edge_weight_rows(E, C) rows of 34 C floats (about 26 GB at configs[4])."""
    return _batmobile.mace_edge_weight_rows(int(num_edges), int(channels)) * NUM_PATHS * int(channels) * 4


def _keep_edge_weights(save, nbytes, device):
    """save: True, False or "auto" (keep R when it takes at most half of the free device
    memory; otherwise the backward recomputes it chunk by chunk, with identical results)."""
    if save == "auto":
        free, _ = torch.cuda.mem_get_info(device)
        return nbytes <= free // 2
    if save not in (True, False):
        raise ValueError("save_edge_weights must be True, False or 'auto'")
    return bool(save)


class MaceLayerFunction(torch.autograd.Function):
    """out = layer(positions); backward returns d<out, grad>/d positions."""

    @staticmethod
    def forward(ctx, positions, node_features, w1, b1, w2, graph, cutoff, save_edge_weights=True):
        graph.exact()  # edge arrays of the edge count (a graph built with max_edges)
        pos = positions.detach().contiguous()
        x = node_features.detach().contiguous()
        # the per-edge weights R (34 C floats per edge) are kept for the backward when
        # positions need a gradient and save_edge_weights allows it (the backward then
        # skips the MLP and its GEMM; otherwise it recomputes R, with identical results)
        ew = None
        if ctx.needs_input_grad[0]:
            e, c = graph.src.numel(), x.shape[1]
            if _keep_edge_weights(save_edge_weights, edge_weight_bytes(e, c), x.device):
                ew = torch.empty(_batmobile.mace_edge_weight_rows(e, c), NUM_PATHS * c,
                                 dtype=torch.float32, device=x.device)
        # destination rows in the graph's Morton order: neighbouring destinations share
        # source rows, which then stay in cache
        out = _batmobile.mace_forward(pos, graph.cell, x, w1, b1, w2, graph.src, graph.dst,
                                      graph.row_ptr, float(cutoff), ew, graph.fine_order())
        ctx.save_for_backward(pos, x, w1, b1, w2)
        ctx.edge_weights = ew
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
                                                ctx.edge_weights, g.fine_order())
        ctx.edge_weights = None
        return grad_pos, None, None, None, None, None, None, None


class MACEInteraction(torch.nn.Module):
    """Interaction layer with per-edge radial weights (weights as buffers).

    W1 [8, 64] ~ N(0, 1/8), b1 = 0, W2 [64, 34 C] ~ N(0, 1/64), column p * C + c
    weighting path p of channel c.

    save_edge_weights: keep the per-edge weights R from the forward for the backward
    (edge_weight_bytes(E, C) of device memory, about 26 GB at configs[4]): True, False
    (the backward recomputes them) or "auto" (keep them when they take at most half of
    the free device memory).
    """

    def __init__(self, channels, cutoff=5.0, device=None, generator=None, save_edge_weights="auto"):
        super().__init__()
        self.channels = int(channels)
        self.cutoff = float(cutoff)
        if save_edge_weights not in (True, False, "auto"):
            raise ValueError("save_edge_weights must be True, False or 'auto'")
        self.save_edge_weights = save_edge_weights
        g = generator
        w1 = torch.randn(N_BASIS, HIDDEN, generator=g) / math.sqrt(N_BASIS)
        w2 = torch.randn(HIDDEN, NUM_PATHS * self.channels, generator=g) / math.sqrt(HIDDEN)
        self.register_buffer("W1", w1.to(device))
        self.register_buffer("b1", torch.zeros(HIDDEN, device=device))
        self.register_buffer("W2", w2.to(device))

    def edge_weight_bytes(self, graph):
        """Device bytes the forward keeps for the backward when it saves R."""
        return edge_weight_bytes(graph.num_edges, self.channels)

    def forward(self, graph, positions, node_features):
        return MaceLayerFunction.apply(positions, node_features, self.W1, self.b1, self.W2,
                                       graph, self.cutoff, self.save_edge_weights)
