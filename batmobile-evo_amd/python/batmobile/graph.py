"""A periodic atom graph prepared once for the fused message-passing kernels.

Not a reference API: it bundles what the reference callers do by hand
(benchmarks/benchmark_e2e_mace.py:192-278 neighbor list, :308-356 SH -> TP ->
scatter) into GPU-resident tensors that the fused kernel consumes directly:

  src, dst, vec   edges grouped by destination (dst ascending, src ascending within),
                  vec = minimum-image r_dst - r_src
  row_ptr         CSR row pointer over destinations [N + 1]
  order           spatial order of the atoms (the cell list's cells along a serpentine
                  path, atoms of a cell ascending)
  schedule        processing schedule of the destinations in that order (mp_schedule)

The neighbor relation of a cell list is symmetric, so the neighbor list sorted
by (i, j) read with roles swapped is exactly the edge list sorted by destination,
with vectors negated (exactly, in fp32).

With max_edges the edge arrays hold max_edges entries and the build runs without a
host synchronisation (the edge count stays on the device, in row_ptr[-1]): the step
of a simulation whose positions change every step then queues the graph build and
the fused kernel back to back.  check() raises if the edges outgrew max_edges (the
rows are then left empty, so the kernels that follow read nothing past the arrays).
Such an overflow is silent until check() runs: every kernel queued on the graph then
returns all-zero sums (no messages, no forces).  A loop that builds with max_edges
must call check() (one host synchronisation) before it trusts a result, e.g. once
every few steps with max_edges sized with headroom, and rebuild larger on an error.

Up to 8192 atoms (and 4096 cells) the whole build runs in four kernels
(_batmobile.graph_build); larger systems take the neighbor list's passes and
mp_schedule, with the same results (fast_build=False forces that path).  row_ptr,
order and the schedule, and src, dst and edge_perm, may be views into one
allocation each (or row_ptr into the neighbor list's workspace): saving one
serialises its whole storage; clone() keeps a tensor alone.
"""
import torch

import _batmobile


class Graph:
    def __init__(self, positions, cell, cutoff, channels, self_loops=False, max_edges=None,
                 fast_build=True):
        self.cell = cell
        self.cutoff = float(cutoff)
        self.positions = positions
        self._rev = None
        self._fine_order = None
        self._order_w = None
        self.n_atoms = positions.shape[0]
        self.channels = int(channels)
        cap = -1 if max_edges is None else int(max_edges)
        # up to 8192 atoms: the whole build in four kernels (graph.hip); larger systems,
        # or fast_build=False, the neighbor list passes then mp_schedule (same results)
        res = None
        if fast_build:
            res = _batmobile.graph_build(positions, cell, self.cutoff, bool(self_loops),
                                         self.channels, cap, 0)
        if res is not None:
            (self.src, self.dst, self.vec, self.row_ptr, self.order, self.row_ptr_s,
             self.edge_perm, self.row_dst, self.n_blocks, self.rows_per_block,
             self.overflow) = res
            self._num_edges = int(self.src.numel()) if max_edges is None else None
            return
        # the neighbor list written directly in this layout (one pass, no torch glue),
        # with a spatial order of the atoms from its cells
        if max_edges is None:
            src, dst, vec, off, order = _batmobile.neighbor_graph(positions, cell, self.cutoff,
                                                                  bool(self_loops))
            self.overflow = None
            self._num_edges = int(src.numel())
        else:
            src, dst, vec, off, order, self.overflow = _batmobile.neighbor_graph_capacity(
                positions, cell, self.cutoff, bool(self_loops), cap)
            self._num_edges = None
        self.src = src
        self.dst = dst
        self.vec = vec
        self.row_ptr = off
        self.order = order
        (self.row_ptr_s, self.edge_perm, self.row_dst, self.n_blocks,
         self.rows_per_block) = _batmobile.mp_schedule(self.row_ptr, self.order, self.channels,
                                                       None, int(src.numel()))

    @property
    def num_edges(self):
        """The number of edges (with max_edges: read back from the device, once)."""
        if self._num_edges is None:
            self.check()
            self._num_edges = int(self.row_ptr[-1].item())
        return self._num_edges

    def check(self):
        """Raise if the edges outgrew max_edges (a host synchronisation)."""
        if self.overflow is not None and int(self.overflow.item()) != 0:
            raise RuntimeError("batmobile.Graph: the neighbor list has more edges than "
                               f"max_edges = {int(self.src.numel())}")

    def exact(self):
        """The edge arrays cut to the edge count (after check(); a no-op without
        max_edges).  Consumers that take the edge count from the arrays' length (the
        MACE layer, reverse_edges) call it first."""
        e = self.num_edges
        if self.src.numel() != e:
            self.src, self.dst, self.vec = self.src[:e], self.dst[:e], self.vec[:e]
            self.edge_perm = self.edge_perm[:e]
        return self

    def fine_order(self):
        """Morton order of the atoms on a grid of 1 to 8 atoms per cell (spatial_order; built
        on first use).  The MACE layer walks its destination rows in this order, 1.5% faster
        at configs[4] than in the cell list's order.  It is computed from the values that
        the positions tensor given to the constructor holds at the first call (a caller
        that updates positions in place before then gets the order of the new values);
        results never depend on the order, only the speed does."""
        if self._fine_order is None:
            self._fine_order = _batmobile.spatial_order(self.positions, self.cell)
        return self._fine_order

    def weighted_order(self):
        """The weighted scatter's processing order (built on first use): each XCD's range
        of the spatial order, with the destinations of every 16-position window sorted by
        decreasing edge count and then the 4-destination tiles sorted by decreasing edge
        count, so that a tile's destinations have similar counts, the longest tiles start
        first and the short ones fill the last partial round of workgroups (configs[3]:
        137 -> 132 us).  Results do not depend on it."""
        if self._order_w is None:
            self._order_w = _batmobile.weighted_tile_order(self.order, self.row_ptr)
        return self._order_w

    def reverse_edges(self):
        """rev[e]: index of the edge with source and destination swapped (built once)."""
        if self._rev is None:
            self.exact()
            self._rev = _batmobile.mace_reverse_edges(self.row_ptr, self.src)
        return self._rev

    def sh_tp_scatter(self, node_features, normalize=True, weights=None):
        """out[d] = sum_{e -> d} TP_simple(X[src_e], Y_lm(v_e)); one kernel, spatial schedule.

        With weights [34, C_in, C_out]: out[d] = sum_{e -> d} tensor_product(X[src_e],
        Y_lm(v_e), weights), the per-path sums over each destination's edges mixed once
        per destination (destinations processed in weighted_order()).

        A graph built with max_edges whose edges outgrew it gives all-zero sums here
        without an error: call check() before trusting the result."""
        if weights is not None:
            return _batmobile.sh_tp_scatter_weighted(self.vec, node_features, weights, self.src,
                                                     self.row_ptr, None, self.weighted_order(),
                                                     normalize)
        assert node_features.shape[1] == self.channels, "schedule was built for another C"
        return _batmobile.sh_tp_scatter_scheduled(
            self.vec, node_features, self.src, self.row_ptr_s, self.edge_perm, self.row_dst,
            self.n_blocks, self.rows_per_block, self.n_atoms, normalize)

    def sh_tp_scatter_index_order(self, node_features, normalize=True):
        """The same sum, destinations processed in index order (no schedule)."""
        return _batmobile.sh_tp_scatter(self.vec, node_features, self.src, self.row_ptr, None,
                                        normalize)
