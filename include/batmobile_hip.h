/*
 * batmobile_hip.h -- C ABI of libbatmobile_hip.so, the MI355X (gfx950) HIP
 * implementation of batmobile's equivariant message-passing path.
 *
 * Conventions
 *   - Every pointer argument is a device pointer unless marked "host".
 *   - Tensors are dense, row-major, fp32 (int64 for indices) as described.
 *   - Work is enqueued on `stream` and is asynchronous unless stated.
 *   - Return value: 0 on success, a hipError_t value (> 0) on a launch/runtime
 *     error, BATMOBILE_HIP_ERR_ARG (-1) for invalid arguments, BATMOBILE_HIP_ERR_WORKSPACE (-2) for a
 *     missing or too small workspace, BATMOBILE_HIP_ERR_SCRATCH (-4) for a call
 *     too large for the static scratch of the no-allocation entry point.
 *   - No function allocates device memory except the reference-compatible
 *     neighbor_list_cuda(); where scratch is needed the caller passes a
 *     workspace whose size is given by the matching *_workspace_bytes(), except
 *     batteries_tensor_product_backward_l3_noalloc(), whose scratch is a static
 *     device array.  No vendor library is called.
 *
 * Each entry point names the reference function it replaces
 * (paths relative to the reference repository).
 */
#ifndef BATMOBILE_HIP_H_
#define BATMOBILE_HIP_H_

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>
#ifndef __cplusplus
#include <stdbool.h>
#endif

#ifdef __cplusplus
extern "C" {
#endif

#define BATMOBILE_HIP_OK 0
#define BATMOBILE_HIP_ERR_ARG -1
#define BATMOBILE_HIP_ERR_WORKSPACE -2
#define BATMOBILE_HIP_ERR_SCRATCH -4 /* the call needs more than the static scratch holds */

/* Size of the static device scratch of batteries_tensor_product_backward_l3_noalloc
 * (24 MiB per GPU, held from the library's load until the process ends). */
#define BATMOBILE_HIP_NOALLOC_SCRATCH_BYTES (24u << 20)

/* ---------------------------------------------------------------------------
 * Spherical harmonics, L_max in [0, 6]
 * ------------------------------------------------------------------------- */

/* Y_lm[N, (L_max+1)^2] of edge_vectors[N, 3].  normalize = 0 evaluates the
 * polynomials on the vectors as given (reference behaviour); normalize = 1
 * first divides each vector by max(|v|, 1e-10).
 * Replaces batteries::spherical_harmonics_dispatch,
 * src/spherical_harmonics/spherical_harmonics.cu:296-314 (bound at
 * python/bindings.cpp:43-78 and, for the pre-allocated output, :83-114). */
int batteries_spherical_harmonics(const float* edge_vectors, float* Y_lm, int64_t N, int L_max,
                                  int normalize, hipStream_t stream);

/* grad_xyz[N, 3] = sum_lm grad_Y_lm[N, lm] * dY_lm/d(x,y,z).  With normalize = 1
 * the input is the raw vector and the result is chained through v/|v|
 * (python/batmobile/autograd.py:62-92).
 * Replaces batteries::spherical_harmonics_backward_dispatch,
 * src/spherical_harmonics/spherical_harmonics_backward.cu:440-463 (bound at
 * python/bindings.cpp:236-280); also covers L_max 4..6, which the reference
 * kernel rejects. */
int batteries_spherical_harmonics_backward(const float* edge_vectors, const float* grad_Y_lm,
                                           float* grad_xyz, int64_t N, int L_max, int normalize,
                                           hipStream_t stream);

/* ---------------------------------------------------------------------------
 * 34-path L<=3 Clebsch-Gordan tensor products
 * ------------------------------------------------------------------------- */

/* 34.  Replaces batteries::get_num_paths_l3, src/tensor_product/tensor_product.cu:203-205. */
int batteries_get_num_paths_l3(void);

/* path_info (host) [34, 3] = (l1, l2, l_out).  Replaces batteries::get_path_info_l3,
 * src/tensor_product/tensor_product.cu:207-214. */
void batteries_get_path_info_l3(int* path_info);

/* output[N,16] = sum c * input1[N,16]_a * input2[N,16]_b (all three 16-byte aligned).
 * Replaces batteries::tensor_product_simple_l3, src/tensor_product/tensor_product.cu:159-176. */
int batteries_tensor_product_simple_l3(const float* input1, const float* input2, float* output,
                                       int64_t N, hipStream_t stream);

/* (grad_input1, grad_input2)[N,16] (all five arrays 16-byte aligned).  Replaces
 * batteries::tensor_product_simple_backward_l3, src/tensor_product/tensor_product_backward.cu:1007-1026. */
int batteries_tensor_product_simple_backward_l3(const float* input1, const float* input2,
                                                const float* grad_output, float* grad_input1,
                                                float* grad_input2, int64_t N, hipStream_t stream);

/* output[N, C_out, 16] = sum_p sum_ci weights[p, ci, co] * TP_p(input1[N, C_in, 16], input2[N, 16]).
 * Replaces batteries::tensor_product_l3, src/tensor_product/tensor_product.cu:178-201. */
int batteries_tensor_product_l3(const float* input1, const float* input2, const float* weights,
                                float* output, int64_t N, int C_in, int C_out, hipStream_t stream);

/* Workspace for batteries_tensor_product_backward_l3 with grad_weights != NULL. */
size_t batteries_tensor_product_backward_workspace_bytes(int64_t N, int C_in, int C_out);

/* Exact adjoint of batteries_tensor_product_l3.  Any of grad_input1 [N,C_in,16],
 * grad_input2 [N,16], grad_weights [34,C_in,C_out] may be NULL (not computed).
 * grad_weights is a deterministic reduction over rows; N = 0 gives zeros.
 * input1 and grad_output 16-byte aligned.  Replaces batteries::tensor_product_backward_l3,
 * src/tensor_product/tensor_product_backward.cu:948-1005 (bound at
 * python/bindings.cpp:325-393). */
int batteries_tensor_product_backward_l3(const float* input1, const float* input2,
                                         const float* weights, const float* grad_output,
                                         float* grad_input1, float* grad_input2,
                                         float* grad_weights, int64_t N, int C_in, int C_out,
                                         void* workspace, size_t workspace_bytes,
                                         hipStream_t stream);

/* The backward above without any allocation, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  No counterpart in the reference.  Same arguments and results
 * as batteries_tensor_product_backward_l3 minus the workspace: the grad_W partials
 * live in a static device array of BATMOBILE_HIP_NOALLOC_SCRATCH_BYTES per GPU.
 * Returns BATMOBILE_HIP_ERR_SCRATCH (and touches nothing) when grad_weights is
 * requested and batteries_tensor_product_backward_workspace_bytes(N, C_in, C_out)
 * exceeds it.  The partials fit for every N when 3 ceil(C_in/16) ceil(C_out/64)
 * <= 512 (e.g. C_in = C_out = 256).  The first call on a device
 * resolves the array's device address (hipGetSymbolAddress, no allocation by this
 * library); make it outside graph capture.  All calls on one GPU share the array,
 * so calls that overlap on one GPU (concurrent streams, threads) race. */
int batteries_tensor_product_backward_l3_noalloc(const float* input1, const float* input2,
                                                 const float* weights, const float* grad_output,
                                                 float* grad_input1, float* grad_input2,
                                                 float* grad_weights, int64_t N, int C_in,
                                                 int C_out, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Fused SH + TP, scatter-add, CSR
 * ------------------------------------------------------------------------- */

/* messages[E, C, 16] = TP_simple(node_features[source_idx[e], C, 16], Y(edge_vectors[e])),
 * node_features [N_nodes, C, 16].
 * normalize as in batteries_spherical_harmonics (0 = reference behaviour).
 * node_features and messages must be 16-byte aligned.
 * Replaces batteries::fused_sh_tp_simple, src/message_passing/fused_sh_tp.cu:125-146. */
int batteries_fused_sh_tp_simple(const float* edge_vectors, const float* node_features,
                                 const int64_t* source_idx, float* messages, int64_t N_nodes,
                                 int64_t N_edges, int C, int normalize, hipStream_t stream);

/* Fused SH + TP + scatter-add into destinations (node_features [N_src, C, 16],
 * node_output [N_dst, C, 16]), one pass, no atomics,
 * deterministic:
 *   node_output[d, C, 16] = sum_{k in [row_ptr[d], row_ptr[d+1])}
 *        TP_simple(node_features[source_idx[e_k]], Y(edge_vectors[e_k])),
 *   e_k = perm ? perm[k] : k.
 * Destinations with no edges get zeros.  No counterpart as a single call in the
 * reference: it is the composition fused_sh_tp_simple -> index_add_
 * (benchmarks/benchmark_fused_sh_tp.py:96-98,105-107) and the engine of
 * batteries::fused_message_passing_simple below. */
int batteries_sh_tp_scatter_csr(const float* edge_vectors, const float* node_features,
                                const int64_t* source_idx, const int64_t* perm,
                                const int64_t* row_ptr, float* node_output, int64_t N_src,
                                int64_t N_dst, int64_t N_edges, int C, int normalize,
                                hipStream_t stream);

/* Spatial processing schedule for the fused scatter (no reference counterpart:
 * the reference processes destinations in index order).  Built once per graph:
 *   batteries_spatial_order      order[N] = atoms sorted by the Morton code of
 *                                their cell in a 2^b-per-axis grid over the box (host
 *                                box[3]; b <= 5 the largest with 8^b <= N)
 *   batteries_mp_schedule_shape  n_blocks (multiple of 8) x rows_per_block for C
 *   batteries_mp_schedule        row_ptr_s[n_blocks*rows_per_block + 1],
 *                                row_dst[n_blocks*rows_per_block] (-1 = empty slot),
 *                                edge_perm[E] (scheduled slot -> original edge; col_perm,
 *                                if given, is applied as in fused_message_passing_simple);
 *                                rows are dealt so that workgroups hold nearly equal
 *                                numbers of edges
 * and consumed by batteries_sh_tp_scatter_scheduled, whose result equals
 * batteries_sh_tp_scatter_csr on the same graph. */
size_t batteries_spatial_order_workspace_bytes(int64_t N);
int batteries_spatial_order(const float* positions, const float* box, int64_t N, void* workspace,
                            size_t workspace_bytes, int64_t* order, hipStream_t stream);
int batteries_mp_schedule_shape(int64_t N_dst, int C, int* n_blocks, int* rows_per_block);
size_t batteries_mp_schedule_workspace_bytes(int n_blocks, int rows_per_block);
int batteries_mp_schedule(const int64_t* row_ptr, const int64_t* col_perm, const int64_t* order,
                          int64_t N_dst, int64_t N_edges, int C, int n_blocks, int rows_per_block,
                          int64_t* row_ptr_s, int64_t* row_dst, int64_t* edge_perm,
                          void* workspace, size_t workspace_bytes, hipStream_t stream);
int batteries_sh_tp_scatter_scheduled(const float* edge_vectors, const float* node_features,
                                      const int64_t* source_idx, const int64_t* row_ptr_s,
                                      const int64_t* edge_perm, const int64_t* row_dst,
                                      int n_blocks, int rows_per_block, float* node_output,
                                      int64_t N_src, int64_t N_edges, int C, int normalize,
                                      hipStream_t stream);
/* Extension with no counterpart in the reference: the same sums over the same schedule for
 * graphs whose sources have no spatial order (sources spread over all atoms, as in the
 * reference's benchmark graph), where one XCD's L2 cannot hold the rows it gathers.  XCDs
 * 0-3 then take channels 0-31 of each 64-channel group and XCDs 4-7 channels 32-63, and the
 * four waves of a workgroup take quarters of its edges.  Rows that the quarter boundaries
 * cut are summed in pieces (in a fixed order), so those rows can differ from
 * batteries_sh_tp_scatter_scheduled in the last bits; every other row is identical.
 * C must be a multiple of 64 with C * 64 <= 16383 bytes per row, X under 2 GiB and
 * edge_perm given; other inputs run batteries_sh_tp_scatter_scheduled's kernel. */
int batteries_sh_tp_scatter_scheduled_chsplit(const float* edge_vectors,
                                              const float* node_features,
                                              const int64_t* source_idx, const int64_t* row_ptr_s,
                                              const int64_t* edge_perm, const int64_t* row_dst,
                                              int n_blocks, int rows_per_block, float* node_output,
                                              int64_t N_src, int64_t N_edges, int C, int normalize,
                                              hipStream_t stream);

/* Weighted scatter: node_output[N_dst, C_out, 16] with
 *   node_output[d] = sum_{k in [row_ptr[d], row_ptr[d+1])}
 *                    tensor_product(X[source_idx[e_k]], Y(v_{e_k}), weights),  e_k = perm ? perm[k] : k,
 * weights [34, C_in, C_out] shared by every edge, Y of v / |v| when normalize.
 * Replaces the reference interaction block's SH -> batteries::tensor_product ->
 * scatter_add (benchmarks/benchmark_e2e_mace.py:308-349; examples/mace_inference.py:
 * 152-168), without the [E, C_out, 16] messages.  order (optional, [N_dst]) is the
 * order in which destinations are processed: a permutation of 0..N_dst-1 (a spatial
 * order keeps source rows in L2); entries outside [0, N_dst) are skipped, leaving rows
 * that no entry names unwritten.  One fused kernel, no workspace (the workspace size is 0;
 * the arguments are kept for callers written against a version that had one). */
size_t batteries_sh_tp_scatter_weighted_workspace_bytes(int64_t N_dst, int64_t N_edges, int C_in,
                                                        int C_out);
int batteries_sh_tp_scatter_weighted(const float* edge_vectors, const float* node_features,
                                     const float* weights, const int64_t* source_idx,
                                     const int64_t* perm, const int64_t* row_ptr,
                                     const int64_t* order, float* node_output, int64_t N_src,
                                     int64_t N_dst, int64_t N_edges, int C_in, int C_out,
                                     int normalize, void* workspace, size_t workspace_bytes,
                                     hipStream_t stream);

/* Extension with no counterpart in the reference (like the spatial order): a processing
 * order for batteries_sh_tp_scatter_weighted that keeps each XCD's range of 4-destination
 * tiles (as the kernel deals them).  Inside a range, the destinations of each window of 16
 * consecutive positions are sorted by decreasing edge count, then the tiles by decreasing
 * edge count (ties by position in both), so that a tile's destinations have similar counts
 * and the longest tiles start first; a partial last tile keeps its place.  order
 * (nullable: 0..N_dst-1) is the order to rearrange, row_ptr the CSR rows [N_dst + 1];
 * order_out [N_dst].  Ranges of more than 2048 tiles are copied unchanged.  The results of
 * the weighted scatter do not depend on the order. */
int batteries_weighted_tile_order(const int64_t* order, const int64_t* row_ptr, int64_t N_dst,
                                  int64_t* order_out, hipStream_t stream);

/* node_output[N_atoms, C, 16]; CSR slot k is edge col_idx[k], whose source is
 * edge_index[0, col_idx[k]] and vector edge_vectors[col_idx[k]].
 * Replaces batteries::fused_message_passing_simple,
 * src/message_passing/fused_message_passing.cu:257-280. */
int batteries_fused_message_passing_simple(const float* node_features, const float* edge_vectors,
                                           const int64_t* edge_index, const int64_t* row_ptr,
                                           const int64_t* col_idx, float* node_output,
                                           int64_t N_atoms, int64_t N_edges, int C,
                                           hipStream_t stream);

/* Workspace for batteries_fused_message_passing. */
size_t batteries_fused_message_passing_workspace_bytes(int64_t N_atoms, int C_in);

/* node_output[N_atoms, C_out, 16] = sum_ci weights[ci, co] * S[t, ci, :] where S is
 * the simple fused pass with source atom col_idx[k] and vector edge_vectors[k] for
 * CSR slot k (the reference kernel's indexing, fused_message_passing.cu:332-337).
 * Replaces batteries::fused_message_passing,
 * src/message_passing/fused_message_passing.cu:376-400. */
int batteries_fused_message_passing(const float* node_features, const float* edge_vectors,
                                    const float* weights, const int64_t* row_ptr,
                                    const int64_t* col_idx, float* node_output, int64_t N_atoms,
                                    int64_t N_edges, int C_in, int C_out, void* workspace,
                                    size_t workspace_bytes, hipStream_t stream);

/* Workspace for batteries_edge_index_to_csr. */
size_t batteries_edge_index_to_csr_workspace_bytes(int64_t N_atoms);

/* row_ptr[N_atoms+1] and col_idx[E] (original edge ids grouped by target
 * edge_index[1, e], ascending inside each row).  Replaces
 * batteries::edge_index_to_csr, src/message_passing/fused_message_passing.cu:108-165. */
int batteries_edge_index_to_csr(const int64_t* edge_index, int64_t* row_ptr, int64_t* col_idx,
                                int64_t N_atoms, int64_t N_edges, void* workspace,
                                size_t workspace_bytes, hipStream_t stream);

/* out[0..n] = exclusive prefix sum of in[0..n-1], out[n] = total (one
 * workgroup, fixed order).  Replaces the cub::DeviceScan::ExclusiveSum calls of
 * src/neighbor_list/neighbor_list.cu:332-336,356-360 and
 * src/message_passing/fused_message_passing.cu:140-151. */
int batteries_exclusive_scan_i64(const int64_t* in, int64_t* out, int64_t n, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Cell-list neighbor list (orthorhombic PBC)
 * ------------------------------------------------------------------------- */

/* Workspace for the two-phase build; box (host) = cell diagonal. 0 if invalid. */
size_t batteries_neighbor_list_workspace_bytes(int64_t N, const float* box, float cutoff);

/* Byte offset, inside that workspace, of the row offsets (int64 [N+1]) that phase 1
 * leaves there: a caller may read them in place (until the workspace is reused)
 * instead of a copy through row_offsets.  0 if invalid (a valid offset is never 0).
 * No counterpart in the reference, whose offsets stay internal to
 * batteries::neighbor_list_cuda. */
size_t batteries_neighbor_list_offsets_at(int64_t N, const float* box, float cutoff);

/* Phase 1: bins, per-atom counts, offsets; writes E to *d_num_edges (device,
 * may be NULL).  Steps :261-366 of batteries::neighbor_list_cuda,
 * src/neighbor_list/neighbor_list.cu. */
int batteries_neighbor_list_count(const float* positions, const float* box, int64_t N,
                                  float cutoff, int self_loops, void* workspace,
                                  size_t workspace_bytes, int64_t* d_num_edges, hipStream_t stream);

/* Phase 2 (same workspace, after phase 1): edge_src[E] = i, edge_dst[E] = j,
 * edge_vectors[E,3] = minimum-image pos[j] - pos[i], sorted by (i, j);
 * row_offsets[N+1] (may be NULL) = start of each i.  Steps :367-402 of
 * batteries::neighbor_list_cuda. */
int batteries_neighbor_list_write(const float* positions, const float* box, int64_t N,
                                  float cutoff, int self_loops, void* workspace,
                                  size_t workspace_bytes, int* edge_src, int* edge_dst,
                                  float* edge_vectors, int64_t* row_offsets, hipStream_t stream);

/* Phase 2 in the layout of the message-passing kernels (same workspace, after
 * phase 1): the neighbor list read with roles swapped, src[E] = j, dst[E] = i
 * (int64, sorted by (i, j): grouped by destination), edge_vectors[E,3] =
 * minimum-image pos[i] - pos[j] (the phase-2 vector negated exactly);
 * row_offsets[N+1] (may be NULL) = start of each destination; spatial_order[N]
 * (may be NULL) = the atoms by cell of the cell list, cells along a serpentine
 * path (consecutive cells adjacent), atoms of a cell in ascending index (a
 * processing order for batteries_mp_schedule).  tmp_j [E] and tmp_vec [E,3] are
 * scratch.  No counterpart in the reference, whose message
 * passing callers convert edge_index and negate the vectors with torch
 * (benchmarks/benchmark_e2e_mace.py:192-278); the neighbor set and vectors are
 * those of batteries::neighbor_list_cuda. */
int batteries_neighbor_graph_write(const float* positions, const float* box, int64_t N,
                                   float cutoff, int self_loops, void* workspace,
                                   size_t workspace_bytes, int* tmp_j, float* tmp_vec,
                                   int64_t* src, int64_t* dst, float* edge_vectors,
                                   int64_t* row_offsets, int64_t* spatial_order,
                                   hipStream_t stream);

/* batteries_neighbor_graph_write without knowing E on the host: the arrays hold
 * `capacity` edges (tmp_j, tmp_vec, src, dst, edge_vectors), E stays on the device
 * (row_offsets[N], or the workspace's offsets), and *overflow (device int) is set to
 * 1 when E > capacity, in which case every row is left empty (row offsets all 0, so
 * that no later kernel reads past the arrays), else to 0.  spatial_order as there.
 * Lets a caller build the graph and launch its kernels with no host
 * synchronisation.  No counterpart in the reference, whose neighbor list
 * synchronises twice (neighbor_list.cu:262,363-366). */
int batteries_neighbor_graph_write_capacity(const float* positions, const float* box, int64_t N,
                                            float cutoff, int self_loops, void* workspace,
                                            size_t workspace_bytes, int64_t capacity, int* tmp_j,
                                            float* tmp_vec, int64_t* src, int64_t* dst,
                                            float* edge_vectors, int64_t* row_offsets,
                                            int64_t* spatial_order, int* overflow,
                                            hipStream_t stream);

/* Graph build in four kernels, for systems of up to 8192 atoms and 4096 cells with
 * atoms x cells <= 2^23 and at most 256 schedule groups for C channels
 * (workspace_bytes returns 0 otherwise: use the neighbor graph calls above and
 * batteries_mp_schedule).  Results bit-identical to those calls
 * (graph layout, spatial order, schedule of batteries_mp_schedule_shape(N, C)).
 *
 * Count (three kernels): binning, one workgroup per cell writing each atom's row
 * sorted by j into a workspace slab of row_capacity entries per atom (0: chosen
 * from the density; longer rows are found again by the write), then one workgroup
 * for the row offsets and the schedule: row_offsets [N+1] (row_offsets[N] = E),
 * order [N] (spatial order), row_ptr_s [n_blocks*rows_per_block + 1] and row_dst
 * [n_blocks*rows_per_block].  capacity >= 0: the edge arrays hold `capacity` edges;
 * when E > capacity *overflow (device int, may be NULL with capacity < 0) is set
 * to 1 and every row is left empty (as batteries_neighbor_graph_write_capacity).
 * Write (one kernel, same workspace, after count, no host synchronisation needed):
 * src, dst [E] int64, edge_vectors [E, 3] (the layout of
 * batteries_neighbor_graph_write) and edge_perm [E] (of batteries_mp_schedule with
 * col_perm NULL).  No counterpart in the reference, whose e2e pipeline rebuilds
 * its neighbor list and converts it with torch per step
 * (benchmarks/benchmark_e2e_mace.py:192-278); the neighbor set is that of
 * batteries::neighbor_list_cuda (src/neighbor_list/neighbor_list.cu:242-430). */
size_t batteries_graph_build_workspace_bytes(int64_t N, const float* box, float cutoff, int C,
                                             int row_capacity);
int batteries_graph_build_count(const float* positions, const float* box, int64_t N,
                                float cutoff, int self_loops, int C, int n_blocks,
                                int rows_per_block, int64_t capacity, int row_capacity,
                                void* workspace, size_t workspace_bytes, int64_t* row_offsets,
                                int64_t* order, int64_t* row_ptr_s, int64_t* row_dst,
                                int* overflow, hipStream_t stream);
int batteries_graph_build_write(const float* positions, const float* box, int64_t N,
                                float cutoff, int self_loops, int row_capacity, void* workspace,
                                size_t workspace_bytes, const int64_t* row_offsets,
                                const int* overflow, int64_t* src, int64_t* dst,
                                float* edge_vectors, int64_t* edge_perm, hipStream_t stream);

/* Phase 2 with int64 indices in the neighbor list's own orientation (same
 * workspace, after phase 1; num_edges = E from phase 1): edge_index [2, E] (row 0 =
 * i, row 1 = j, sorted by (i, j)), edge_vectors [E, 3] = minimum-image pos[j] -
 * pos[i], row_offsets [N+1] (may be NULL); tmp_j [E] and tmp_vec [E,3] are
 * scratch.  The layout torch callers index with (int64); the reference's C ABI
 * writes int32 (batteries_neighbor_list_write).  No counterpart in the reference. */
int batteries_neighbor_list_write_i64(const float* positions, const float* box, int64_t N,
                                      float cutoff, int self_loops, void* workspace,
                                      size_t workspace_bytes, int64_t num_edges, int* tmp_j,
                                      float* tmp_vec, int64_t* edge_index, float* edge_vectors,
                                      int64_t* row_offsets, hipStream_t stream);

/* The neighbor list in three kernels and a scan, for systems of up to 8192 atoms and
 * 4096 cells with atoms x cells <= 2^23 (workspace_bytes returns 0 otherwise: use the
 * count / write calls above): binning, one workgroup per cell writing each atom's
 * neighbors already sorted by j into a workspace slab of row_capacity entries per atom
 * (0: chosen from the density; longer rows are found again by the write), and the
 * exclusive scan of the counts into row_offsets [N+1] (row_offsets[N] = E, also to
 * *d_num_edges, a device int64, when not NULL).  Write (same workspace, after count):
 * edge_index [2, num_edges] int64 (row 0 = i, row 1 = j, sorted by (i, j)) and
 * edge_vectors [num_edges, 3] = minimum-image pos[j] - pos[i], the arrays of
 * batteries_neighbor_list_write_i64 bit for bit.  neighbor_list_cuda takes this path
 * for such systems.  Replaces the reference's passes, src/neighbor_list/neighbor_list.cu:
 * 242-430, for them. */
size_t batteries_neighbor_list_cells_workspace_bytes(int64_t N, const float* box, float cutoff,
                                                     int row_capacity);
int batteries_neighbor_list_cells_count(const float* positions, const float* box, int64_t N,
                                        float cutoff, int self_loops, int row_capacity,
                                        void* workspace, size_t workspace_bytes,
                                        int64_t* row_offsets, int64_t* d_num_edges,
                                        hipStream_t stream);
int batteries_neighbor_list_cells_write_i64(const float* positions, const float* box, int64_t N,
                                            float cutoff, int self_loops, int row_capacity,
                                            void* workspace, size_t workspace_bytes,
                                            const int64_t* row_offsets, int64_t num_edges,
                                            int64_t* edge_index, float* edge_vectors,
                                            hipStream_t stream);

/* Result of neighbor_list_cuda; same layout as include/neighbor_list.cuh:25-33. */
typedef struct NeighborListResult {
    int* edge_index;      /* [2, num_edges] int32: row 0 = src i, row 1 = dst j */
    float* edge_vectors;  /* [num_edges, 3] */
    int64_t num_edges;
    int* d_edge_index;    /* owned by the library, released by neighbor_list_free */
    float* d_edge_vectors;
} NeighborListResult;

/* Reference-compatible entry points (same names and arguments):
 * src/neighbor_list/neighbor_list.cu:458-468, :470-472, :474-476.
 * cell is a device [3,3] matrix; the call synchronises once to size the output
 * and allocates it (freed by neighbor_list_free). */
int neighbor_list_cuda(const float* positions, const float* cell, int64_t N, float cutoff,
                       bool self_loops, NeighborListResult* result, hipStream_t stream);
void neighbor_list_free(NeighborListResult* result);
size_t neighbor_list_estimate_memory(int64_t N, float density, float cutoff);

/* ---------------------------------------------------------------------------
 * MACE-style interaction layer with per-edge radial weights (no single
 * reference counterpart: the reference composes SH -> TP -> scatter with one
 * shared W[34,C,C] in benchmarks/benchmark_e2e_mace.py:281-355 and takes forces
 * by backward through the edge vectors, :412-420; the per-edge radial weights
 * are the baseline's configs[4]).
 *   v_e = min_image(pos[dst] - pos[src]); B_k(r) = sqrt(2/rc) sin(k pi r/rc)/r f(r/rc),
 *   f(d) = 1 - 28 d^6 + 48 d^7 - 21 d^8; h = silu(B W1 + b1) with W1 [8,64], b1 [64];
 *   R[e,c,p] = (h W2)[p*C + c] with W2 [64, 34 C];
 *   out[d,c,o] = sum_{e->d} sum_p R[e,c,p] sum_{(a,b) in p->o} CG x[src,c,a] Y(v_e/|v_e|)[b].
 * Edges grouped by destination (row_ptr [N+1]) with sources ascending per row,
 * symmetric (every (j->i) has (i->j)), as batmobile.Graph builds them.  box is a
 * host float[3] (orthorhombic cell diagonal).  C <= 256.
 * ------------------------------------------------------------------------- */
/* C[M,N] = A[M,K] B on MFMA (fp32); B is [K,N] row-major, or [N,K] row-major when trans_b. */
int batteries_gemm_f32(const float* A, const float* B, float* C, int64_t M, int N, int K,
                       int trans_b, hipStream_t stream);
/* Workspace of one forward (backward = 0) or backward (backward = 1) pass: per-edge
 * arrays (unit vector, indices, the MLP's 64 hidden values; the backward adds its
 * derivative factors and per-channel-quad gradient shares), about 0.35 KB per edge
 * forward and 1.2 KB backward at C = 128.  The per-edge weights R are never stored. */
size_t batteries_mace_workspace_bytes(int64_t N, int64_t N_edges, int C, int backward);
/* rev[e] = index of the edge with source and destination swapped (-1 if absent);
 * *d_missing (device int) counts the absent ones. */
int batteries_mace_reverse_edges(const int64_t* row_ptr, const int64_t* src, int64_t* rev,
                                 int* d_missing, int64_t N, int64_t N_edges, hipStream_t stream);
/* out [N, C, 16] (node_features and out 16-byte aligned).  order (nullable, [N]): the
 * order in which destinations are processed, a permutation of 0..N-1 (a spatial order
 * keeps the source rows that neighbouring destinations share in cache); the results
 * do not depend on it, bit for bit.  An order that is not a permutation gives wrong
 * results (never an access out of bounds). */
int batteries_mace_forward(const float* positions, const float* box, const float* node_features,
                           const float* w1, const float* b1, const float* w2, const int64_t* src,
                           const int64_t* dst, const int64_t* row_ptr, const int64_t* order,
                           float* out, int64_t N, int64_t N_edges, int C, float cutoff,
                           void* workspace, size_t workspace_bytes, hipStream_t stream);
/* grad_pos[N,3] = d <out, grad_out> / d positions (rev from batteries_mace_reverse_edges;
 * node_features and grad_out 16-byte aligned). */
int batteries_mace_backward(const float* positions, const float* box, const float* node_features,
                            const float* w1, const float* b1, const float* w2, const int64_t* src,
                            const int64_t* dst, const int64_t* row_ptr, const int64_t* order,
                            const int64_t* rev, const float* grad_out, float* grad_pos,
                            int64_t N, int64_t N_edges, int C, float cutoff, void* workspace,
                            size_t workspace_bytes, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Self test (no reference counterpart): D[16,16] = A[16,4] B[4,16] through one
 * v_mfma_f32_16x16x4f32 with the lane layout the kernels above assume.
 * ------------------------------------------------------------------------- */
int batteries_selftest_mfma_16x16x4(const float* A, const float* B, float* D, hipStream_t stream);
/* D[16][64][4]: for every ABID k in 0..15, lane l's accumulator (4 values) after one
 * v_mfma_f32_4x4x1_16b_f32 with CBSZ = 4, ABID = k, A[l] and B[l] from lane l and a zero
 * accumulator.  The weighted scatter assumes D[k][4b + j][r] = A[4k + r] * B[4b + j]. */
int batteries_selftest_mfma_4x4x1_bcast(const float* A, const float* B, float* D,
                                        hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* BATMOBILE_HIP_H_ */
