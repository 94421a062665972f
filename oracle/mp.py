"""Message passing: fused SH+TP, scatter-add, CSR, single-kernel CSR passes.

Restates:
  fused_sh_tp_simple   reference src/message_passing/fused_sh_tp.cu:73-123:
                       messages[e,c,:] = TP_simple(X[src_e,c,:], Y(v_e)), Y of the
                       raw vector (no normalisation, :88-94)
  scatter_add          caller-side index_add_, benchmarks/benchmark_fused_sh_tp.py:96-98
  edge_index_to_csr    fused_message_passing.cu:108-165 (row_ptr by target,
                       col_idx = original edge ids).  The reference fills each row
                       in atomic order; the restatement keeps ascending edge id,
                       which is one of the orders the reference can produce.
  fused_message_passing_simple  fused_message_passing.cu:174-255
  fused_message_passing         fused_message_passing.cu:287-374 (dense W[c_in,c_out]
                       applied to the simple product; col_idx read as the source atom
                       and edge_vectors indexed by CSR slot, :332-337)
  weighted_message_passing      composition SH -> tensor_product -> index_add_
                       (benchmarks/benchmark_e2e_mace.py:681-687, examples/
                       mace_inference.py:152-168) with per-path W[34, c_in, c_out]
"""
import numpy as np

from . import cg, sh, tp


def edge_operator(y):
    """M[e, o, a] = sum_b C[a, b, o] * y[e, b]: TP_simple(x, y) = M @ x."""
    return np.einsum("abo,eb->eoa", cg.dense(), y, optimize=True)


def fused_sh_tp_simple(vec, x, src, chunk=4096):
    e = vec.shape[0]
    out = np.empty((e,) + x.shape[1:])
    for s in range(0, e, chunk):
        m = edge_operator(sh.spherical_harmonics(vec[s:s + chunk], 3))
        out[s:s + chunk] = np.einsum("eoa,eca->eco", m, x[src[s:s + chunk]], optimize=True)
    return out


def scatter_add(messages, dst, n):
    out = np.zeros((n,) + messages.shape[1:])
    np.add.at(out, dst, messages)
    return out


def sh_tp_scatter(vec, x, src, dst, n, normalize=False, chunk=4096):
    """out[d] = sum_{e: dst_e = d} TP_simple(X[src_e], Y(v_e)) without storing messages."""
    if normalize:
        vec, _ = sh.normalize(np.asarray(vec, dtype=np.float64))
    out = np.zeros((n,) + x.shape[1:])
    for s in range(0, vec.shape[0], chunk):
        m = edge_operator(sh.spherical_harmonics(vec[s:s + chunk], 3))
        msg = np.einsum("eoa,eca->eco", m, x[src[s:s + chunk]], optimize=True)
        np.add.at(out, dst[s:s + chunk], msg)
    return out


def edge_index_to_csr(edge_index, n_atoms):
    tgt = np.asarray(edge_index[1], dtype=np.int64)
    counts = np.bincount(tgt, minlength=n_atoms).astype(np.int64)
    row_ptr = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    col_idx = np.argsort(tgt, kind="stable").astype(np.int64)
    return row_ptr, col_idx


def fused_message_passing_simple(x, vec, edge_index, row_ptr, col_idx):
    n = x.shape[0]
    eids = np.asarray(col_idx, dtype=np.int64)
    tgt = np.repeat(np.arange(n), np.diff(row_ptr))
    src = np.asarray(edge_index[0], dtype=np.int64)[eids]
    return sh_tp_scatter(np.asarray(vec)[eids], x, src, tgt, n)


def fused_message_passing(x, vec, w, row_ptr, col_idx):
    n = x.shape[0]
    tgt = np.repeat(np.arange(n), np.diff(row_ptr))
    src = np.asarray(col_idx, dtype=np.int64)
    simple = sh_tp_scatter(np.asarray(vec)[: tgt.size], x, src, tgt, n)   # [N, Ci, 16]
    return np.einsum("nio,ic->nco", simple, w, optimize=True)


def weighted_message_passing(vec, x, w, src, dst, n, normalize=True, chunk=2048):
    """SH(unit v) -> tensor_product(X[src], Y, W[34,Ci,Co]) -> index_add_ over dst."""
    if normalize:
        vec, _ = sh.normalize(np.asarray(vec, dtype=np.float64))
    out = np.zeros((n, w.shape[2], 16))
    for s in range(0, vec.shape[0], chunk):
        y = sh.spherical_harmonics(vec[s:s + chunk], 3)
        msg = tp.tensor_product(x[src[s:s + chunk]], y, w)
        np.add.at(out, dst[s:s + chunk], msg)
    return out
