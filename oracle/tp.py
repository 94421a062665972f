"""Tensor products with the 34-path L<=3 CG table, float64.

Restates:
  tensor_product_simple      reference src/tensor_product/tensor_product.cu:29-50
                             (helper include/tensor_product_fused.cuh:16-700):
                             out[n,o] = sum_(a,b,o) c * x[n,a] * y[n,b]
  tensor_product_simple_bwd  tensor_product_backward.cu:912-942
                             (helper tensor_product_fused.cuh:2286-3583)
  tensor_product (weighted)  tensor_product.cu:133-156 (helper
                             tensor_product_fused.cuh:1509-2276), weight index
                             W[p, c_in, c_out] (tensor_product.cu:100)
  tensor_product_backward    the adjoint documented at
                             tensor_product_backward.cu:7-16 (NOT the
                             hand-written grad_W kernel at :136-902, whose CG
                             lines disagree with the forward table on 15 paths)
"""
import numpy as np

from . import cg


def _cy(y):
    """Cy[n, a, q] = sum_b Cp[a, b, q] * y[n, b] (per-path slots)."""
    cp, _ = cg.dense_paths()
    return np.einsum("abq,nb->naq", cp, y, optimize=True)


def tensor_product_simple(x, y):
    c = cg.dense()
    return np.einsum("abo,na,nb->no", c, x, y, optimize=True)


def tensor_product_simple_backward(x, y, g):
    c = cg.dense()
    gx = np.einsum("abo,nb,no->na", c, y, g, optimize=True)
    gy = np.einsum("abo,na,no->nb", c, x, g, optimize=True)
    return gx, gy


def per_path(x, y):
    """T[n, ci, q]: per-path products (156 slots) of x [N,Ci,16] with y [N,16]."""
    return np.matmul(x, _cy(y))


def _slot_weights(w):
    """Wq[q, ci, co] = W[path(q), ci, co]."""
    return w[cg.slot_to_path()]


def _slot_scatter():
    s = np.zeros((cg.slot_to_output().size, 16))
    s[np.arange(s.shape[0]), cg.slot_to_output()] = 1.0
    return s


def tensor_product(x, y, w):
    """out[n, co, o] = sum_p sum_ci W[p,ci,co] sum_(a,b,o) c x[n,ci,a] y[n,b]."""
    t = per_path(x, y)                                   # [N, Ci, 156]
    u = np.einsum("niq,qic->ncq", t, _slot_weights(w), optimize=True)
    return u @ _slot_scatter()                           # [N, Co, 16]


def tensor_product_backward(x, y, w, g):
    """(grad_x [N,Ci,16], grad_y [N,16], grad_W [34,Ci,Co]) -- exact adjoint."""
    wq = _slot_weights(w)                                # [156, Ci, Co]
    gq = g[:, :, cg.slot_to_output()]                    # [N, Co, 156]
    h = np.einsum("qic,ncq->niq", wq, gq, optimize=True)  # [N, Ci, 156]
    cp, _ = cg.dense_paths()
    gx = np.einsum("abq,niq,nb->nia", cp, h, y, optimize=True)
    gy = np.einsum("abq,niq,nia->nb", cp, h, x, optimize=True)
    t = per_path(x, y)
    gwq = np.einsum("niq,ncq->qic", t, gq, optimize=True)  # [156, Ci, Co]
    gw = np.zeros((cg.NUM_PATHS,) + gwq.shape[1:])
    np.add.at(gw, cg.slot_to_path(), gwq)
    return gx, gy, gw
