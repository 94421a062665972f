"""The reference's CPU/PyTorch composition in float32, for bench.py's cpu_baseline.

TEST INFRASTRUCTURE (timed as a reported baseline, never shipped).  Restates
the composition the reference benchmarks run on the GPU:
  SH polynomials                python/batmobile/autograd.py:284-341 (same
                                polynomials as oracle/sh.py, float32 torch)
  per-edge CG tensor product    tests/test_tensor_product.py:274-282 (einsum
                                with the CG table fixture)
  gather + scatter-add          benchmarks/benchmark_fused_sh_tp.py:96-98
                                (X[src], index_add_)
  weighted variant              the interaction block SH -> tensor_product(X[src], Y, W)
                                -> index_add_ (benchmarks/benchmark_e2e_mace.py:308-349):
                                per path p, t_p = CG_p(x, y) then W[p] mixing, per edge
"""
import torch

from . import cg, sh

_C = None


def _cg32():
    global _C
    if _C is None:
        _C = torch.as_tensor(cg.dense(), dtype=torch.float32)
    return _C


def sh_tp_scatter(vec, x, src, dst, n, normalize=True):
    """out[d] = sum_{e: dst_e = d} TP_simple(X[src_e], Y(v_e)), all float32 on CPU."""
    if normalize:
        vec = vec / vec.norm(dim=1, keepdim=True).clamp(min=1e-10)
    y = sh.spherical_harmonics(vec, 3, xp=torch)
    msg = torch.einsum("abo,eca,eb->eco", _cg32(), x[src], y)
    out = torch.zeros((n,) + tuple(x.shape[1:]), dtype=x.dtype)
    out.index_add_(0, dst, msg)
    return out


_PATHS = None


def _path_blocks():
    """Per path: (a-range, b-range, o-range, CG block [na, nb, no]) in float32, from the
    per-path table (slot order of tensor_product_fused.cuh:1509-2276)."""
    global _PATHS
    if _PATHS is None:
        c, slots = cg.dense_paths()  # [a, b, slot]
        out = []
        for p, (l1, l2, lo) in enumerate(cg.path_info()):
            a = slice(int(l1 * l1), int((l1 + 1) ** 2))
            b = slice(int(l2 * l2), int((l2 + 1) ** 2))
            o = slice(int(lo * lo), int((lo + 1) ** 2))
            blk = torch.as_tensor(c[a, b, int(slots[p]):int(slots[p + 1])], dtype=torch.float32)
            out.append((a, b, o, blk.contiguous()))
        _PATHS = out
    return _PATHS


def weighted_sh_tp_scatter(vec, x, w, src, dst, n, normalize=True, chunk=8192):
    """out[d] = sum_{e: dst_e = d} tensor_product(X[src_e], Y(v_e), W), float32 on CPU:
    per path p, t_p[e, ci, m] = sum CG_p x[e, ci, a] y[e, b] and msg[e, :, o] += t_p W[p]."""
    if normalize:
        vec = vec / vec.norm(dim=1, keepdim=True).clamp(min=1e-10)
    y = sh.spherical_harmonics(vec, 3, xp=torch)
    cout = w.shape[2]
    out = torch.zeros((n, cout, 16), dtype=x.dtype)
    blocks = _path_blocks()
    for s0 in range(0, vec.shape[0], chunk):
        xs = x[src[s0:s0 + chunk]]
        ys = y[s0:s0 + chunk]
        msg = torch.zeros((xs.shape[0], cout, 16), dtype=x.dtype)
        for p, (a, b, o, blk) in enumerate(blocks):
            t = torch.einsum("eca,eb,abm->ecm", xs[:, :, a], ys[:, b], blk)
            msg[:, :, o] += torch.einsum("ecm,cd->edm", t, w[p])
        out.index_add_(0, dst[s0:s0 + chunk], msg)
    return out
