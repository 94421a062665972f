"""The reference's CPU/PyTorch composition in float32, for bench.py's cpu_baseline.

TEST INFRASTRUCTURE (timed as a reported baseline, never shipped).  Restates
the composition the reference benchmarks run on the GPU:
  SH polynomials                python/batmobile/autograd.py:284-341 (same
                                polynomials as oracle/sh.py, float32 torch)
  per-edge CG tensor product    tests/test_tensor_product.py:274-282 (einsum
                                with the CG table fixture)
  gather + scatter-add          benchmarks/benchmark_fused_sh_tp.py:96-98
                                (X[src], index_add_)
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
