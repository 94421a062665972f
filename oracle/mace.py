"""MACE-style interaction layer with per-edge radial weights.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

No reference API has per-edge weights: the reference's interaction block
(benchmarks/benchmark_e2e_mace.py:281-355) applies one shared W[34, C, C] per
edge, then scatter_add and a linear layer.  The configuration named in the
baseline (8-function Bessel basis -> MLP [8 -> 64 -> 34 C] -> channel-wise
weighted CG product -> scatter-add, forward and backward with respect to
positions) is defined here, in float64 torch, and the HIP layer is checked
against this composition:

  v_e      = minimum image of pos[dst_e] - pos[src_e]      (benchmark_e2e_mace.py:412-420)
  r_e      = |v_e|, u_e = v_e / r_e
  B_k(r)   = sqrt(2 / rc) sin(k pi r / rc) / r * f(r / rc), k = 1..8
  f(d)     = 1 - 28 d^6 + 48 d^7 - 21 d^8 for d < 1, else 0
             (Bessel radial basis with the p = 6 polynomial envelope of
             Gasteiger, Gross, Guennemann, "Directional message passing for
             molecular graphs", ICLR 2020)
  h_e      = silu(B(r_e) W1 + b1)                           [E, 64]
  R[e,c,p] = (h_e W2)[p * C + c]                            W2 [64, 34 C]
  Y_e      = SH_3(u_e)                                      (spherical_harmonics.cu:33-97)
  m[e,c,o] = sum_p R[e,c,p] sum_{(a,b) in p -> o} CG x[src_e, c, a] Y_e[b]
  out[d]   = sum_{e: dst_e = d} m[e]

Pinned by: the envelope's values and vanishing derivatives at d = 1, the
orthonormality of the bare Bessel functions on [0, rc] (weight r^2), R = 1
reducing the product to TP_simple (pinned in tp/cg), and finite differences
of the forces.
"""
import math

import numpy as np

from . import cg, sh

N_BASIS = 8
HIDDEN = 64
NUM_PATHS = 34


def envelope(d, xp=np):
    """f(d) = 1 - 28 d^6 + 48 d^7 - 21 d^8 on [0, 1), 0 beyond."""
    d6 = d ** 6
    f = 1.0 - 28.0 * d6 + 48.0 * d6 * d - 21.0 * d6 * d * d
    return xp.where(d < 1.0, f, 0.0 * d)


def bessel_bare(r, rc, n=N_BASIS, xp=np):
    """sqrt(2/rc) sin(k pi r / rc) / r, k = 1..n -> [..., n]."""
    k = xp.arange(1, n + 1, dtype=r.dtype) if xp is np else xp.arange(1, n + 1, dtype=r.dtype)
    rr = r[..., None]
    return math.sqrt(2.0 / rc) * xp.sin(k * math.pi * rr / rc) / rr


def radial_basis(r, rc, n=N_BASIS, xp=np):
    return bessel_bare(r, rc, n, xp) * envelope(r / rc, xp)[..., None]


def min_image(t, box, xp=np):
    return t - xp.round(t / box) * box


def layer(pos, box, x, src, dst, w1, b1, w2, rc):
    """float64 torch composition; differentiable with respect to pos (and x)."""
    import torch
    box_t = torch.as_tensor(np.asarray(box, dtype=np.float64))
    v = min_image(pos[dst] - pos[src], box_t, xp=torch)
    r = v.norm(dim=1).clamp(min=1e-10)
    u = v / r[:, None]
    b = radial_basis(r, rc, xp=torch)
    h = torch.nn.functional.silu(b @ w1 + b1)
    c = x.shape[1]
    R = (h @ w2).view(-1, NUM_PATHS, c).transpose(1, 2)          # [E, C, 34]
    y = sh.spherical_harmonics(u, 3, xp=torch)
    m = channelwise_tp(x[src], y, R)                                # [E, C, 16]
    return torch.zeros(pos.shape[0], c, 16, dtype=torch.float64).index_add_(0, dst, m)


def channelwise_tp(xs, y, R):
    """m[e,c,o] = sum_p R[e,c,p] sum_{(a,b) in p -> o} CG xs[e,c,a] y[e,b] (torch float64)."""
    import torch
    cp, _ = cg.dense_paths()
    cp = torch.as_tensor(cp)
    t = torch.einsum("abq,eb,eca->ecq", cp, y, xs)                 # [E, C, 156]
    rq = R[:, :, torch.as_tensor(cg.slot_to_path())]               # [E, C, 156]
    s = torch.zeros(cp.shape[2], 16, dtype=torch.float64)
    s[torch.arange(cp.shape[2]), torch.as_tensor(cg.slot_to_output())] = 1.0
    return (t * rq) @ s


def layer_and_position_grad(pos, box, x, src, dst, w1, b1, w2, rc, grad_out):
    """(out, d<out, grad_out>/d pos) in float64."""
    import torch
    p = torch.as_tensor(np.asarray(pos, dtype=np.float64)).clone().requires_grad_(True)
    args = [torch.as_tensor(np.asarray(a, dtype=np.float64)) for a in (x, w1, b1, w2)]
    s_t = torch.as_tensor(np.asarray(src, dtype=np.int64))
    d_t = torch.as_tensor(np.asarray(dst, dtype=np.int64))
    out = layer(p, box, args[0], s_t, d_t, args[1], args[2], args[3], rc)
    (g,) = torch.autograd.grad(out, p, torch.as_tensor(np.asarray(grad_out, dtype=np.float64)))
    return out.detach().numpy(), g.numpy()
