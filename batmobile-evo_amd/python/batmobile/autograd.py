"""Autograd wrappers over the HIP kernels.

Mirrors reference python/batmobile/autograd.py: the same Function classes,
forward/backward signatures and wrapper functions.  Every forward and backward
runs a HIP kernel; there is no PyTorch fallback path.

Differences from the reference, both mathematically neutral:
  * SphericalHarmonicsFunction with normalize=True fuses the normalisation
    (autograd.py:46-58) and its chain rule (autograd.py:83-92) into the SH
    kernels instead of running them as separate PyTorch ops.
  * backward for L_max 4..6 runs on the GPU (the reference falls back to
    PyTorch autograd there, autograd.py:247-257).
"""
from typing import Optional, Tuple

import torch
from torch import Tensor

import _batmobile


class SphericalHarmonicsFunction(torch.autograd.Function):
    """Y_lm of (optionally normalised) edge vectors; reference autograd.py:18-94."""

    @staticmethod
    def forward(ctx, edge_vectors: Tensor, lmax: int, normalize: bool = True) -> Tensor:
        ctx.lmax = lmax
        ctx.normalize = normalize
        edge_vectors = edge_vectors.contiguous()
        ctx.save_for_backward(edge_vectors)
        if normalize:
            return _batmobile.spherical_harmonics_normalized(edge_vectors, lmax)
        return _batmobile.spherical_harmonics(edge_vectors, lmax)

    @staticmethod
    def backward(ctx, grad_output: Tensor) -> Tuple[Optional[Tensor], None, None]:
        (edge_vectors,) = ctx.saved_tensors
        grad_output = grad_output.contiguous()
        if ctx.normalize:
            grad = _batmobile.spherical_harmonics_normalized_backward(edge_vectors, grad_output)
        else:
            grad = _batmobile.spherical_harmonics_backward(edge_vectors, grad_output)
        return grad, None, None


def spherical_harmonics(edge_vectors: Tensor, lmax: int, normalize: bool = True) -> Tensor:
    """Spherical harmonics with autograd support (reference autograd.py:404-416)."""
    return SphericalHarmonicsFunction.apply(edge_vectors, lmax, normalize)


class TensorProductSimpleFunction(torch.autograd.Function):
    """Simple CG product [N,16] x [N,16]; reference autograd.py:501-544."""

    @staticmethod
    def forward(ctx, input1: Tensor, input2: Tensor) -> Tensor:
        ctx.save_for_backward(input1, input2)
        return _batmobile.tensor_product_simple(input1, input2)

    @staticmethod
    def backward(ctx, grad_output: Tensor) -> Tuple[Tensor, Tensor]:
        input1, input2 = ctx.saved_tensors
        grad_output = grad_output.contiguous()
        return _batmobile.tensor_product_simple_backward(input1, input2, grad_output)


class TensorProductFunction(torch.autograd.Function):
    """Channel-weighted CG product; reference autograd.py:547-599."""

    @staticmethod
    def forward(ctx, input1: Tensor, input2: Tensor, weights: Tensor, c_in: int,
                c_out: int) -> Tensor:
        ctx.save_for_backward(input1, input2, weights)
        ctx.c_in = c_in
        ctx.c_out = c_out
        return _batmobile.tensor_product(input1, input2, weights)

    @staticmethod
    def backward(ctx, grad_output: Tensor):
        input1, input2, weights = ctx.saved_tensors
        grad_output = grad_output.contiguous()
        g1, g2, gw = _batmobile.tensor_product_backward(
            input1, input2, weights, grad_output,
            ctx.needs_input_grad[0], ctx.needs_input_grad[1], ctx.needs_input_grad[2])
        return g1, g2, gw, None, None


def tensor_product_simple(input1: Tensor, input2: Tensor) -> Tensor:
    """reference autograd.py:602-613"""
    return TensorProductSimpleFunction.apply(input1, input2)


def tensor_product(input1: Tensor, input2: Tensor, weights: Tensor, c_in: int,
                   c_out: int) -> Tensor:
    """reference autograd.py:616-631"""
    return TensorProductFunction.apply(input1, input2, weights, c_in, c_out)


__all__ = [
    "spherical_harmonics", "SphericalHarmonicsFunction",
    "tensor_product_simple", "TensorProductSimpleFunction",
    "tensor_product", "TensorProductFunction",
]
