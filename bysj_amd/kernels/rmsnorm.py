"""Last-axis RMSNorm on gfx950 with input and scale gradients.

Public surface of python/kernels/rmsnorm.py in the reference: ``rmsnorm`` and
``rmsnorm_available``, with the same validation.  Standalone primitive; it
has no DeepMD dispatch seam.
"""
from __future__ import annotations

import math

import torch

from .native import apply_function, _extension, require_dcu


def _validate(x, scale, eps) -> float:
    if not isinstance(x, torch.Tensor):
        raise TypeError("RMSNorm input must be a tensor")
    if x.dtype != torch.float32:
        raise TypeError("RMSNorm requires float32 input")
    if x.ndim < 1:
        raise ValueError("RMSNorm input must have at least one dimension")
    if x.shape[-1] <= 0:
        raise ValueError("RMSNorm feature dimension must be positive")
    if not x.is_contiguous():
        raise ValueError("RMSNorm input must be contiguous")
    if scale is not None:
        if not isinstance(scale, torch.Tensor):
            raise TypeError("RMSNorm scale must be a tensor or None")
        if scale.dtype != torch.float32:
            raise TypeError("RMSNorm scale must be float32")
        if tuple(scale.shape) != (x.shape[-1],):
            raise ValueError("RMSNorm scale must have shape (feature_dim,)")
        if scale.device != x.device:
            raise ValueError("RMSNorm input and scale must share a device")
        if not scale.is_contiguous():
            raise ValueError("RMSNorm scale must be contiguous")
    try:
        eps = float(eps)
    except (TypeError, ValueError) as error:
        raise ValueError("RMSNorm eps must be a finite positive number") from error
    if not math.isfinite(eps) or eps <= 0.0:
        raise ValueError("RMSNorm eps must be a finite positive number")
    return eps


class _RMSNormFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, scale, eps):
        native = _extension("rmsnorm_forward")
        out, inverse_rms = native.rmsnorm_forward(x, scale, eps)
        ctx.save_for_backward(x, scale, inverse_rms)
        ctx.has_scale = scale.numel() != 0
        return out

    @staticmethod
    def backward(ctx, grad_output):
        x, scale, inverse_rms = ctx.saved_tensors
        want_scale = ctx.has_scale and ctx.needs_input_grad[1]
        native = _extension("rmsnorm_backward")
        grad_x, grad_scale = native.rmsnorm_backward(
            grad_output.contiguous(), x, scale, inverse_rms, want_scale
        )
        return (grad_x if ctx.needs_input_grad[0] else None, grad_scale if want_scale else None, None)


def rmsnorm(x: torch.Tensor, scale: torch.Tensor | None = None, eps: float = 1.0e-6) -> torch.Tensor:
    """``x * rsqrt(mean(x**2, -1) + eps) * scale`` over the last axis (no bias).

    Contiguous float32 input with any leading dimensions, optional float32
    ``scale`` of shape ``(x.shape[-1],)``, finite positive ``eps``.
    """
    eps = _validate(x, scale, eps)
    scale_tensor = scale if scale is not None else x.new_empty((0,))
    require_dcu(x, scale_tensor)
    return apply_function(_RMSNormFunction, x, scale_tensor, eps)


def rmsnorm_available() -> bool:
    """Whether both RMSNorm entry points can run on a gfx950 device in this process."""
    try:
        require_dcu()
        native = _extension("rmsnorm_forward")
        return hasattr(native, "rmsnorm_backward")
    except (ImportError, OSError, RuntimeError):
        return False


__all__ = ["rmsnorm", "rmsnorm_available"]
