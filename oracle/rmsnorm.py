"""CPU oracle of the last-axis RMSNorm -- test infrastructure only.

Restates python/reference/rmsnorm.py:9-52 of lipengfei1409/bysj:
``x * rsqrt(mean(x**2, -1) + eps) * scale`` with no bias.
"""
from __future__ import annotations

import math

import torch


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
        if scale.shape != (x.shape[-1],):
            raise ValueError("RMSNorm scale must have shape (feature_dim,)")
        if not scale.is_contiguous():
            raise ValueError("RMSNorm scale must be contiguous")
    try:
        eps = float(eps)
    except (TypeError, ValueError) as error:
        raise ValueError("RMSNorm eps must be a finite positive number") from error
    if not math.isfinite(eps) or eps <= 0.0:
        raise ValueError("RMSNorm eps must be a finite positive number")
    return eps


def rmsnorm(x, scale=None, eps=1.0e-6):
    eps = _validate(x, scale, eps)
    inverse_rms = torch.rsqrt(x.square().mean(dim=-1, keepdim=True) + eps)
    out = x * inverse_rms
    if scale is not None:
        out = out * scale
    return out


def rmsnorm_backward_reference(grad_output, x, scale=None, eps=1.0e-6):
    """Autograd of :func:`rmsnorm`: ``(grad_x, grad_scale or None)``."""
    with torch.enable_grad():
        xx = x.detach().clone().requires_grad_(True)
        ss = None if scale is None else scale.detach().clone().requires_grad_(True)
        out = rmsnorm(xx, ss, eps)
        inputs = (xx,) if ss is None else (xx, ss)
        grads = torch.autograd.grad(out, inputs, grad_output)
    return grads[0], (grads[1] if ss is not None else None)


__all__ = ["rmsnorm", "rmsnorm_backward_reference"]
