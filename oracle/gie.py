"""CPU oracle of the GIE zonal scatter -- test infrastructure only.

Restates python/reference/gie.py:7-65 of lipengfei1409/bysj (validation,
then gather of the radial slots -> per-edge messages -> ``index_add_`` into
rows 1..R -> scale by the inverse degree, i.e. normalise after the sum).
"""
from __future__ import annotations

import torch


def _validate(zonal, radial, dst, radial_slot, inv_sqrt_deg):
    for label, tensor in (("zonal", zonal), ("radial", radial), ("dst", dst), ("radial_slot", radial_slot),
                          ("inv_sqrt_deg", inv_sqrt_deg)):
        if not isinstance(tensor, torch.Tensor):
            raise TypeError(f"GIE {label} must be a tensor")
    if zonal.dtype != torch.float32 or radial.dtype != torch.float32 or inv_sqrt_deg.dtype != torch.float32:
        raise TypeError("GIE value tensors must be float32")
    if dst.dtype != torch.int64 or radial_slot.dtype != torch.int64:
        raise TypeError("GIE dst and radial_slot must be int64")
    if zonal.ndim != 2:
        raise ValueError("GIE zonal must have shape (n_edges, n_rows)")
    if radial.ndim != 3 or radial.shape[0] != zonal.shape[0]:
        raise ValueError("GIE radial must have shape (n_edges, n_radial, channels)")
    n_edges, n_rows = zonal.shape
    if dst.shape != (n_edges,):
        raise ValueError("GIE dst must have shape (n_edges,)")
    if radial_slot.shape != (n_rows,):
        raise ValueError("GIE radial_slot must have shape (n_rows,)")
    if inv_sqrt_deg.ndim not in (1, 3) or (inv_sqrt_deg.ndim == 3 and inv_sqrt_deg.shape[1:] != (1, 1)):
        raise ValueError("GIE inv_sqrt_deg must have shape (n_nodes,) or (n_nodes, 1, 1)")
    if n_rows and radial.shape[1] == 0:
        raise ValueError("GIE radial must contain slots when zonal rows are present")
    if n_edges and inv_sqrt_deg.shape[0] == 0:
        raise ValueError("GIE degree normalization must contain destination nodes")


def zonal_scatter_reference(zonal, radial, dst, radial_slot, inv_sqrt_deg):
    """``out[n, r+1, c] = inv[n] * sum_{dst[e]=n} zonal[e, r] * radial[e, slot[r], c]``; row 0 = 0."""
    _validate(zonal, radial, dst, radial_slot, inv_sqrt_deg)
    inverse = inv_sqrt_deg.reshape(-1)
    n_edges, n_rows = zonal.shape
    n_nodes = inverse.shape[0]
    channels = radial.shape[2]
    if n_edges and (bool((dst < 0).any()) or bool((dst >= n_nodes).any())):
        raise ValueError("GIE dst values must be within the node range")
    if n_rows and (bool((radial_slot < 0).any()) or bool((radial_slot >= radial.shape[1]).any())):
        raise ValueError("GIE radial_slot values must be within the radial range")
    output = radial.new_zeros((n_nodes, n_rows + 1, channels))
    if n_edges and n_rows and channels:
        slots = radial_slot.reshape(1, n_rows, 1).expand(n_edges, n_rows, channels)
        messages = zonal.unsqueeze(-1) * radial.gather(1, slots)
        output[:, 1:, :].index_add_(0, dst, messages)
    return output * inverse.reshape(n_nodes, 1, 1)


gie_zonal_scatter_reference = zonal_scatter_reference


def zonal_scatter_backward_reference(grad_output, zonal, radial, dst, radial_slot, inv_sqrt_deg):
    """Autograd of :func:`zonal_scatter_reference`: ``(grad_zonal, grad_radial, grad_inv_sqrt_deg)``."""
    with torch.enable_grad():
        z = zonal.detach().clone().requires_grad_(True)
        r = radial.detach().clone().requires_grad_(True)
        inv = inv_sqrt_deg.detach().clone().requires_grad_(True)
        out = zonal_scatter_reference(z, r, dst, radial_slot, inv)
        grads = torch.autograd.grad(out, (z, r, inv), grad_output, allow_unused=True)
    return tuple(torch.zeros_like(t) if g is None else g for g, t in zip(grads, (zonal, radial, inv_sqrt_deg)))


__all__ = ["gie_zonal_scatter_reference", "zonal_scatter_backward_reference", "zonal_scatter_reference"]
