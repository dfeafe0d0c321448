"""DPA4 geometric-initial-embedding zonal scatter on gfx950.

Public surface of python/kernels/gie.py in the reference: ``zonal_scatter``,
its alias ``gie_zonal_scatter`` and ``gie_available``, with the same
validation.  The forward groups the (possibly unsorted) ``dst`` into a
destination CSR on the device once and keeps it for the backward, so neither
pass uses atomics.  Out-of-range ``dst`` or ``radial_slot`` values raise
``ValueError`` instead of being read out of bounds.
"""
from __future__ import annotations

import torch

from .native import _extension, require_dcu


def _validate(zonal, radial, dst, radial_slot, inv_sqrt_deg):
    named = (
        ("zonal", zonal),
        ("radial", radial),
        ("dst", dst),
        ("radial_slot", radial_slot),
        ("inv_sqrt_deg", inv_sqrt_deg),
    )
    for label, tensor in named:
        if not isinstance(tensor, torch.Tensor):
            raise TypeError(f"GIE {label} must be a tensor")
    if any(t.dtype != torch.float32 for t in (zonal, radial, inv_sqrt_deg)):
        raise TypeError("GIE value tensors must be float32")
    if dst.dtype != torch.int64 or radial_slot.dtype != torch.int64:
        raise TypeError("GIE dst and radial_slot must be int64")
    if zonal.ndim != 2:
        raise ValueError("GIE zonal must have shape (n_edges, n_rows)")
    if radial.ndim != 3 or radial.shape[0] != zonal.shape[0]:
        raise ValueError("GIE radial must have shape (n_edges, n_radial, channels)")
    n_edges, n_rows = zonal.shape
    if tuple(dst.shape) != (n_edges,):
        raise ValueError("GIE dst must have shape (n_edges,)")
    if tuple(radial_slot.shape) != (n_rows,):
        raise ValueError("GIE radial_slot must have shape (n_rows,)")
    if inv_sqrt_deg.ndim not in (1, 3) or (inv_sqrt_deg.ndim == 3 and tuple(inv_sqrt_deg.shape[1:]) != (1, 1)):
        raise ValueError("GIE inv_sqrt_deg must have shape (n_nodes,) or (n_nodes, 1, 1)")
    if n_rows and radial.shape[1] == 0:
        raise ValueError("GIE radial must contain slots when zonal rows are present")
    if n_edges and inv_sqrt_deg.shape[0] == 0:
        raise ValueError("GIE degree normalization must contain destination nodes")
    tensors = [tensor for _, tensor in named]
    if not all(tensor.is_contiguous() for tensor in tensors):
        raise ValueError("GIE inputs must be contiguous")
    if len({tensor.device for tensor in tensors}) != 1:
        raise ValueError("all GIE inputs must share a device")


class _GIEZonalScatterFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, zonal, radial, dst, radial_slot, inv_sqrt_deg):
        native = _extension("gie_zonal_scatter_forward")
        n_edges, n_rows = int(zonal.shape[0]), int(zonal.shape[1])
        n_nodes, n_radial, channels = int(inv_sqrt_deg.shape[0]), int(radial.shape[1]), int(radial.shape[2])
        ctx.empty = n_nodes == 0 or n_edges * n_rows * channels == 0
        if ctx.empty:
            ctx.save_for_backward(zonal, radial, dst, radial_slot, inv_sqrt_deg)
            return torch.zeros((n_nodes, n_rows + 1, channels), dtype=torch.float32, device=zonal.device)
        offsets, order, info = native.gie_group(dst, radial_slot, n_nodes, n_radial)
        out = native.gie_zonal_scatter_forward_csr(zonal, radial, offsets, order, radial_slot, inv_sqrt_deg)
        ctx.slots_distinct = bool(info & 2)
        ctx.has_order = order is not None
        saved = [zonal, radial, radial_slot, inv_sqrt_deg, offsets]
        if order is not None:
            saved.append(order)
        ctx.save_for_backward(*saved)
        return out

    @staticmethod
    def backward(ctx, grad_output):
        need = (ctx.needs_input_grad[0], ctx.needs_input_grad[1], ctx.needs_input_grad[4])
        if ctx.empty:
            zonal, radial, _, _, inv_sqrt_deg = ctx.saved_tensors
            grads = (torch.zeros_like(zonal), torch.zeros_like(radial), torch.zeros_like(inv_sqrt_deg))
        else:
            saved = ctx.saved_tensors
            zonal, radial, radial_slot, inv_sqrt_deg, offsets = saved[:5]
            order = saved[5] if ctx.has_order else None
            native = _extension("gie_zonal_scatter_backward")
            grads = native.gie_zonal_scatter_backward_csr(
                grad_output.contiguous(), zonal, radial, offsets, order, radial_slot, inv_sqrt_deg,
                ctx.slots_distinct, need=need,
            )
        return (
            grads[0] if need[0] else None,
            grads[1] if need[1] else None,
            None,
            None,
            grads[2] if need[2] else None,
        )


def zonal_scatter(zonal, radial, dst, radial_slot, inv_sqrt_deg):
    """DPA4 GIE zonal scatter: ``(n_nodes, n_rows + 1, channels)`` with row 0 reserved (zero).

    ``out[n, r+1, c] = inv_sqrt_deg[n] * sum_{dst[e]=n} zonal[e, r] * radial[e, radial_slot[r], c]``
    (normalised after the sum).  Value tensors contiguous float32, indices
    contiguous int64; ``dst`` need not be sorted.  Gradients flow to zonal,
    radial and inv_sqrt_deg.
    """
    _validate(zonal, radial, dst, radial_slot, inv_sqrt_deg)
    require_dcu(zonal, radial, dst, radial_slot, inv_sqrt_deg)
    return _GIEZonalScatterFunction.apply(zonal, radial, dst, radial_slot, inv_sqrt_deg)


def gie_zonal_scatter(zonal, radial, dst, radial_slot, inv_sqrt_deg):
    """Alias of :func:`zonal_scatter` named after the DPA4 GIE stage."""
    return zonal_scatter(zonal, radial, dst, radial_slot, inv_sqrt_deg)


def gie_available() -> bool:
    """Whether both GIE entry points can run on a gfx950 device in this process."""
    try:
        require_dcu()
        native = _extension("gie_zonal_scatter_forward")
        return hasattr(native, "gie_zonal_scatter_backward")
    except (ImportError, OSError, RuntimeError):
        return False


__all__ = ["gie_available", "gie_zonal_scatter", "zonal_scatter"]
