"""DPA4 geometric-initial-embedding zonal scatter on gfx950.

Public surface of python/kernels/gie.py in the reference: ``zonal_scatter``,
its alias ``gie_zonal_scatter`` and ``gie_available``, with the same
validation.  The forward groups the (possibly unsorted) ``dst`` into a
destination CSR on the device and keeps it for the backward, so neither pass
uses atomics; the grouping is cached per ``dst`` tensor, so later calls on
the same graph skip it.  Out-of-range ``dst`` or ``radial_slot`` values raise
``ValueError`` instead of being read out of bounds.

``gie_zonal_scatter_rmsnorm`` (an extension, not in ``__all__``) fuses the
scatter with the RMSNorm that follows it over each node's flattened row.
"""
from __future__ import annotations

import weakref

import torch

from .native import apply_function, _extension, require_dcu, version_stamp


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


def _capturing(tensor: torch.Tensor) -> bool:
    return tensor.is_cuda and torch.cuda.is_current_stream_capturing()


class _GroupingCache:
    """Destination CSRs of live ``dst`` tensors, so that a graph is grouped once.

    Grouping costs a pass over ``dst`` (and a sort when it is unsorted) plus a
    host synchronisation that reports out-of-range indices.  An entry belongs
    to the ``dst`` tensor object and, within it, to the ``radial_slot`` tensor
    object (whose values decide the slot checks and the backward kernel); it
    is dropped when ``dst`` is freed and rebuilt when either tensor's storage
    or version counter (an in-place write) changes, or the node or slot count
    does.  A few ``radial_slot`` objects are kept per ``dst``.  Grouping
    synchronises, so under HIP graph capture only a cached grouping can be
    used: run the operator once on the same tensors before capturing it.
    Inference tensors keep no version counter, so a grouping of one is built
    on every call and not cached.
    """

    SLOTS_PER_DST = 4

    def __init__(self):
        self._entries: dict[int, tuple] = {}

    def get(self, native, dst, radial_slot, n_nodes: int, n_radial: int):
        key = id(dst)
        dst_stamp, slot_stamp = version_stamp(dst), version_stamp(radial_slot)
        if dst_stamp is None or slot_stamp is None:
            if _capturing(dst):
                raise RuntimeError("GIE: grouping synchronises, and the grouping of an inference tensor is not "
                                   "cached; make dst and radial_slot outside torch.inference_mode to capture")
            return native.gie_group(dst, radial_slot, n_nodes, n_radial)
        stamp = dst_stamp + (n_nodes,)
        entry = self._entries.get(key)
        if entry is not None and (entry[0]() is not dst or entry[1] != stamp):
            entry = None
        groupings = entry[2] if entry is not None else {}
        slot_key = (id(radial_slot), n_radial)
        found = groupings.get(slot_key)
        if found is not None and found[0]() is radial_slot and found[1] == slot_stamp:
            return found[2]
        if _capturing(dst):
            raise RuntimeError("GIE: this dst has no cached grouping, and grouping synchronises; "
                               "run the operator once on the same tensors before HIP graph capture")
        grouping = native.gie_group(dst, radial_slot, n_nodes, n_radial)
        if entry is None:
            reference = weakref.ref(dst, lambda _, key=key: self._entries.pop(key, None))
            entry = (reference, stamp, groupings)
            self._entries[key] = entry
        groupings.pop(slot_key, None)
        groupings[slot_key] = (weakref.ref(radial_slot), slot_stamp, grouping)
        while len(groupings) > self.SLOTS_PER_DST:
            groupings.pop(next(iter(groupings)))
        return grouping

    def clear(self) -> None:
        self._entries.clear()

    def __len__(self) -> int:
        return len(self._entries)


_GROUPINGS = _GroupingCache()


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
        offsets, order, info = _GROUPINGS.get(native, dst, radial_slot, n_nodes, n_radial)
        out = native.gie_zonal_scatter_forward_csr(zonal, radial, offsets, order, radial_slot, inv_sqrt_deg, info)
        ctx.slot_info = info
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
                ctx.slot_info, need=need,
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
    return apply_function(_GIEZonalScatterFunction, zonal, radial, dst, radial_slot, inv_sqrt_deg)


def gie_zonal_scatter(zonal, radial, dst, radial_slot, inv_sqrt_deg):
    """Alias of :func:`zonal_scatter` named after the DPA4 GIE stage."""
    return zonal_scatter(zonal, radial, dst, radial_slot, inv_sqrt_deg)


class _GIERMSNormFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, zonal, radial, dst, radial_slot, inv_sqrt_deg, scale, eps):
        native = _extension("gie_zonal_scatter_forward")
        n_nodes, n_radial = int(inv_sqrt_deg.shape[0]), int(radial.shape[1])
        offsets, order, info = _GROUPINGS.get(native, dst, radial_slot, n_nodes, n_radial)
        keep_x = any(ctx.needs_input_grad)
        y, x, inverse_rms = native.gie_rmsnorm_forward_csr(zonal, radial, offsets, order, radial_slot,
                                                          inv_sqrt_deg, scale, eps, keep_x)
        ctx.slot_info = info
        ctx.has_order = order is not None
        ctx.has_scale = scale.numel() != 0
        saved = [zonal, radial, radial_slot, inv_sqrt_deg, scale, inverse_rms, offsets]
        if keep_x:
            saved.append(x)
        if order is not None:
            saved.append(order)
        ctx.save_for_backward(*saved)
        return y

    @staticmethod
    def backward(ctx, grad_y):
        saved = ctx.saved_tensors
        zonal, radial, radial_slot, inv_sqrt_deg, scale, inverse_rms, offsets, x = saved[:8]
        order = saved[8] if ctx.has_order else None
        native = _extension("rmsnorm_backward")
        n_nodes, width = x.shape[0], x.shape[1] * x.shape[2]
        want_scale = ctx.has_scale and ctx.needs_input_grad[5]
        grad_x, grad_scale = native.rmsnorm_backward(grad_y.contiguous().reshape(n_nodes, width),
                                                     x.reshape(n_nodes, width), scale, inverse_rms, want_scale)
        need = (ctx.needs_input_grad[0], ctx.needs_input_grad[1], ctx.needs_input_grad[4])
        if any(need):
            grads = native.gie_zonal_scatter_backward_csr(
                grad_x.reshape(x.shape), zonal, radial, offsets, order, radial_slot, inv_sqrt_deg,
                ctx.slot_info, need=need,
            )
        else:
            grads = (None, None, None)
        return (
            grads[0] if need[0] else None,
            grads[1] if need[1] else None,
            None,
            None,
            grads[2] if need[2] else None,
            grad_scale if want_scale else None,
            None,
        )


def gie_zonal_scatter_rmsnorm(zonal, radial, dst, radial_slot, inv_sqrt_deg, scale=None, eps=1e-6):
    """``rmsnorm(zonal_scatter(...).reshape(n_nodes, -1), scale, eps)`` reshaped back, in one pass.

    An extension of the reference (which runs ``zonal_scatter`` and then
    ``rmsnorm``): the node rows of ``(n_rows + 1) * channels`` floats are
    normalised where the GIE kernel forms them, so the pre-norm rows are
    written only when a gradient is needed (the RMSNorm backward reads them)
    and never read back in the forward.  Same validation as the two
    operators; ``scale`` has shape ``((n_rows + 1) * channels,)``.  The
    result equals the two operators run back to back bit for bit.  Shapes
    the fused kernel does not take (channels not a multiple of 4, rows over
    2048 + channels floats, no edges) run the two operators.
    """
    from .rmsnorm import _validate as _validate_rmsnorm
    from .rmsnorm import rmsnorm

    _validate(zonal, radial, dst, radial_slot, inv_sqrt_deg)
    n_nodes = int(inv_sqrt_deg.shape[0])
    n_edges, n_rows = int(zonal.shape[0]), int(zonal.shape[1])
    channels = int(radial.shape[2])
    width = (n_rows + 1) * channels
    probe = torch.empty((1, width), dtype=torch.float32, device=zonal.device) if width > 0 else None
    if probe is None:
        raise ValueError("GIE RMSNorm rows must contain at least one channel")
    eps = _validate_rmsnorm(probe, scale, eps)
    require_dcu(zonal, radial, dst, radial_slot, inv_sqrt_deg, scale)
    native = _extension("gie_zonal_scatter_forward")
    fused = (n_nodes > 0 and n_edges * n_rows > 0 and native.gie_rmsnorm_supported(n_rows, channels)
             and radial.data_ptr() % 16 == 0 and (scale is None or scale.data_ptr() % 16 == 0))
    if not fused:
        rows = zonal_scatter(zonal, radial, dst, radial_slot, inv_sqrt_deg)
        return rmsnorm(rows.reshape(n_nodes, width), scale, eps).reshape(n_nodes, n_rows + 1, channels)
    empty = torch.empty((0,), dtype=torch.float32, device=zonal.device)
    return apply_function(_GIERMSNormFunction, zonal, radial, dst, radial_slot, inv_sqrt_deg,
                                     scale if scale is not None else empty, eps)


def gie_available() -> bool:
    """Whether both GIE entry points can run on a gfx950 device in this process."""
    try:
        require_dcu()
        native = _extension("gie_zonal_scatter_forward")
        return hasattr(native, "gie_zonal_scatter_backward")
    except (ImportError, OSError, RuntimeError):
        return False


__all__ = ["gie_available", "gie_zonal_scatter", "zonal_scatter"]
