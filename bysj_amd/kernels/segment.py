"""Destination-segmented operators of the DPA4 edge stream on gfx950.

Public surface of python/kernels/segment.py in the reference (same names,
arguments, validation order, error types and return arity):

``segment_sum``      ``out[n] = node_scale[n] * sum_{dst(e)=n} edge_scale[e] * src[e]``
``segment_softmax``  envelope-gated softmax over each destination's incoming edges
``force_assembly``   per-atom force and virial from per-edge energy gradients
``segment_offsets``  CSR offsets of a destination list
``group_by_source``  stable source grouping ``(order, offsets)``

Grouping contract: ``offsets`` is the exclusive prefix sum of the per-node
edge counts of ``dst``; with ``order=None`` the edges are in natural order
grouped by destination, otherwise ``order`` lists each segment's edges and the
outputs stay in natural edge order.  Build the CSR once per neighbour graph and
reuse it for every block and for the backward.

Unlike the reference (python/kernels/segment.py:221-230), ``segment_sum``
propagates a gradient to ``edge_scale``; DeepMD's envelope seam passes
``edge_scale = edge_env * gate``, which depends on the coordinates.
"""
from __future__ import annotations

import os
import weakref

import torch

from .native import apply_function, _extension, require_dcu, version_stamp

_CHECK_GROUPING = os.environ.get("DPA4_CHECK_GROUPING", "0").strip().lower() in {"1", "true", "yes", "on"}


# ---------------------------------------------------------------------------
# CSR helpers (python/kernels/segment.py:46-71)
# ---------------------------------------------------------------------------

def segment_offsets(dst: torch.Tensor, n_nodes: int) -> torch.Tensor:
    """Exclusive prefix sum of the destination group sizes of an edge list.

    gfx950 tensors: a check pass, a stable radix sort when ``dst`` is not
    already non-decreasing, and a boundary pass that writes each offset once
    (one host sync for the range check, like the reference's
    ``dst.min()/dst.max()``).  CPU tensors never reach the device: the
    reference's helper is device-agnostic torch (bincount and cumsum), and so
    is this one for them.
    """
    if not isinstance(dst, torch.Tensor):
        raise TypeError("segment offsets require a tensor of destinations")
    if dst.dtype != torch.int64:
        raise TypeError("segment offsets require int64 destinations")
    if n_nodes <= 0:
        raise ValueError("segment offsets require a positive node count")
    n_nodes = int(n_nodes)
    if dst.device.type == "cpu":
        if dst.numel() and (int(dst.min()) < 0 or int(dst.max()) >= n_nodes):
            raise ValueError("destination values must be within the node range")
        counts = torch.bincount(dst, minlength=n_nodes)
        return torch.cat([counts.new_zeros(1), torch.cumsum(counts, 0)])
    require_dcu(dst)
    extension = _extension("segment_offsets")
    try:
        return extension.segment_offsets(dst.contiguous(), n_nodes)
    except ValueError as error:
        raise ValueError("destination values must be within the node range") from error


def group_by_source(src: torch.Tensor, n_nodes: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Stable ``(order, offsets)`` grouping an edge list by source atom."""
    if not isinstance(src, torch.Tensor):
        raise TypeError("group_by_source requires a tensor of sources")
    if src.dtype != torch.int64:
        raise TypeError("group_by_source requires int64 sources")
    if n_nodes <= 0:
        raise ValueError("group_by_source requires a positive node count")
    n_nodes = int(n_nodes)
    if src.device.type == "cpu":
        if src.numel() and (int(src.min()) < 0 or int(src.max()) >= n_nodes):
            raise ValueError("source values must be within the node range")
        return torch.argsort(src, stable=True), segment_offsets(src, n_nodes)
    require_dcu(src)
    extension = _extension("group_by_key")
    try:
        return extension.group_by_key(src.contiguous(), n_nodes)
    except ValueError as error:
        raise ValueError("source values must be within the node range") from error


def destination_grouping(dst: torch.Tensor, n_nodes: int) -> tuple[torch.Tensor, torch.Tensor | None]:
    """``(offsets, order)`` grouping an edge list by destination; ``order`` is None when ``dst`` is sorted.

    An extension of the reference API for callers that cache a CSR per
    neighbour graph (the seam layer's ``_CsrView``): the reference's seam
    groups with :func:`group_by_source` and passes its order, which is the
    identity for an already non-decreasing ``dst``.  Returning None there lets
    ``segment_sum``/``segment_softmax`` take their natural-order kernels,
    which read rows without the extra indirection.  Same validation and
    errors as :func:`group_by_source`; on the device, one check pass (and a
    sort only when ``dst`` is unsorted).
    """
    if not isinstance(dst, torch.Tensor):
        raise TypeError("destination grouping requires a tensor of destinations")
    if dst.dtype != torch.int64:
        raise TypeError("destination grouping requires int64 destinations")
    if n_nodes <= 0:
        raise ValueError("destination grouping requires a positive node count")
    n_nodes = int(n_nodes)
    if dst.device.type == "cpu":
        if dst.numel() and (int(dst.min()) < 0 or int(dst.max()) >= n_nodes):
            raise ValueError("destination values must be within the node range")
        ordered = dst.numel() < 2 or bool((dst[1:] >= dst[:-1]).all())
        return segment_offsets(dst, n_nodes), (None if ordered else torch.argsort(dst, stable=True))
    require_dcu(dst)
    extension = _extension("gie_group")
    try:
        offsets, order, _ = extension.gie_group(dst.contiguous(), dst.new_empty(0), n_nodes, 0)
    except ValueError as error:
        raise ValueError("destination values must be within the node range") from error
    return offsets, order


# ---------------------------------------------------------------------------
# validators (python/kernels/segment.py:74-193)
# ---------------------------------------------------------------------------

def _validate_order(order, edges, name):
    if order is None:
        return None
    if not isinstance(order, torch.Tensor) or order.dtype != torch.int64:
        raise TypeError(f"{name} order must be an int64 tensor")
    if tuple(order.shape) != (edges,):
        raise ValueError(f"{name} order must have shape (n_edges,)")
    if not order.is_contiguous():
        raise ValueError(f"{name} order must be contiguous")
    return order


def _present(*tensors):
    return [tensor for tensor in tensors if tensor is not None]


def _contiguous_and_colocated(tensors, name):
    if not all(tensor.is_contiguous() for tensor in tensors):
        raise ValueError(f"{name} inputs must be contiguous")
    if len({tensor.device for tensor in tensors}) != 1:
        raise ValueError(f"all {name} inputs must share a device")


def _validate_segment_sum(src, dst, offsets, edge_scale, node_scale, order=None):
    for label, tensor in (("src", src), ("dst", dst), ("offsets", offsets)):
        if not isinstance(tensor, torch.Tensor):
            raise TypeError(f"segment sum {label} must be a tensor")
    if src.dtype != torch.float32:
        raise TypeError("segment sum src must be float32")
    if dst.dtype != torch.int64 or offsets.dtype != torch.int64:
        raise TypeError("segment sum dst and offsets must be int64")
    if src.ndim != 2:
        raise ValueError("segment sum src must have shape (n_edges, channels)")
    edges = int(src.shape[0])
    if tuple(dst.shape) != (edges,):
        raise ValueError("segment sum dst must have shape (n_edges,)")
    if offsets.ndim != 1 or offsets.numel() < 2:
        raise ValueError("segment sum offsets must be a one-dimensional prefix sum")
    n_nodes = int(offsets.numel()) - 1
    if edge_scale is not None:
        if not isinstance(edge_scale, torch.Tensor) or edge_scale.dtype != torch.float32:
            raise TypeError("segment sum edge_scale must be a float32 tensor")
        if tuple(edge_scale.shape) != (edges,):
            raise ValueError("segment sum edge_scale must have shape (n_edges,)")
    if node_scale is not None:
        if not isinstance(node_scale, torch.Tensor) or node_scale.dtype != torch.float32:
            raise TypeError("segment sum node_scale must be a float32 tensor")
        if node_scale.numel() != n_nodes:
            raise ValueError("segment sum node_scale must have one value per segment")
    _validate_order(order, edges, "segment sum")
    _contiguous_and_colocated(_present(src, dst, offsets, order, edge_scale, node_scale), "segment sum")
    return n_nodes


def _validate_segment_softmax(logit, env, offsets, null_logit, order=None):
    for label, tensor in (("logit", logit), ("env", env), ("offsets", offsets)):
        if not isinstance(tensor, torch.Tensor):
            raise TypeError(f"segment softmax {label} must be a tensor")
    if logit.dtype != torch.float32 or env.dtype != torch.float32:
        raise TypeError("segment softmax logit and env must be float32")
    if offsets.dtype != torch.int64:
        raise TypeError("segment softmax offsets must be int64")
    if logit.ndim != 2:
        raise ValueError("segment softmax logit must have shape (n_edges, channels)")
    edges, channels = int(logit.shape[0]), int(logit.shape[1])
    if tuple(env.shape) != (edges,):
        raise ValueError("segment softmax env must have shape (n_edges,)")
    if offsets.ndim != 1 or offsets.numel() < 2:
        raise ValueError("segment softmax offsets must be a one-dimensional prefix sum")
    n_nodes = int(offsets.numel()) - 1
    if null_logit is not None:
        if not isinstance(null_logit, torch.Tensor) or null_logit.dtype != torch.float32:
            raise TypeError("segment softmax null_logit must be a float32 tensor")
        if tuple(null_logit.shape) != (n_nodes, channels):
            raise ValueError("segment softmax null_logit must have shape (n_nodes, channels)")
    _validate_order(order, edges, "segment softmax")
    _contiguous_and_colocated(_present(logit, env, offsets, order, null_logit), "segment softmax")
    return n_nodes, channels


_FORCE_DTYPES = (torch.float32, torch.float64)


def _validate_force_assembly(grad_edge, edge_vec, dst_offsets, src_offsets, src_order):
    for label, tensor in (
        ("grad_edge", grad_edge),
        ("edge_vec", edge_vec),
        ("dst_offsets", dst_offsets),
        ("src_offsets", src_offsets),
        ("src_order", src_order),
    ):
        if not isinstance(tensor, torch.Tensor):
            raise TypeError(f"force assembly {label} must be a tensor")
    # fp64 is an extension of the reference's fp32-only contract: both value
    # tensors must then be fp64 and the outputs are fp64.
    if grad_edge.dtype not in _FORCE_DTYPES or edge_vec.dtype != grad_edge.dtype:
        raise TypeError("force assembly grad_edge and edge_vec must both be float32 (or both float64)")
    if grad_edge.dim() != 2 or grad_edge.shape[1] != 3:
        raise ValueError("force assembly grad_edge must have shape (n_edges, 3)")
    if edge_vec.shape != grad_edge.shape:
        raise ValueError("force assembly edge_vec must match grad_edge")
    for label, tensor in (("dst_offsets", dst_offsets), ("src_offsets", src_offsets)):
        if tensor.dtype != torch.int64 or tensor.ndim != 1 or tensor.numel() < 2:
            raise ValueError(f"force assembly {label} must be an int64 prefix sum")
    if dst_offsets.numel() != src_offsets.numel():
        raise ValueError("force assembly offsets must describe the same atom count")
    if src_order.dtype != torch.int64 or tuple(src_order.shape) != (grad_edge.shape[0],):
        raise ValueError("force assembly src_order must be int64 with shape (n_edges,)")
    _contiguous_and_colocated([grad_edge, edge_vec, dst_offsets, src_offsets, src_order], "force assembly")
    return int(dst_offsets.numel()) - 1


def _should_check(explicit):
    """Grouping validation is opt-in: it costs a pass over the edge list."""
    return _CHECK_GROUPING if explicit is None else bool(explicit)


def _check_csr(dst, offsets, n_nodes, name):
    if not torch.equal(segment_offsets(dst, n_nodes), offsets):
        raise ValueError(
            f"{name} requires the natural edge order grouped by destination; "
            "offsets must be the exclusive prefix sum of the dst group sizes"
        )


# ---------------------------------------------------------------------------
# degree plans of the softmax kernels
# ---------------------------------------------------------------------------

class _PlanCache:
    """Softmax degree plans, kept per ``offsets`` tensor object.

    A plan lists the segments of a CSR too long for the register path; the
    kernels give each of them a workgroup of its own.  Building one costs a
    device pass and a host synchronisation, so it is done once per graph:
    entries are keyed by the identity of the ``offsets`` tensor and
    invalidated when its storage or version counter changes (an in-place
    write) or the tensor is freed.  During HIP graph capture a missing plan
    is not built; the kernels then run without one (same results).  Nor is
    one built for an inference tensor, whose in-place writes a cached plan
    could not follow: a plan per call would add a synchronisation to every
    call.
    """

    def __init__(self):
        self._entries: dict[int, tuple] = {}

    def get(self, offsets: torch.Tensor, n_edges: int, channels: int):
        stamp = version_stamp(offsets)
        if stamp is None:
            return None
        key = id(offsets)
        entry = self._entries.get(key)
        if entry is not None and (entry[0]() is not offsets or entry[1] != stamp):
            entry = None
        plans = entry[2] if entry is not None else {}
        plan = plans.get((n_edges, channels))
        if plan is not None:
            return plan
        if offsets.is_cuda and torch.cuda.is_current_stream_capturing():
            return None
        plan = _extension("segment_softmax_plan").segment_softmax_plan(offsets, n_edges, channels)
        if entry is None:
            reference = weakref.ref(offsets, lambda _, key=key: self._entries.pop(key, None))
            entry = (reference, stamp, plans)
            self._entries[key] = entry
        plans[(n_edges, channels)] = plan
        return plan

    def clear(self) -> None:
        self._entries.clear()


_PLANS = _PlanCache()


# ---------------------------------------------------------------------------
# autograd functions
# ---------------------------------------------------------------------------

class _SegmentSumFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, src, dst, offsets, edge_scale, node_scale, order):
        native = _extension("segment_sum_forward")
        out = native.segment_sum_forward(src, offsets, edge_scale, node_scale, order)
        ctx.save_for_backward(src, dst, offsets, edge_scale, node_scale, order)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        src, dst, offsets, edge_scale, node_scale, order = ctx.saved_tensors
        want_edge = edge_scale is not None and ctx.needs_input_grad[3]
        want_node = node_scale is not None and ctx.needs_input_grad[4]
        native = _extension("segment_sum_backward")
        grads = native.segment_sum_backward(
            grad_out.contiguous(), src, dst, offsets, edge_scale, node_scale, want_node, order,
            want_edge_scale_grad=want_edge,
        )
        grad_src, grad_node = grads[0], grads[1]
        grad_edge = grads[2] if want_edge else None
        return (
            grad_src if ctx.needs_input_grad[0] else None,
            None,
            None,
            grad_edge if want_edge else None,
            grad_node.reshape(node_scale.shape) if want_node else None,
            None,
        )


def _softmax_plan(offsets, logit):
    return _PLANS.get(offsets, int(logit.shape[0]), int(logit.shape[1]))


class _SegmentSoftmaxFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, logit, env, offsets, order):
        native = _extension("segment_softmax_forward")
        plan = _softmax_plan(offsets, logit)
        alpha, _ = native.segment_softmax_forward(logit, env, offsets, None, order, plan=plan)
        ctx.save_for_backward(alpha, env, offsets, order)
        ctx.plan = plan
        return alpha

    @staticmethod
    def backward(ctx, grad_alpha):
        alpha, env, offsets, order = ctx.saved_tensors
        native = _extension("segment_softmax_backward")
        grad_logit, _, grad_env = native.segment_softmax_backward(
            alpha, grad_alpha.contiguous(), env, offsets, None, None, order, plan=ctx.plan
        )
        return grad_logit, grad_env, None, None


class _SegmentSoftmaxNullFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, logit, env, offsets, null_logit, order):
        native = _extension("segment_softmax_forward")
        plan = _softmax_plan(offsets, logit)
        alpha, null_alpha = native.segment_softmax_forward(logit, env, offsets, null_logit, order, plan=plan)
        ctx.save_for_backward(alpha, null_alpha, env, offsets, order)
        ctx.plan = plan
        return alpha, null_alpha

    @staticmethod
    def backward(ctx, grad_alpha, grad_null_alpha):
        alpha, null_alpha, env, offsets, order = ctx.saved_tensors
        grad_alpha = torch.zeros_like(alpha) if grad_alpha is None else grad_alpha.contiguous()
        grad_null_alpha = (
            torch.zeros_like(null_alpha) if grad_null_alpha is None else grad_null_alpha.contiguous()
        )
        native = _extension("segment_softmax_backward")
        grad_logit, grad_null_logit, grad_env = native.segment_softmax_backward(
            alpha, grad_alpha, env, offsets, null_alpha, grad_null_alpha, order, plan=ctx.plan
        )
        return grad_logit, grad_env, None, grad_null_logit, None


# ---------------------------------------------------------------------------
# public operators
# ---------------------------------------------------------------------------

def segment_sum(src, dst, offsets, edge_scale=None, node_scale=None, *, order=None, check_grouping=None):
    """``out[n] = node_scale[n] * sum_{dst(e)=n} edge_scale[e] * src[e]``.

    ``src`` contiguous float32 ``(n_edges, channels)``, ``dst`` int64
    ``(n_edges,)``, ``offsets`` its CSR prefix sum.  Gradients flow to
    ``src``, ``edge_scale`` and ``node_scale``, never to the indices.
    """
    n_nodes = _validate_segment_sum(src, dst, offsets, edge_scale, node_scale, order)
    if _should_check(check_grouping):
        _check_csr(dst, offsets, n_nodes, "segment sum")
    require_dcu(src, dst, offsets, edge_scale, node_scale, order)
    return apply_function(_SegmentSumFunction, src, dst, offsets, edge_scale, node_scale, order)


def segment_softmax(logit, env, offsets, null_logit=None, *, order=None, check_grouping=None):
    """Envelope-gated softmax over each destination segment, per channel.

    Returns ``alpha`` ``(n_edges, channels)``, or ``(alpha, null_alpha)``
    when ``null_logit`` ``(n_nodes, channels)`` is given.  Edges with a
    non-positive envelope carry no mass.  ``check_grouping`` is accepted for
    signature compatibility; the softmax has no ``dst`` to check against.
    The first call on an ``offsets`` tensor builds its degree plan (one host
    synchronisation); reuse the tensor across calls.
    """
    _validate_segment_softmax(logit, env, offsets, null_logit, order)
    require_dcu(logit, env, offsets, null_logit, order)
    if null_logit is None:
        return apply_function(_SegmentSoftmaxFunction, logit, env, offsets, order)
    return apply_function(_SegmentSoftmaxNullFunction, logit, env, offsets, null_logit, order)


class _ForcePlanCache:
    """Blob plans of force graphs, kept per ``src_order`` tensor object and dtype.

    The planned force assembly (a once-per-graph blob layout, then two
    streaming passes per call) replaces the direct kernel's gathers of
    12- or 24-byte source rows, which cost a cache line each when atom
    numbering has no spatial locality and still bound the kernel by its load
    latency when it has.  The first call on a graph builds the plan, using
    that call's ``edge_vec`` to order the atoms in space (one build: a few
    host synchronisations), and keeps it when the blobs are compact: at
    least ``MIN_EDGES_PER_RECORD`` edges per record on average (the records
    are what the planned path writes and reads back).  float64 rows make
    records twice as large, and there the direct kernel stays faster when
    the numbering already follows space: a float64 graph is planned only
    when fewer than ``LOCAL_SHARE`` of its consecutive source slots name
    edges within ``LOCAL_SPAN`` of each other (one host synchronisation).
    Otherwise, and for graphs under ``MIN_EDGES`` edges, inference tensors
    and calls during HIP graph capture without a cached entry, the direct
    kernel runs.  Entries follow the three graph tensors like the CSR
    caches: keyed by object identity, dropped when one is written in place
    or ``src_order`` is freed.
    """

    MIN_EDGES = 1 << 16
    MIN_EDGES_PER_RECORD = 3.0
    LOCAL_SPAN = 4096
    LOCAL_SHARE = 0.5

    def __init__(self):
        self._entries: dict[tuple, tuple] = {}

    def get(self, native, dst_offsets: torch.Tensor, src_offsets: torch.Tensor, src_order: torch.Tensor,
            edge_vec: torch.Tensor):
        edges = int(src_order.numel())
        if edges < self.MIN_EDGES or not src_order.is_cuda:
            return None
        stamps = tuple(version_stamp(t) for t in (src_order, src_offsets, dst_offsets))
        if any(stamp is None for stamp in stamps):
            return None
        key = (id(src_order), edge_vec.dtype)
        entry = self._entries.get(key)
        stamp = stamps + (id(src_offsets), id(dst_offsets))
        if entry is not None and entry[0]() is src_order and entry[1] == stamp:
            return entry[2]
        if torch.cuda.is_current_stream_capturing():
            return None
        plan = None
        local = 0.0
        if edge_vec.dtype == torch.float64:
            local = ((src_order[1:] - src_order[:-1]).abs() < self.LOCAL_SPAN).float().mean().item()
        if local < self.LOCAL_SHARE:
            try:
                plan = native.force_assembly_plan(dst_offsets, src_offsets, src_order, edge_vec,
                                                  value_bytes=edge_vec.element_size())
            except ValueError:  # not a pair of CSRs of the edge list: the direct kernel clamps such offsets
                plan = None
        if plan is not None and edges < self.MIN_EDGES_PER_RECORD * max(plan.n_records, 1):
            plan = None
        reference = weakref.ref(src_order, lambda _, key=key: self._entries.pop(key, None))
        self._entries[key] = (reference, stamp, plan)
        return plan

    def clear(self) -> None:
        self._entries.clear()


_FORCE_PLANS = _ForcePlanCache()


def force_assembly(grad_edge, edge_vec, src, dst, dst_offsets, src_offsets=None, src_order=None):
    """``(force, virial)`` from per-edge energy gradients (inference only).

    ``src_order``/``src_offsets`` group the edges by source; when omitted they
    are derived from ``src`` with :func:`group_by_source` (cache them when this
    runs every step).  float32 in/out as in the reference; float64 inputs give
    float64 outputs.  On a graph of at least 65,536 edges the first call
    builds a blob plan of the graph (ordered in space with that call's
    ``edge_vec``) and later calls run the planned kernels: the same sums in
    another fixed order, reproducible run to run.
    """
    n_nodes = int(dst_offsets.numel()) - 1
    if src_order is None or src_offsets is None:
        order, offsets = group_by_source(src, n_nodes)
        src_order = order if src_order is None else src_order
        src_offsets = offsets if src_offsets is None else src_offsets
    _validate_force_assembly(grad_edge, edge_vec, dst_offsets, src_offsets, src_order)
    require_dcu(grad_edge, edge_vec, dst_offsets, src_offsets, src_order)
    native = _extension("force_assembly")
    plan = _FORCE_PLANS.get(native, dst_offsets, src_offsets, src_order, edge_vec)
    if plan is not None:
        return native.force_assembly(grad_edge, edge_vec, dst_offsets, src_offsets, src_order, plan=plan)
    return native.force_assembly(grad_edge, edge_vec, dst_offsets, src_offsets, src_order)


def segment_available() -> bool:
    """Whether this process can run every segmented entry point on a gfx950 device."""
    required = (
        "segment_sum_forward",
        "segment_sum_backward",
        "segment_softmax_forward",
        "segment_softmax_backward",
        "force_assembly",
    )
    try:
        require_dcu()
        native = _extension("segment_sum_forward")
    except (ImportError, OSError, RuntimeError):
        return False
    return all(hasattr(native, symbol) for symbol in required)


__all__ = [
    "force_assembly",
    "group_by_source",
    "segment_available",
    "segment_offsets",
    "segment_softmax",
    "segment_sum",
]
